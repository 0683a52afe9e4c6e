"""Tensor-level ops with the surface of the reference's src/kernels.rs, on torch device tensors.

PyTorch only provides device memory and the current HIP stream; all arithmetic runs in the
gfx950 kernels of libq35.so.  Reference wrappers mirrored here:
  q8_embedding_lookup  kernels.rs:669-679      q8_gemv              kernels.rs:681-688
  q8_gemv_partial_sum  kernels.rs:690-700      gate_proj            kernels.rs:702-722
  q8_lm_head           kernels.rs:724-731      argmax               kernels.rs:733-739
Differences from the reference, by design: batches of M rows are accepted (the reference
squeezes [1,1,K] and panics otherwise) and q8_gemv_partial_sum sums every input row (the
reference kernel skips rows when K / splits is not a multiple of 8, kernels.rs:119-133,504).
"""
import torch

from . import _lib as L

_workspaces = {}


def _stream():
    return ctypes_stream(torch.cuda.current_stream())


def ctypes_stream(s):
    return s.cuda_stream


def workspace(nbytes, device=None):
    """Zero-filled scratch shared by calls on the current stream (every call leaves its
    completion counters zero again, so one buffer serves all calls in stream order)."""
    device = torch.device(device or "cuda")
    key = (device.type, device.index if device.index is not None else torch.cuda.current_device())
    buf = _workspaces.get(key)
    if buf is None or buf.numel() < nbytes:
        buf = torch.zeros(max(int(nbytes), 1 << 20), dtype=torch.uint8, device=device)
        _workspaces[key] = buf
    return buf


class Q8FTensor:
    """Q8F matrix: int8 values + one f32 scale per 64 consecutive elements of a stored row.

    layout Q35_KN: q [K(in)][N(out)], scale [K][N/64]  (Burn Linear weight, kernels.rs:56-57)
    layout Q35_NK: q [N][K],          scale [N][K/64]  (embedding table, kernels.rs:253-255)
    """

    def __init__(self, q, scale, layout=L.Q35_KN):
        assert q.dtype == torch.int8 and scale.dtype == torch.float32 and q.dim() == 2
        assert scale.shape == (q.shape[0], q.shape[1] // 64), (scale.shape, q.shape)
        self.q, self.scale, self.layout = q.contiguous(), scale.contiguous(), layout

    @property
    def shape(self):
        return tuple(self.q.shape)

    @property
    def in_dim(self):
        return self.q.shape[0] if self.layout == L.Q35_KN else self.q.shape[1]

    @property
    def out_dim(self):
        return self.q.shape[1] if self.layout == L.Q35_KN else self.q.shape[0]

    def desc(self):
        return L.Q8F(self.q.data_ptr(), self.scale.data_ptr(), self.q.shape[0], self.q.shape[1], self.layout)


def _rows(x, k):
    x2 = x.reshape(-1, k)
    assert x2.dtype == torch.float32
    return x2.contiguous()


def q8_gemv(hidden_states, weights: Q8FTensor):
    """y = hidden_states @ dequant(W); hidden_states [..., K] -> [..., N]."""
    K, N = weights.in_dim, weights.out_dim
    x = _rows(hidden_states, K)
    y = torch.empty((x.shape[0], N), dtype=torch.float32, device=x.device)
    W = weights.desc()
    nbytes = L.lib().q35_q8_gemv_ws_bytes(x.shape[0], W)
    ws = workspace(nbytes, x.device)
    L.check(L.lib().q35_q8_gemv(x.data_ptr(), x.shape[0], W, y.data_ptr(), ws.data_ptr(), ws.numel(), _stream()))
    return y.reshape(*hidden_states.shape[:-1], N)


def q8_gemv_partial_sum(hidden_states, weights: Q8FTensor):
    K, N = weights.in_dim, weights.out_dim
    x = _rows(hidden_states, K)
    y = torch.empty((x.shape[0], N), dtype=torch.float32, device=x.device)
    W = weights.desc()
    ws = workspace(L.lib().q35_q8_gemv_ws_bytes(x.shape[0], W), x.device)
    L.check(L.lib().q35_q8_gemv_partial_sum(x.data_ptr(), x.shape[0], W, y.data_ptr(), ws.data_ptr(), ws.numel(),
                                            _stream()))
    return y.reshape(*hidden_states.shape[:-1], N)


def q8_lm_head(hidden_states, embeddings: Q8FTensor):
    """logits = hidden_states @ dequant(E)^T with E the [V][D] table."""
    assert embeddings.layout == L.Q35_NK
    V, D = embeddings.q.shape
    x = _rows(hidden_states, D)
    y = torch.empty((x.shape[0], V), dtype=torch.float32, device=x.device)
    L.check(L.lib().q35_q8_lm_head(x.data_ptr(), x.shape[0], embeddings.desc(), y.data_ptr(), _stream()))
    return y.reshape(*hidden_states.shape[:-1], V)


def q8_embedding_lookup(embeddings: Q8FTensor, input_ids):
    assert embeddings.layout == L.Q35_NK
    ids = input_ids.reshape(-1).to(torch.int32).contiguous()
    out = torch.empty((ids.numel(), embeddings.q.shape[1]), dtype=torch.float32, device=ids.device)
    L.check(L.lib().q35_q8_embedding_lookup(embeddings.desc(), ids.data_ptr(), ids.numel(), out.data_ptr(), _stream()))
    return out


def gate_proj(hidden_states, w_b, w_a, a_log, dt_bias):
    """(beta, g) with beta = sigmoid(x W_b), g = -exp(A_log) * softplus(x W_a + dt_bias)."""
    K, nh = w_b.shape
    x = _rows(hidden_states, K)
    out = torch.empty((x.shape[0], 2 * nh), dtype=torch.float32, device=x.device)
    L.check(L.lib().q35_gate_proj(x.data_ptr(), x.shape[0], K, w_b.contiguous().data_ptr(), w_a.contiguous().data_ptr(),
                                  a_log.contiguous().data_ptr(), dt_bias.contiguous().data_ptr(), nh, out.data_ptr(),
                                  _stream()))
    lead = hidden_states.shape[:-1]
    return out[:, :nh].reshape(*lead, nh), out[:, nh:].reshape(*lead, nh)


def argmax(logits):
    v = logits.reshape(-1).contiguous()
    out = torch.empty(1, dtype=torch.int32, device=v.device)
    ws = workspace(L.lib().q35_argmax_ws_bytes(v.numel()), v.device)
    L.check(L.lib().q35_argmax(v.data_ptr(), v.numel(), out.data_ptr(), ws.data_ptr(), ws.numel(), _stream()))
    return out
