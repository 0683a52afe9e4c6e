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
import atexit

import numpy as np
import torch

from . import _lib as L

_workspaces = {}


def release_workspaces():
    """Drop the cached workspaces (their device memory returns to torch's allocator).  Called
    at interpreter exit so that no tensor is released during module teardown."""
    _workspaces.clear()


atexit.register(release_workspaces)


def _stream():
    return ctypes_stream(torch.cuda.current_stream())


def ctypes_stream(s):
    return s.cuda_stream


def workspace(nbytes, device=None, key="default"):
    """Zero-filled scratch for one kind of entry point on the current stream.  Each call leaves
    its completion counters and fixed-point accumulators zero again, so a buffer serves every
    later call of the same entry point in stream order; different entry points lay out their
    workspace differently and get separate buffers (`key`)."""
    device = torch.device(device or "cuda")
    k = (key, device.type, device.index if device.index is not None else torch.cuda.current_device())
    buf = _workspaces.get(k)
    if buf is None or buf.numel() < nbytes:
        buf = torch.zeros(max(int(nbytes), 1 << 20), dtype=torch.uint8, device=device)
        _workspaces[k] = buf
    return buf


class Q8FTensor:
    """Q8F matrix: int8 values + one f32 scale per 64 consecutive elements of a stored row.

    layout Q35_KN: q [K(in)][N(out)], scale [K][N/64]  (Burn Linear weight, kernels.rs:56-57)
    layout Q35_NK: q [N][K],          scale [N][K/64]  (embedding table, kernels.rs:253-255)
    layout Q35_KN_TILED: the Q35_KN matrix cut into 256-column tiles, tile-major:
        q [ceil(N/256)][K][256], scale [ceil(N/256)][K][4], columns past N zero
    layout Q35_KN_MB: the f16 matrix-core records (q [N/64][K/32][2048] bytes q + 128, scale
        [N/64][K]), made on the device by mb()
    """

    def __init__(self, q, scale, layout=L.Q35_KN, shape=None):
        assert q.dtype == torch.int8 and scale.dtype == torch.float32
        if layout == L.Q35_KN_TILED:
            assert shape is not None and q.dim() == 3 and q.shape[2] == 256 and scale.shape == q.shape[:2] + (4,)
            self.rows, self.cols = shape
            assert q.shape[:2] == ((self.cols + 255) // 256, self.rows), (q.shape, shape)
        elif layout == L.Q35_KN_MB:
            assert shape is not None and q.numel() == shape[0] * shape[1]
            self.rows, self.cols = shape
            assert scale.shape == (self.cols // 64, self.rows)
        elif layout == L.Q35_KN_PANEL:
            assert shape is not None and q.dim() == 3 and q.shape[2] == 16
            self.rows, self.cols = shape
            assert q.shape[:2] == (self.cols // 16, self.rows) and scale.shape == (self.cols // 64, self.rows)
        else:
            assert q.dim() == 2 and scale.shape == (q.shape[0], q.shape[1] // 64), (scale.shape, q.shape)
            self.rows, self.cols = q.shape
        self.q, self.scale, self.layout = q.contiguous(), scale.contiguous(), layout

    @property
    def shape(self):
        return (self.rows, self.cols)

    @property
    def in_dim(self):
        return self.cols if self.layout == L.Q35_NK else self.rows

    @property
    def out_dim(self):
        return self.rows if self.layout == L.Q35_NK else self.cols

    def desc(self):
        return L.Q8F(self.q.data_ptr(), self.scale.data_ptr(), self.rows, self.cols, self.layout)

    def tiled(self):
        """Q35_KN -> Q35_KN_TILED copy, packed on the host through q35_q8f_pack_kn_tiled."""
        assert self.layout == L.Q35_KN
        K, N = self.rows, self.cols
        q = self.q.cpu().numpy()
        s = self.scale.cpu().numpy()
        qt = np.empty(L.lib().q35_q8f_tiled_q_count(K, N), dtype=np.int8)
        st = np.empty(L.lib().q35_q8f_tiled_scale_count(K, N), dtype=np.float32)
        L.check(L.lib().q35_q8f_pack_kn_tiled(q.ctypes.data, s.ctypes.data, K, N, qt.ctypes.data, st.ctypes.data))
        nt = (N + 255) // 256
        return Q8FTensor(torch.from_numpy(qt.reshape(nt, K, 256)).to(self.q.device),
                         torch.from_numpy(st.reshape(nt, K, 4)).to(self.q.device), L.Q35_KN_TILED, (K, N))

    def mb(self, stream=None):
        """Q35_KN / Q35_KN_TILED -> Q35_KN_MB copy, packed on the device (q35_q8f_pack_mb)."""
        assert self.layout in (L.Q35_KN, L.Q35_KN_TILED)
        K, N = self.rows, self.cols
        qm = torch.empty((N // 64, K // 32, 2048), dtype=torch.int8, device=self.q.device)
        sm = torch.empty((N // 64, K), dtype=torch.float32, device=self.q.device)
        st = stream if stream is not None else _stream()
        L.check(L.lib().q35_q8f_pack_mb(self.desc(), qm.data_ptr(), sm.data_ptr(), st))
        return Q8FTensor(qm, sm, L.Q35_KN_MB, (K, N))

    def panel(self):
        """Q35_KN -> Q35_KN_PANEL copy, packed on the host through q35_q8f_pack_kn_panel."""
        assert self.layout == L.Q35_KN
        K, N = self.rows, self.cols
        q = np.ascontiguousarray(self.q.cpu().numpy())
        s = np.ascontiguousarray(self.scale.cpu().numpy())
        qp = np.empty((N // 16, K, 16), dtype=np.int8)
        sp = np.empty((N // 64, K), dtype=np.float32)
        L.check(L.lib().q35_q8f_pack_kn_panel(q.ctypes.data, s.ctypes.data, K, N, qp.ctypes.data, sp.ctypes.data))
        return Q8FTensor(torch.from_numpy(qp).to(self.q.device), torch.from_numpy(sp).to(self.q.device),
                         L.Q35_KN_PANEL, (K, N))


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
    ws = workspace(L.lib().q35_q8_gemv_ws_bytes(x.shape[0], W), x.device, "gemv")
    L.check(L.lib().q35_q8_gemv(x.data_ptr(), x.shape[0], W, y.data_ptr(), ws.data_ptr(), ws.numel(), _stream()))
    return y.reshape(*hidden_states.shape[:-1], N)


def q8_gemv_partial_sum(hidden_states, weights: Q8FTensor):
    K, N = weights.in_dim, weights.out_dim
    x = _rows(hidden_states, K)
    y = torch.empty((x.shape[0], N), dtype=torch.float32, device=x.device)
    W = weights.desc()
    ws = workspace(L.lib().q35_q8_gemv_ws_bytes(x.shape[0], W), x.device, "gemv")
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
    ws = workspace(L.lib().q35_argmax_ws_bytes(v.numel()), v.device, "argmax")
    L.check(L.lib().q35_argmax(v.data_ptr(), v.numel(), out.data_ptr(), ws.data_ptr(), ws.numel(), _stream()))
    return out
