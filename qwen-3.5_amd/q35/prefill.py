"""Prompt (seq_len > 1) surface on torch device tensors: the reference's Linear::forward on Q8F
weights for a prompt (dequantise + f32 matmul), the prompt branches of GatedDeltaNet
(causal conv + chunked gated delta rule) and of Attention (causal attention over the cache).

  q8_gemm                   Linear::forward, text_modules.rs:500-508,578-595,638-647,880-890,
                            1003-1005; the lm_head matmul model.rs:130-138 (NK layout)
  gate_proj_prompt          text_modules.rs:578-595
  gated_delta_rule_prefill  causal_conv1d_fn + burn_chunk_gated_delta_rule, :164-182,189-363
  attention_core_prefill    Attention::forward between the projections, :860-936
"""
import ctypes

import torch

from . import _lib as L
from .kernels import _stream, workspace


def _p(t):
    return t.data_ptr() if t is not None else None


def q8_gemm(x, W, y=None, accumulate=False, split_k=False):
    """y[M][N] (+)= x[M][K] @ dequant(W) on the fp32 matrix cores, or on the f16 matrix cores with
    f32-equivalent products for W in Q35_KN_MB (always with a workspace).  split_k: pass a
    workspace (q35_q8_gemm_ws), so that the launcher may split K for shapes with few output
    tiles."""
    assert x.dtype == torch.float32 and x.dim() == 2 and x.stride(1) == 1
    M = x.shape[0]
    if y is None:
        y = torch.empty((M, W.out_dim), dtype=torch.float32, device=x.device)
    assert y.stride(1) == 1 and y.shape[0] == M
    acc = 1 if accumulate else 0
    if split_k or W.layout == L.Q35_KN_MB:
        nb = L.lib().q35_q8_gemm_ws_bytes(M, W.desc())
        ws = workspace(nb, x.device, key="gemm")
        L.check(L.lib().q35_q8_gemm_ws(x.data_ptr(), M, x.stride(0), W.desc(), y.data_ptr(), y.stride(0), acc,
                                       ws.data_ptr(), ws.numel(), _stream()))
    else:
        L.check(L.lib().q35_q8_gemm(x.data_ptr(), M, x.stride(0), W.desc(), y.data_ptr(), y.stride(0), acc,
                                    _stream()))
    return y


def gate_proj_prompt(x, w_b, w_a, a_log, dt_bias):
    """[T][2 heads] = [beta | g] with the prompt branch's softplus rule (input > 20)."""
    T, H = x.shape
    nh = w_b.shape[1]
    out = torch.empty((T, 2 * nh), dtype=torch.float32, device=x.device)
    L.check(L.lib().q35_gate_proj_prompt(_p(x), T, H, _p(w_b), _p(w_a), _p(a_log), _p(dt_bias), nh, out.data_ptr(),
                                         _stream()))
    return out


def gated_delta_rule_prefill(mixed_qkv, beta_g, conv_state, conv_w, recurrent_state, heads, dk=128, dv=128):
    """Causal conv + chunked gated delta rule over T prompt rows of one sequence.  mixed_qkv
    [T, >= conv_dim] (pre-conv); beta_g [T, 2 heads]; conv_state [conv_dim, 3] and
    recurrent_state [heads, 128, 128] updated in place; returns the core output [T, heads*dv]."""
    T = mixed_qkv.shape[0]
    out = torch.empty((T, heads * dv), dtype=torch.float32, device=mixed_qkv.device)
    nbytes = L.lib().q35_gated_delta_rule_prefill_ws_bytes(T, heads)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=mixed_qkv.device)
    L.check(L.lib().q35_gated_delta_rule_prefill(_p(mixed_qkv), T, mixed_qkv.stride(0), _p(beta_g),
                                                 conv_state.data_ptr(), _p(conv_w), recurrent_state.data_ptr(),
                                                 out.data_ptr(), heads, dk, dv, ws.data_ptr(), nbytes, _stream()))
    return out


def attention_core_prefill(dims, q_gate, k_new, v_new, q_norm, k_norm, k_cache, v_cache, p0, rope_cos, rope_sin):
    """q/k norm, RoPE, KV append at rows p0.., causal GQA attention and sigmoid gate for T prompt
    rows of one sequence.  q_gate [T, heads*512]; k_new/v_new [T, kv_heads*256]; caches
    [kv_heads, tmax, 256]; returns [T, heads*256]."""
    T = q_gate.shape[0]
    tmax = k_cache.shape[-2]
    out = torch.empty((T, dims.attn_heads * dims.head_dim), dtype=torch.float32, device=q_gate.device)
    nbytes = L.lib().q35_attention_prefill_ws_bytes(ctypes.byref(dims), T)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=q_gate.device)
    L.check(L.lib().q35_attention_core_prefill(ctypes.byref(dims), _p(q_gate), q_gate.stride(0), _p(k_new),
                                               _p(v_new), k_new.stride(0), T, int(p0), _p(q_norm), _p(k_norm),
                                               k_cache.data_ptr(), v_cache.data_ptr(), tmax, _p(rope_cos),
                                               _p(rope_sin), out.data_ptr(), ws.data_ptr(), nbytes, _stream()))
    return out
