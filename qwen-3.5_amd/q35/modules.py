"""Layer forwards with the surface of the reference's src/text_modules.rs decode branches.

  GatedDeltaNet.forward   text_modules.rs:484-667   (seq_len == 1 with cached states)
  Attention.forward       text_modules.rs:842-944   (seq_len == 1)
  MLP.forward             text_modules.rs:1000-1011
  Cache                   text_modules.rs:445-461   (preallocated here: KV [B][kv][tmax][256])
Each forward is one call into libq35.so (which launches the fused gfx950 kernels).
"""
import ctypes

import torch

from . import _lib as L
from .kernels import Q8FTensor, workspace, _stream


def _p(t):
    return t.contiguous().data_ptr()


class GatedDeltaNet:
    def __init__(self, dims, in_proj_qkv: Q8FTensor, in_proj_z: Q8FTensor, out_proj: Q8FTensor, in_proj_b, in_proj_a,
                 a_log, dt_bias, conv_w, norm_w):
        self.dims = dims
        self.t = dict(in_proj_qkv=in_proj_qkv, in_proj_z=in_proj_z, out_proj=out_proj, in_proj_b=in_proj_b.contiguous(),
                      in_proj_a=in_proj_a.contiguous(), a_log=a_log.contiguous(), dt_bias=dt_bias.contiguous(),
                      conv_w=conv_w.contiguous(), norm_w=norm_w.contiguous())
        t = self.t
        self.w = L.GdnWeights(t["in_proj_qkv"].desc(), t["in_proj_z"].desc(), t["out_proj"].desc(), _p(t["in_proj_b"]),
                              _p(t["in_proj_a"]), _p(t["a_log"]), _p(t["dt_bias"]), _p(t["conv_w"]), _p(t["norm_w"]))

    def forward(self, hidden_states, conv_state, recurrent_state):
        """hidden_states [B, hidden] (already input-normed); conv_state [B, conv_dim, 3] and
        recurrent_state [B, heads, 128, dv] are updated in place; returns [B, hidden]."""
        d = self.dims
        x = hidden_states.reshape(-1, d.hidden).contiguous()
        B = x.shape[0]
        out = torch.empty_like(x)
        ws = workspace(L.lib().q35_layer_ws_bytes(ctypes.byref(d), B, 1), x.device, ("gated_deltanet", B))
        L.check(L.lib().q35_gated_deltanet_decode(ctypes.byref(d), ctypes.byref(self.w), x.data_ptr(), B,
                                                  conv_state.data_ptr(), recurrent_state.data_ptr(), out.data_ptr(),
                                                  ws.data_ptr(), ws.numel(), _stream()))
        return out


class Attention:
    def __init__(self, dims, q_proj: Q8FTensor, k_proj: Q8FTensor, v_proj: Q8FTensor, o_proj: Q8FTensor, q_norm, k_norm):
        self.dims = dims
        self.t = dict(q_proj=q_proj, k_proj=k_proj, v_proj=v_proj, o_proj=o_proj, q_norm=q_norm.contiguous(),
                      k_norm=k_norm.contiguous())
        t = self.t
        self.w = L.AttnWeights(q_proj.desc(), k_proj.desc(), v_proj.desc(), o_proj.desc(), _p(t["q_norm"]),
                               _p(t["k_norm"]))

    def forward(self, hidden_states, k_cache, v_cache, pos, rope_cos, rope_sin):
        """hidden_states [B, hidden]; k/v_cache [B, kv_heads, tmax, 256]; pos int32 [B] on the
        device (tokens already cached); rope tables [tmax, rot_dim].  Returns [B, hidden]."""
        d = self.dims
        x = hidden_states.reshape(-1, d.hidden).contiguous()
        B = x.shape[0]
        tmax = k_cache.shape[2]
        out = torch.empty_like(x)
        ws = workspace(L.lib().q35_layer_ws_bytes(ctypes.byref(d), B, tmax), x.device, ("attention", B, tmax))
        L.check(L.lib().q35_attention_decode(ctypes.byref(d), ctypes.byref(self.w), x.data_ptr(), B, k_cache.data_ptr(),
                                             v_cache.data_ptr(), tmax, pos.data_ptr(), rope_cos.data_ptr(),
                                             rope_sin.data_ptr(), out.data_ptr(), ws.data_ptr(), ws.numel(), _stream()))
        return out


class MLP:
    def __init__(self, dims, gate_proj: Q8FTensor, up_proj: Q8FTensor, down_proj: Q8FTensor):
        self.dims = dims
        self.t = dict(gate_proj=gate_proj, up_proj=up_proj, down_proj=down_proj)
        self.w = L.MlpWeights(gate_proj.desc(), up_proj.desc(), down_proj.desc())

    def forward(self, x, check=False):
        """check=True synchronises and raises Q35Error (Q35_E_RANGE) if a row held a value that
        the fixed-point sums cannot take (NaN / Inf, or products of magnitude >= 2^31), as
        q35_workspace_status documents."""
        d = self.dims
        x2 = x.reshape(-1, d.hidden).contiguous()
        B = x2.shape[0]
        out = torch.empty_like(x2)
        ws = workspace(L.lib().q35_layer_ws_bytes(ctypes.byref(d), B, 1), x2.device, ("mlp", B))
        L.check(L.lib().q35_mlp_decode(ctypes.byref(d), ctypes.byref(self.w), x2.data_ptr(), B, out.data_ptr(),
                                       ws.data_ptr(), ws.numel(), _stream()))
        if check:
            L.check(L.lib().q35_workspace_status(ws.data_ptr(), _stream()))
        return out


def gated_delta_rule_decode(mixed_qkv, beta_g, conv_state, conv_w, recurrent_state, heads, dk=128, dv=128,
                            fused=True):
    """Conv update + recurrent gated delta rule for one token (text_modules.rs:134-162,
    :365-443).  mixed_qkv [B, conv_dim]; beta_g [B, 2*heads]; states updated in place;
    returns the core output [B, heads*dv] (before the gated norm).  fused: pass a workspace so
    that one kernel also advances the conv state (else a second kernel does)."""
    B = mixed_qkv.shape[0]
    out = torch.empty((B, heads * dv), dtype=torch.float32, device=mixed_qkv.device)
    ws = workspace(1 << 16, mixed_qkv.device, "delta_rule") if fused else None
    L.check(L.lib().q35_gated_delta_rule_decode(_p(mixed_qkv), B, _p(beta_g), conv_state.data_ptr(), _p(conv_w),
                                                recurrent_state.data_ptr(), out.data_ptr(), heads, dk, dv,
                                                ws.data_ptr() if fused else None, ws.numel() if fused else 0,
                                                _stream()))
    return out


def attention_core_decode(dims, q_gate, k_new, v_new, q_norm, k_norm, k_cache, v_cache, pos, rope_cos, rope_sin,
                          check=False):
    """q/k norm, RoPE, KV append, GQA softmax attention and sigmoid gate for one token
    (text_modules.rs:860-936).  q_gate [B, heads*512]; k_new/v_new [B, kv_heads*256].
    check=True synchronises and raises Q35Error if a position lay outside [0, tmax) (that row
    is then skipped on the device, as q35_workspace_status documents)."""
    B = q_gate.shape[0]
    tmax = k_cache.shape[2]
    out = torch.empty((B, dims.attn_heads * dims.head_dim), dtype=torch.float32, device=q_gate.device)
    ws = workspace(L.lib().q35_layer_ws_bytes(ctypes.byref(dims), B, tmax), q_gate.device, ("attention_core", B, tmax))
    L.check(L.lib().q35_attention_core_decode(ctypes.byref(dims), _p(q_gate), _p(k_new), _p(v_new), k_new.shape[1], B,
                                              _p(q_norm), _p(k_norm), k_cache.data_ptr(), v_cache.data_ptr(), tmax,
                                              pos.data_ptr(), _p(rope_cos), _p(rope_sin), out.data_ptr(), ws.data_ptr(),
                                              ws.numel(), _stream()))
    if check:
        L.check(L.lib().q35_workspace_status(ws.data_ptr(), _stream()))
    return out


def rope_tables(dims, tmax):
    """cos/sin [tmax, rot_dim] of TextRotaryEmbedding (text_modules.rs:30-43,73-81)."""
    import numpy as np
    c = np.empty((tmax, dims.rot_dim), np.float32)
    s = np.empty((tmax, dims.rot_dim), np.float32)
    L.check(L.lib().q35_rope_tables(ctypes.byref(dims), tmax, c.ctypes.data, s.ctypes.data))
    return c, s
