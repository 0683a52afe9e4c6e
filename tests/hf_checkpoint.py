"""Writes a small Hugging Face-style safetensors checkpoint of a Qwen3.5-shaped decoder for the
loader tests: the tensors the reference's loader reads (main.rs:160-222), named as the HF
checkpoint names them (`model.language_model.layers.{i}.linear_attn.in_proj_qkv.weight`,
`...linear_attn.A_log`, ...) and laid out as PyTorch stores them (Linear weights [out][in],
conv1d [channels][1][k]), with the values of the library's seeded synthetic model."""
import numpy as np
import torch
from safetensors.torch import save_file

import q35


def decoder_tensors(d):
    """(builder name, HF suffix, rows, cols, linear): the decoder's tensors in the builder's
    [in][out] shapes; `linear` marks the reference's Linear modules (stored transposed)."""
    H, F, V = d.hidden, d.ffn, d.vocab
    nh, vd, kd = d.lin_heads, d.lin_heads * d.lin_dv, d.lin_heads * d.lin_dk
    conv = 2 * kd + vd
    ah, kvh, hd = d.attn_heads, d.kv_heads, d.head_dim
    out = [("embed_tokens", "embed_tokens.weight", V, H, False), ("norm", "norm.weight", 1, H, False)]
    for l in range(d.n_layers):
        p = f"layers.{l}."
        out += [(p + "input_layernorm", p + "input_layernorm.weight", 1, H, False),
                (p + "post_attention_layernorm", p + "post_attention_layernorm.weight", 1, H, False)]
        if (l + 1) % d.full_interval != 0:
            a = p + "linear_attn."
            out += [(a + "in_proj_qkv", a + "in_proj_qkv.weight", H, conv, True),
                    (a + "in_proj_z", a + "in_proj_z.weight", H, vd, True),
                    (a + "out_proj", a + "out_proj.weight", vd, H, True),
                    (a + "in_proj_b", a + "in_proj_b.weight", H, nh, True),
                    (a + "in_proj_a", a + "in_proj_a.weight", H, nh, True),
                    (a + "a_log", a + "A_log", 1, nh, False),
                    (a + "dt_bias", a + "dt_bias", 1, nh, False),
                    (a + "conv1d", a + "conv1d.weight", conv, d.conv_k, False),
                    (a + "norm", a + "norm.weight", 1, d.lin_dv, False)]
        else:
            a = p + "self_attn."
            out += [(a + "q_proj", a + "q_proj.weight", H, ah * hd * 2, True),
                    (a + "k_proj", a + "k_proj.weight", H, kvh * hd, True),
                    (a + "v_proj", a + "v_proj.weight", H, kvh * hd, True),
                    (a + "o_proj", a + "o_proj.weight", ah * hd, H, True),
                    (a + "q_norm", a + "q_norm.weight", 1, hd, False),
                    (a + "k_norm", a + "k_norm.weight", 1, hd, False)]
        m = p + "mlp."
        out += [(m + "gate_proj", m + "gate_proj.weight", H, F, True),
                (m + "up_proj", m + "up_proj.weight", H, F, True),
                (m + "down_proj", m + "down_proj.weight", F, H, True)]
    return out


def write(path, d, seed, dtype=torch.float32, prefix="model.language_model.", extra=None, drop=()):
    """Saves the checkpoint; returns {builder name: f32 values in the builder's layout, after the
    round trip through `dtype`}."""
    tensors, expect = {}, {}
    for name, hf, rows, cols, linear in decoder_tensors(d):
        v = q35.synth_model_tensor(d, seed, name, rows * cols).reshape(rows, cols)
        if linear:
            t = torch.from_numpy(np.ascontiguousarray(v.T))
        elif name.endswith("conv1d"):
            t = torch.from_numpy(v.reshape(rows, 1, cols))
        elif rows == 1:
            t = torch.from_numpy(v.reshape(cols))
        else:
            t = torch.from_numpy(v)
        t = t.to(dtype).contiguous()
        if name not in drop:
            tensors[prefix + hf] = t
        back = t.to(torch.float32).numpy()
        expect[name] = np.ascontiguousarray(back.T if linear else back).reshape(-1)
    for k, t in (extra or {}).items():
        tensors[k] = t
    save_file(tensors, str(path), metadata={"format": "pt"})
    return expect
