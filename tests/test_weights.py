"""CPU tests of the safetensors ingestion (main.rs:160-222) against the safetensors library's
own writer: every decoder tensor read back through the loader equals the written values in the
builder's layout (Linear weights transposed to [in][out], conv1d squeezed, F32 / F16 / BF16
cast to f32 exactly), under the key forms the reference accepts (`model.language_model.` or
`language_model.`, `A_log`), and bad checkpoints are refused with the offending key named."""
import numpy as np
import pytest
import torch

import q35
from hf_checkpoint import decoder_tensors, write


def tiny():
    return q35.make_dims(hidden=256, ffn=512, vocab=1024, n_layers=4, lin_heads=2, attn_heads=4, kv_heads=2)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("prefix", ["model.language_model.", "language_model."])
def test_loader_reads_every_decoder_tensor(tmp_path, dtype, prefix):
    d = tiny()
    path = tmp_path / "model.safetensors"
    expect = write(path, d, seed=5, dtype=dtype, prefix=prefix,
                   extra={"lm_head.weight": torch.zeros(4, 4), "model.visual.blocks.0.attn.qkv.weight": torch.ones(8)})
    for name, _, rows, cols, _ in decoder_tensors(d):
        got = q35.safetensors_tensor(path, d, name, rows * cols)
        np.testing.assert_array_equal(got, expect[name], err_msg=name)


def test_loader_transposes_linear_weights(tmp_path):
    """A Linear weight written as PyTorch's [out][in] comes back as [in][out]: element
    (out o, in i) lands at row i, column o."""
    d = tiny()
    path = tmp_path / "m.safetensors"
    write(path, d, seed=1)
    name = "layers.0.mlp.down_proj"  # [in = ffn][out = hidden]
    w = q35.safetensors_tensor(path, d, name, d.ffn * d.hidden).reshape(d.ffn, d.hidden)
    from safetensors.numpy import load_file
    raw = load_file(str(path))["model.language_model." + name + ".weight"]
    assert raw.shape == (d.hidden, d.ffn)
    np.testing.assert_array_equal(w, raw.T)


def test_loader_reports_missing_and_misshaped_tensors(tmp_path):
    d = tiny()
    p1 = tmp_path / "missing.safetensors"
    write(p1, d, seed=2, drop=("layers.1.linear_attn.in_proj_z",))
    with pytest.raises(q35.Q35Error, match="layers.1.linear_attn.in_proj_z"):
        q35.safetensors_tensor(p1, d, "layers.1.linear_attn.in_proj_z", d.hidden * d.lin_heads * d.lin_dv)
    p2 = tmp_path / "bias.safetensors"
    write(p2, d, seed=2, extra={"model.language_model.layers.0.linear_attn.conv1d.bias": torch.zeros(8)})
    conv = 2 * d.lin_heads * d.lin_dk + d.lin_heads * d.lin_dv
    with pytest.raises(q35.Q35Error, match="conv1d.bias"):
        q35.safetensors_tensor(p2, d, "layers.0.linear_attn.conv1d", conv * d.conv_k)
    d2 = q35.make_dims(hidden=256, ffn=640, vocab=1024, n_layers=4, lin_heads=2, attn_heads=4, kv_heads=2)
    with pytest.raises(q35.Q35Error, match="gate_proj"):
        q35.safetensors_tensor(p1, d2, "layers.0.mlp.gate_proj", d2.hidden * d2.ffn)
    p3 = tmp_path / "garbage.safetensors"
    p3.write_bytes(b"\x10\x00\x00\x00\x00\x00\x00\x00{not json}......")
    with pytest.raises(q35.Q35Error, match="header"):
        q35.safetensors_tensor(p3, d, "norm", d.hidden)
