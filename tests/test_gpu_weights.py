"""The decoder built from a safetensors checkpoint (main.rs:160-222 ingestion) on the GPU:
with the synthetic model's values written as an F32 checkpoint it is the same model (identical
greedy ids and bit-identical logits); from a BF16 checkpoint it decodes the oracle's greedy ids
for the bf16-rounded weights, through the prompt path and the persistent decode kernel."""
import numpy as np
import pytest
import torch

import oracle as O
import q35
from hf_checkpoint import write

pytestmark = pytest.mark.gpu


def hybrid_dims():
    return q35.make_dims(hidden=512, ffn=1536, vocab=8192, n_layers=4, lin_heads=4, attn_heads=4, kv_heads=2)


def test_f32_checkpoint_is_the_synthetic_model(tmp_path):
    print("[weights f32]", flush=True)
    d = hybrid_dims()
    path = tmp_path / "model.safetensors"
    write(path, d, seed=3)
    prompt = np.random.default_rng(3).integers(0, d.vocab, 8).astype(np.int32)
    a = q35.TextForCausalLM(d, seed=3, tmax=96)
    ta, _ = a.generate(prompt, 30, mode="persistent")
    a.check()
    la = a.tensor("logits", np.float32).copy()
    a.close()
    b = q35.TextForCausalLM.from_safetensors(path, d, tmax=96)
    tb, _ = b.generate(prompt, 30, mode="persistent")
    b.check()
    np.testing.assert_array_equal(tb, ta)
    np.testing.assert_array_equal(b.tensor("logits", np.float32), la)
    b.close()


def test_bf16_checkpoint_matches_oracle(tmp_path):
    print("[weights bf16]", flush=True)
    d = hybrid_dims()
    path = tmp_path / "model.safetensors"
    vals = write(path, d, seed=7, dtype=torch.bfloat16)
    prompt = np.random.default_rng(7).integers(0, d.vocab, 40).astype(np.int32)
    ref = O.Model(O.cfg_from_dims(d), lambda name, n: vals[name][:n], 160)
    rt, margins = ref.generate(prompt, 40)
    m = q35.TextForCausalLM.from_safetensors(path, d, tmax=160)
    for prefill in (False, True):
        m.reset()
        toks, _ = m.generate(prompt, 40, mode="persistent", prefill=prefill)
        m.check()
        print("prefill", prefill, "tokens", toks[:8], "min margin", margins.min(), flush=True)
        np.testing.assert_array_equal(toks, rt)
    m.close()


def test_missing_tensor_is_reported(tmp_path):
    d = hybrid_dims()
    path = tmp_path / "model.safetensors"
    write(path, d, seed=1, drop=("layers.3.self_attn.k_norm",))
    with pytest.raises(q35.Q35Error, match="k_norm"):
        q35.TextForCausalLM.from_safetensors(path, d, tmax=32)
