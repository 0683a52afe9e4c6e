"""End-to-end decode on the GPU (captured hipGraph and eager launches) against the oracle: greedy
token ids must be identical; the final logits agree to rel-L2 <= 1e-5."""
import numpy as np
import pytest

import oracle as O
import q35
from conftest import rel_l2

pytestmark = pytest.mark.gpu


def tiny_dims():
    return q35.make_dims(hidden=256, ffn=512, vocab=4096, n_layers=8, lin_heads=4, attn_heads=4, kv_heads=2)


def oracle_model(d, seed, tmax):
    return O.Model(O.cfg_from_dims(d), lambda name, n: q35.synth_model_tensor(d, seed, name, n), tmax)


@pytest.mark.parametrize("use_graph", [True, False])
def test_tiny_model_generate_matches_oracle(use_graph):
    d = tiny_dims()
    seed, tmax = 5, 128
    prompt = np.random.default_rng(0).integers(0, d.vocab, 16).astype(np.int32)
    m = q35.TextForCausalLM(d, seed=seed, tmax=tmax)
    toks, _ = m.generate(prompt, 48, use_graph=use_graph)
    logits = m.tensor("logits", np.float32)
    ref = oracle_model(d, seed, tmax)
    rt, margins = ref.generate(prompt, 48)
    print("tokens", toks[:12], "min margin", margins.min(), flush=True)
    np.testing.assert_array_equal(toks, rt)
    # logits of the last decode step
    _, _, last = ref.step(rt[-1], want_logits=True)  # one more step on both sides
    m.set_token(int(rt[-1]))
    m.step(use_graph=use_graph)
    assert rel_l2(m.tensor("logits", np.float32), last) <= 1e-5
    m.close()


def test_graph_replays_match_eager_and_reset():
    d = tiny_dims()
    prompt = np.arange(10, dtype=np.int32) * 37 % d.vocab
    a = q35.TextForCausalLM(d, seed=9, tmax=96)
    t1, _ = a.generate(prompt, 30, use_graph=True)
    a.reset()
    t2, _ = a.generate(prompt, 30, use_graph=False)
    a.reset()
    t3, _ = a.generate(prompt, 30, use_graph=True, readback_each=True)
    np.testing.assert_array_equal(t1, t2)
    np.testing.assert_array_equal(t1, t3)
    # continuing a conversation (cache kept) equals one long prompt
    a.reset()
    first, _ = a.generate(prompt[:4], 0)
    rest, _ = a.generate(prompt[4:], 30)
    np.testing.assert_array_equal(rest, t1)
    a.close()


def test_model_rejects_overflow():
    d = tiny_dims()
    m = q35.TextForCausalLM(d, seed=1, tmax=8)
    with pytest.raises(q35.Q35Error):
        m.generate(np.zeros(4, np.int32), 5)
    with pytest.raises(q35.Q35Error):
        m.set_token(d.vocab)
    m.close()
