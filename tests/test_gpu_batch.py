"""Batched greedy decode (B sequences through the whole step at once) against independent
single-sequence runs: every row's greedy ids equal the oracle's for that sequence alone (tiny
hybrid model; B = 3, 8, 11 and 33, so 16- and 32-row launches and a second row group are covered; ragged
prompt lengths; stream launches and the captured graph; prompts through the decode step and
through the prompt path), and at the 2B shape each row equals the single-sequence persistent
kernel, with the benchmarked 512-token prompt's row equal to its golden ids."""
import os

import numpy as np
import pytest

import oracle as O
import q35

pytestmark = pytest.mark.gpu


def hybrid_dims():
    return q35.make_dims(hidden=512, ffn=1536, vocab=8192, n_layers=4, lin_heads=4, attn_heads=4, kv_heads=2)


def oracle_run(d, seed, prompt, n_new, tmax):
    ref = O.Model(O.cfg_from_dims(d), lambda name, n: q35.synth_model_tensor(d, seed, name, n), tmax)
    return ref.generate(prompt, n_new)[0]


@pytest.mark.parametrize("B", [3, 8, 11, 33])
@pytest.mark.parametrize("mode,prefill", [("graph", False), ("stream", False), ("graph", True)])
def test_batch_rows_match_independent_oracle_runs(B, mode, prefill):
    print(f"[batch] B={B} mode={mode} prefill={prefill}", flush=True)
    d = hybrid_dims()
    seed, n_new = 3, 20
    rng = np.random.default_rng(B)
    lens = rng.integers(1, 40, B)
    prompts = [rng.integers(0, d.vocab, n).astype(np.int32) for n in lens]
    tmax = int(lens.max()) + n_new + 8
    m = q35.TextForCausalLM(d, seed=seed, tmax=tmax)
    bt = q35.BatchDecoder(m, B, tmax)
    toks, _ = bt.generate(prompts, n_new, mode=mode, prefill=prefill)
    for r in range(B):
        want = oracle_run(d, seed, prompts[r], n_new, tmax)
        np.testing.assert_array_equal(toks[r], want, err_msg=f"row {r} (prompt length {lens[r]})")
    if prefill:
        np.testing.assert_array_equal(bt.positions(), lens + n_new)
    bt.close()
    m.close()


@pytest.mark.parametrize("B", [5, 20])
def test_batch_logits_match_oracle(B):
    """Every row's last-step logits against the oracle's for that sequence alone (rel-L2 <= 1e-5
    after the prompt and 12 greedy steps; measured 5e-7 to 8e-7 with the 22-bit f16 hi + lo
    operands), for a 16-row (B = 5) and a 32-row (B = 20) launch."""
    print(f"[batch logits] B={B}", flush=True)
    d = hybrid_dims()
    seed, n_new, plen = 4, 12, 9
    rng = np.random.default_rng(100 + B)
    prompts = [rng.integers(0, d.vocab, plen).astype(np.int32) for _ in range(B)]
    tmax = plen + n_new + 8
    m = q35.TextForCausalLM(d, seed=seed, tmax=tmax)
    bt = q35.BatchDecoder(m, B, tmax)
    toks, _ = bt.generate(prompts, n_new, mode="graph")
    logits = bt.tensor("logits", np.float32).reshape(B, d.vocab).copy()
    for r in range(B):
        ref = O.Model(O.cfg_from_dims(d), lambda name, n: q35.synth_model_tensor(d, seed, name, n), tmax)
        for tok in prompts[r]:
            t, _, _ = ref.step(tok)
        for i in range(n_new):
            t, _, lg = ref.step(t, want_logits=(i == n_new - 1))
        np.testing.assert_array_equal(toks[r][-1], t, err_msg=f"row {r}")
        err = np.linalg.norm(logits[r] - lg) / np.linalg.norm(lg)
        print(f"row {r}: logits rel-L2 {err:.3e}", flush=True)
        assert err <= 1e-5, f"row {r}: logits rel-L2 {err:.2e}"
    bt.close()
    m.close()


def test_batch_continues_and_resets():
    """Decoding on after generate, and a reset batch, give the same ids as a fresh run."""
    d = hybrid_dims()
    rng = np.random.default_rng(5)
    prompts = [rng.integers(0, d.vocab, n).astype(np.int32) for n in (7, 12, 3, 9)]
    m = q35.TextForCausalLM(d, seed=3, tmax=96)
    bt = q35.BatchDecoder(m, 4, 96)
    t1, _ = bt.generate(prompts, 10, mode="graph")
    bt.decode(5, mode="graph")
    hist = bt.tensor("hist", np.int32).reshape(4, 96)
    bt.reset()
    t2, _ = bt.generate(prompts, 10, mode="graph")
    np.testing.assert_array_equal(t1, t2)
    for r, p in enumerate(prompts):
        want = oracle_run(d, 3, p, 10 + (12 - len(p)) + 5, 96)
        np.testing.assert_array_equal(hist[r, len(p) - 1:len(p) - 1 + len(want)], want, err_msg=str(r))
    bt.close()
    m.close()


def test_batch_2b_rows_match_single_sequence_decode():
    print("[batch 2b] B=16", flush=True)
    d = q35.dims_2b()
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "e2e_2b_seed0.npz"))
    B, n_new = 16, 24
    rng = np.random.default_rng(16)
    prompts = [g["prompt"]] + [rng.integers(0, d.vocab, n).astype(np.int32) for n in rng.integers(5, 60, B - 1)]
    tmax = len(g["prompt"]) + n_new + 8
    m = q35.TextForCausalLM(d, seed=int(g["seed"]), tmax=tmax)
    bt = q35.BatchDecoder(m, B, tmax)
    toks, secs = bt.generate(prompts, n_new, mode="graph", prefill=True)
    print(f"batched steps: {B * n_new / secs:.0f} tok/s", flush=True)
    np.testing.assert_array_equal(toks[0], g["tokens"][:n_new + 1])
    for r in range(1, B):
        m.reset()
        want, _ = m.generate(prompts[r], n_new, mode="persistent")
        m.check()
        np.testing.assert_array_equal(toks[r], want, err_msg=f"row {r}")
    bt.close()
    m.close()


def test_batch_weight_copies_match_their_layouts():
    """The copies a batch decoder reads, bit for bit against their definitions: each projection's
    stream-order copy is its MB copy with every 2 KB record's 64 lane records of 32 bytes split in
    two 1 KB halves (lane l's bytes 0-15 at 16 l, bytes 16-31 at 1024 + 16 l); the lm_head's copy
    of the tied [V][H] table is in load order (per 64-row tile t, 128-k round r and (kb, nt) pair,
    lane l = 16 g + c holds row 64 t + 16 nt + c, k = 128 r + 64 kb + 16 g .. + 15; rows past V
    repeat row V - 1: vocab 8100 leaves a partial last tile)."""
    d = q35.make_dims(hidden=512, ffn=1536, vocab=8100, n_layers=4, lin_heads=4, attn_heads=4, kv_heads=2)
    m = q35.TextForCausalLM(d, seed=5, tmax=64)
    bt = q35.BatchDecoder(m, 2, 64)
    try:
        for l, proj in [(0, "in_proj_qkv"), (0, "in_proj_z"), (0, "out_proj"), (3, "q_proj"), (3, "o_proj"),
                        (3, "down_proj")]:
            name = f"mb.layers.{l}.{proj}"
            mb = m.tensor(name, np.uint8).reshape(-1, 64, 2, 16)      # [record][lane][half][16]
            st = m.tensor(name + ".stream", np.uint8).reshape(-1, 2, 64, 16)
            np.testing.assert_array_equal(st, mb.transpose(0, 2, 1, 3), err_msg=name)
        V, H = d.vocab, d.hidden
        q = m.tensor("embed_tokens.q", np.int8).reshape(V, H)
        nt = (V + 63) // 64
        E = q[np.minimum(np.arange(nt * 64), V - 1)].reshape(nt, 4, 16, H // 128, 2, 4, 16)  # [t][nt][c][r][kb][g][b]
        exp = E.transpose(0, 3, 4, 1, 5, 2, 6).reshape(-1)                                  # [t][r][kb][nt][g][c][b]
        np.testing.assert_array_equal(m.tensor("mb.embed_lm", np.int8), exp)
    finally:
        bt.close()
        m.close()
