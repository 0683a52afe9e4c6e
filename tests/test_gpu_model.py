"""End-to-end decode on the GPU in every launch mode (persistent step kernel, captured hipGraph,
eager launches) against the oracle: greedy token ids must be identical; the final logits agree
to rel-L2 <= 1e-5."""
import os

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


MODES = ["persistent", "graph", "stream"]


@pytest.mark.parametrize("mode", MODES)
def test_tiny_model_generate_matches_oracle(mode):
    print(f"[model tiny] mode={mode}", flush=True)
    d = tiny_dims()
    seed, tmax = 5, 128
    prompt = np.random.default_rng(0).integers(0, d.vocab, 16).astype(np.int32)
    m = q35.TextForCausalLM(d, seed=seed, tmax=tmax)
    toks, _ = m.generate(prompt, 48, mode=mode)
    m.check()
    logits = m.tensor("logits", np.float32)
    ref = oracle_model(d, seed, tmax)
    rt, margins = ref.generate(prompt, 48)
    print("tokens", toks[:12], "min margin", margins.min(), flush=True)
    np.testing.assert_array_equal(toks, rt)
    # logits of the last decode step
    _, _, last = ref.step(rt[-1], want_logits=True)  # one more step on both sides
    m.set_token(int(rt[-1]))
    m.step(mode=mode)
    m.check()
    assert rel_l2(m.tensor("logits", np.float32), last) <= 1e-5
    m.close()


def test_launch_modes_agree_and_reset():
    print("[model modes]", flush=True)
    d = tiny_dims()
    prompt = np.arange(10, dtype=np.int32) * 37 % d.vocab
    a = q35.TextForCausalLM(d, seed=9, tmax=96)
    t1, _ = a.generate(prompt, 30, mode="graph")
    runs = {}
    for mode in MODES:
        for rb in (False, True):
            a.reset()
            runs[(mode, rb)], _ = a.generate(prompt, 30, mode=mode, readback_each=rb)
            a.check()
    for k, t in runs.items():
        np.testing.assert_array_equal(t, t1, err_msg=str(k))
    # continuing a conversation (cache kept) equals one long prompt, in every mode
    for mode in MODES:
        a.reset()
        first, _ = a.generate(prompt[:4], 0, mode=mode)
        rest, _ = a.generate(prompt[4:], 30, mode=mode)
        a.check()
        np.testing.assert_array_equal(rest, t1, err_msg=mode)
    # mixing modes mid-stream: the persistent kernel and the per-op kernels share all state
    a.reset()
    first, _ = a.generate(prompt, 10, mode="persistent")
    a.decode(12, mode="graph")
    a.decode(8, mode="persistent")
    a.check()
    hist = a.tensor("hist", np.int32)
    np.testing.assert_array_equal(hist[len(prompt) - 1:len(prompt) + 30], t1)
    a.close()


def stop_dims():
    """A 4-layer hybrid whose greedy ids do not repeat one token (38 distinct of 41 at seed 3)."""
    return q35.make_dims(hidden=512, ffn=1536, vocab=8192, n_layers=4, lin_heads=4, attn_heads=4, kv_heads=2)


@pytest.mark.parametrize("mode", MODES)
def test_generate_until_stop_ids(mode):
    """main.rs:105-110: the loop ends at the first current token that is a stop id, which is not
    forwarded; the tokens before it, the position and the token slot are what the reference
    leaves.  Decoding on afterwards (the stop id is forwarded next, as main.rs:141-144 does with
    <|im_end|>) gives the history of a run without stop ids, so a launch that ended early left
    every state and the barrier counters consistent.  Stops are planted at an even and an odd
    index (the persistent kernel double-buffers its states per step) and on the first token."""
    print(f"[model stop ids] mode={mode}", flush=True)
    d = stop_dims()
    seed, tmax, n = 3, 96, 40
    prompt = np.random.default_rng(seed).integers(0, d.vocab, 8).astype(np.int32)
    rt, _ = oracle_model(d, seed, tmax).generate(prompt, n)
    unused = next(t for t in range(d.vocab) if t not in set(rt.tolist()))
    firsts = [j for j in range(4, n) if rt[j] not in set(rt[:j].tolist())]
    cases = [next(j for j in firsts if j % 2 == 0), next(j for j in firsts if j % 2 == 1), 0]
    m = q35.TextForCausalLM(d, seed=seed, tmax=tmax)
    P = len(prompt)
    for j in cases:
        m.reset()
        produced, last, _ = m.generate_until(prompt, n, stop_ids=[unused, int(rt[j])], mode=mode)
        m.check()
        print("stop at", j, "produced", len(produced), "last", last, flush=True)
        np.testing.assert_array_equal(produced, rt[:j])
        assert last == rt[j]
        assert m.position() == P + j
        assert int(m.tensor("pos", np.int32)[0]) == P + j
        assert int(m.tensor("token", np.int32)[0]) == rt[j]
        m.decode(n - j, mode=mode)
        m.check()
        np.testing.assert_array_equal(m.tensor("hist", np.int32)[P - 1:P + n], rt)
    # no stop id met: max_new ids produced, the next argmax returned
    m.reset()
    produced, last, _ = m.generate_until(prompt, 7, stop_ids=[unused], mode=mode)
    m.check()
    np.testing.assert_array_equal(produced, rt[:7])
    assert last == rt[7] and m.position() == P + 7
    # a stop id inside the prompt does not end anything: only generated tokens are checked
    m.reset()
    produced, last, _ = m.generate_until(prompt, 5, stop_ids=[int(prompt[3]), int(prompt[-1])], mode=mode)
    m.check()
    np.testing.assert_array_equal(produced, rt[:5])
    m.close()


def test_persistent_multi_step_launch_equals_single_steps():
    """decode(n) as one launch vs n launches of one step: identical history."""
    print("[model persistent multi]", flush=True)
    d = tiny_dims()
    prompt = np.arange(7, dtype=np.int32) * 11 % d.vocab
    a = q35.TextForCausalLM(d, seed=4, tmax=64)
    a.generate(prompt, 0, mode="persistent")
    a.decode(40, mode="persistent")
    a.check()
    h1 = a.tensor("hist", np.int32)[:47].copy()
    a.reset()
    a.generate(prompt, 0, mode="persistent")
    for _ in range(40):
        a.step(mode="persistent")
    a.check()
    h2 = a.tensor("hist", np.int32)[:47]
    np.testing.assert_array_equal(h1, h2)
    a.close()


@pytest.mark.parametrize("mode", ["persistent", "graph", "prompt"])
def test_fused_argmax_reference_tie_order(mode):
    """The lm_head's fused argmax resolves exact ties as the reference's two-stage argmax
    (kernels.rs:298-371).  The winning row of the tied embedding table is copied into rows that
    the reference's scan visits earlier and later, so those logits are bit-identical to the max;
    the token picked must be the reference order's pick over the GPU's own logits.  mode
    "prompt": the token after a prompt through the prompt path, which picks it in the same order
    (the reference picks that one with Burn's argmax(2), main.rs:92-95, whose tie rule no fixture
    pins: parity unpinned for exact ties there)."""
    print(f"[model argmax ties] mode={mode}", flush=True)
    d = tiny_dims()
    c = d.vocab // 8
    prompt = (np.arange(12, dtype=np.int32) * 97 + 1000) % d.vocab
    m = q35.TextForCausalLM(d, seed=6, tmax=64)
    kw = dict(mode="persistent", prefill=True) if mode == "prompt" else dict(mode=mode)
    toks, _ = m.generate(prompt, 0, **kw)
    m.check()
    w = int(toks[0])
    q = m.tensor("embed_tokens.q", np.int8).reshape(d.vocab, d.hidden).copy()
    sc = m.tensor("embed_tokens.scale", np.float32).reshape(d.vocab, d.hidden // 64).copy()
    cand = {256, c + 256, 3 * c + 1, (w + c) % d.vocab, (w % c) + 256 if (w % c) + 256 < c else 512}
    dups = sorted(cand - {w} - set(prompt.tolist()))  # rows the prompt does not embed
    assert len(dups) >= 3
    q[dups] = q[w]
    sc[dups] = sc[w]
    m.set_tensor("embed_tokens.q", q)
    m.set_tensor("embed_tokens.scale", sc)
    m.reset()
    toks2, _ = m.generate(prompt, 0, **kw)
    m.check()
    logits = m.tensor("logits", np.float32)
    tied = np.flatnonzero(logits == logits.max())
    print("winner", w, "tied", tied.tolist(), "picked", int(toks2[0]), flush=True)
    assert len(tied) >= 2 and set(dups) <= set(tied.tolist())
    assert int(toks2[0]) == O.argmax_reference_order(logits) == O.argmax(logits)
    m.close()


def test_persistent_error_is_sticky():
    """A persistent-kernel failure (forced from the host by setting the error word, so every
    block returns at entry) makes later launches no-ops that leave the state untouched; check()
    keeps raising and persistent steps are refused until reset(), after which decoding matches a
    fresh model."""
    print("[model sticky error]", flush=True)
    d = tiny_dims()
    prompt = np.arange(9, dtype=np.int32) * 13 % d.vocab
    ref = q35.TextForCausalLM(d, seed=8, tmax=64)
    want, _ = ref.generate(prompt, 10, mode="persistent")
    ref.check()
    ref.close()
    m = q35.TextForCausalLM(d, seed=8, tmax=64)
    m.generate(prompt, 2, mode="persistent")
    m.check()
    hist0 = m.tensor("hist", np.int32).copy()
    pos0 = int(m.tensor("pos", np.int32)[0])
    m.set_tensor("step_error", np.ones(1, np.uint32))
    m.decode(5, mode="persistent")
    m.decode(3, mode="persistent")
    with pytest.raises(q35.Q35Error):
        m.check()
    np.testing.assert_array_equal(m.tensor("hist", np.int32), hist0)
    assert int(m.tensor("pos", np.int32)[0]) == pos0
    with pytest.raises(q35.Q35Error):
        m.decode(1, mode="persistent")
    with pytest.raises(q35.Q35Error):
        m.check()
    m.reset()
    got, _ = m.generate(prompt, 10, mode="persistent")
    m.check()
    np.testing.assert_array_equal(got, want)
    m.close()


def test_model_rejects_overflow():
    d = tiny_dims()
    m = q35.TextForCausalLM(d, seed=1, tmax=8)
    with pytest.raises(q35.Q35Error):
        m.generate(np.zeros(4, np.int32), 5)
    with pytest.raises(q35.Q35Error):
        m.set_token(d.vocab)
    m.close()


def test_2b_persistent_matches_oracle_short():
    """Full Qwen3.5-2B shapes: 12-token prompt + 12 greedy steps, persistent kernel vs oracle."""
    print("[model 2b persistent vs oracle]", flush=True)
    d = q35.dims_2b()
    seed, tmax = 0, 64
    prompt = np.random.default_rng(3).integers(0, d.vocab, 12).astype(np.int32)
    m = q35.TextForCausalLM(d, seed=seed, tmax=tmax)
    toks, _ = m.generate(prompt, 12, mode="persistent")
    m.check()
    ref = oracle_model(d, seed, tmax)
    rt, margins = ref.generate(prompt, 12)
    print("tokens", toks, "min margin", margins.min(), flush=True)
    np.testing.assert_array_equal(toks, rt)
    m.close()


def test_2b_persistent_matches_graph_long_context():
    """Full shapes over a 600-token context (many attention chunks per kv head): the persistent
    kernel and the per-op graph give the same greedy ids and near-identical final logits."""
    print("[model 2b persistent vs graph]", flush=True)
    d = q35.dims_2b()
    tmax = 700
    prompt = np.random.default_rng(5).integers(0, d.vocab, 600).astype(np.int32)
    m = q35.TextForCausalLM(d, seed=1, tmax=tmax)
    tp, _ = m.generate(prompt, 40, mode="persistent")
    m.check()
    lp = m.tensor("logits", np.float32).copy()
    m.reset()
    tg, _ = m.generate(prompt, 40, mode="graph")
    lg = m.tensor("logits", np.float32)
    np.testing.assert_array_equal(tp, tg)
    assert rel_l2(lp, lg) <= 1e-4
    m.close()


def test_2b_persistent_matches_graph_beyond_32k():
    """Full shapes over a 34,000-token context: attention items of 266 cached tokens each (more
    than 256), the persistent kernel against the per-op graph step (whose attention is the
    separate attn_chunk / attn_merge kernels): the same greedy ids and near-identical final
    logits.  The prompt goes through the prompt path."""
    print("[model 2b persistent vs graph, 34k context]", flush=True)
    d = q35.dims_2b()
    n_prompt, n_new = 34000, 6
    tmax = n_prompt + n_new + 8
    prompt = np.random.default_rng(7).integers(0, d.vocab, n_prompt).astype(np.int32)
    m = q35.TextForCausalLM(d, seed=2, tmax=tmax)
    tp, _ = m.generate(prompt, n_new, mode="persistent", prefill=True)
    m.check()
    lp = m.tensor("logits", np.float32).copy()
    m.reset()
    tg, _ = m.generate(prompt, n_new, mode="graph", prefill=True)
    m.check()
    lg = m.tensor("logits", np.float32)
    np.testing.assert_array_equal(tp, tg)
    assert rel_l2(lp, lg) <= 1e-4
    m.close()


def test_2b_persistent_matches_golden_512():
    """The benchmarked workload end to end: the 2B-shaped model (weights seed 0), a 512-token
    prompt and 512 greedy steps through the persistent kernel; all 513 greedy ids equal the
    oracle's, stored in tests/golden/e2e_2b_seed0.npz by tests/golden/make_e2e_2b.py (smallest
    oracle top-1 / top-2 margin over the run: 5.1e-4)."""
    print("[model 2b persistent vs golden 512+512]", flush=True)
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "e2e_2b_seed0.npz"))
    prompt, want, margins = g["prompt"], g["tokens"], g["margins"]
    d = q35.dims_2b()
    m = q35.TextForCausalLM(d, seed=int(g["seed"]), tmax=len(prompt) + len(want) + 64)
    toks, _ = m.generate(prompt, len(want) - 1, mode="persistent")
    m.check()
    m.close()
    bad = np.flatnonzero(toks != want)
    if bad.size:
        i = int(bad[0])
        pytest.fail(f"{bad.size} ids differ; first at step {i}: got {toks[i]}, oracle {want[i]} "
                    f"(oracle margin there {margins[i]:.3g})")


def test_decode_stream_matches_decode():
    """Streamed persistent decode (q35_model_decode_stream): the tokens the host reads from the
    pinned token stream while the kernel runs equal the ids the synchronous persistent decode
    records, over two consecutive streamed calls (positions continue) and after a reset; at the
    2B shape (one 24-step launch) and the tiny hybrid model."""
    print("[decode stream]", flush=True)
    for d, seed, plen in ((q35.dims_2b(), 3, 40), (tiny_dims(), 4, 9)):
        rng = np.random.default_rng(seed)
        prompt = rng.integers(0, d.vocab, plen).astype(np.int32)
        m = q35.TextForCausalLM(d, seed=seed, tmax=plen + 64)
        want, _ = m.generate(prompt, 24, mode="persistent")
        m.reset()
        first, _ = m.generate(prompt, 0, mode="persistent")
        got = [int(first[0])] + list(m.decode_stream(16)) + list(m.decode_stream(8))
        np.testing.assert_array_equal(got, want)
        np.testing.assert_array_equal(m.tensor("hist", np.int32)[plen - 1:plen + 24], want)
        m.close()


def test_decode_stream_with_stop_ids_matches_decode_until():
    """Streamed decode with stop ids ends where decode_until does: the tokens it yields are
    decode_until's produced ids (its step inputs) shifted by one plus the stop id, and the model
    is left at the same position with the same token slot (tiny hybrid model; the stop id is the
    10th generated token, then one that never comes)."""
    print("[decode stream stop ids]", flush=True)
    d = tiny_dims()
    prompt = np.random.default_rng(11).integers(0, d.vocab, 9).astype(np.int32)
    m = q35.TextForCausalLM(d, seed=5, tmax=96)
    ref, _ = m.generate(prompt, 40, mode="persistent")
    for stop, expect_stop in ((int(ref[10]), True), (d.vocab - 1 if d.vocab - 1 not in ref else 0, False)):
        m.reset()
        m.generate(prompt, 0, mode="persistent")
        got, last, _ = m.decode_until(30, stop_ids=[stop], mode="persistent")
        pos_u, tok_u = m.position(), m.current_token()
        m.reset()
        m.generate(prompt, 0, mode="persistent")
        cur = m.current_token()
        streamed = list(m.decode_stream(30, stop_ids=[stop]))
        assert cur == got[0]
        np.testing.assert_array_equal(streamed[:-1], got[1:])
        assert streamed[-1] == last
        assert (last == stop) == expect_stop
        assert m.position() == pos_u and m.current_token() == tok_u
    m.close()
