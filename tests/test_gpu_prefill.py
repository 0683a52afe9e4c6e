"""GPU parity of the prompt (seq_len > 1) path against the oracle.

* q35_q8_gemm (fp32 matrix cores) against a float64 x @ dequant(W): rel-L2 <= 1e-5, in every
  weight layout, with row strides and accumulation;
* q35_q8f_pack_mb against the MB record layout rebuilt in numpy (bit-exact), and q35_q8_gemm_ws
  on the f16 matrix cores (Q35_KN_MB) against float64: rel-L2 <= 1e-5 overall and per row, rows
  of very different magnitudes, zero rows, accumulation, split K;
* the causal conv + chunked gated delta rule against T recurrent oracle steps (the reference's
  chunked rule equals them, which tests/test_oracle_modules.py pins): core output rel-L2 <= 1e-5,
  recurrent state <= 1e-4, conv state bit-exact (copies of inputs);
* prompt attention against the oracle's per-row attention over the cache: rel-L2 <= 1e-5, cache
  rows of earlier positions untouched;
* whole-model prefill then greedy decode against the oracle fed the prompt token by token:
  identical greedy ids (tiny hybrid model, several prompt lengths, continuation across calls)
  and, at the benchmarked 2B workload, the 513 golden ids of tests/golden/e2e_2b_seed0.npz.
"""
import os

import numpy as np
import pytest
import torch

import oracle as O
import q35
from conftest import rel_l2
from gpu_util import dev, host, normal, q8, q8_dev
from q35._lib import Q35_E_SHAPE

pytestmark = pytest.mark.gpu


# ---------------------------------------------------------------- GEMM

@pytest.mark.parametrize("layout", ["kn", "tiled"])
@pytest.mark.parametrize("K,N", [(2048, 6144), (6144, 2048), (2048, 512), (4096, 2048)])
@pytest.mark.parametrize("M", [1, 5, 130, 512])
def test_q8_gemm_kn_layouts(M, K, N, layout):
    print(f"[gemm] M={M} K={K} N={N} {layout}", flush=True)
    W = q8(200 + K // 64 + N, K, N)
    x = normal(201 + M, (M, K))
    Wd = q8_dev(W, q35.Q35_KN)
    if layout == "tiled":
        Wd = Wd.tiled()
    y = host(q35.q8_gemm(dev(x), Wd))
    ref = x.astype(np.float64) @ W.dequant()
    assert rel_l2(y, ref) <= 1e-5


@pytest.mark.parametrize("M", [3, 64, 200])
def test_q8_gemm_nk_lm_head_rows(M):
    """The NK layout (tied embedding as lm_head matmul, model.rs:130-138) over M rows."""
    print(f"[gemm nk] M={M}", flush=True)
    V, D = 8192, 2048
    E = q8(210, V, D)
    x = normal(211, (M, D))
    y = host(q35.q8_gemm(dev(x), q8_dev(E, q35.Q35_NK)))
    ref = x.astype(np.float64) @ E.dequant().T
    assert rel_l2(y, ref) <= 1e-5


def test_q8_gemm_strides_and_accumulate():
    """x read as a column slice of a wider matrix, y written into a slice of a wider one and
    accumulated onto what it held (the residual add of out_proj / o_proj / down_proj)."""
    M, K, N = 77, 2048, 2048
    W = q8(220, K, N)
    xf = normal(221, (M, K + 192))
    y0 = normal(222, (M, N + 64))
    yd = dev(y0)
    q35.q8_gemm(dev(xf)[:, 64:64 + K], q8_dev(W, q35.Q35_KN).tiled(), yd[:, 64:], accumulate=True)
    y = host(yd)
    ref = y0[:, 64:].astype(np.float64) + xf[:, 64:64 + K].astype(np.float64) @ W.dequant()
    assert rel_l2(y[:, 64:], ref) <= 1e-6
    np.testing.assert_array_equal(y[:, :64], y0[:, :64])


@pytest.mark.parametrize("accumulate", [False, True])
@pytest.mark.parametrize("K,N", [(2048, 2048), (6144, 2048), (4096, 2048), (2048, 512)])
@pytest.mark.parametrize("M", [130, 512])
def test_q8_gemm_split_k(M, K, N, accumulate):
    """q35_q8_gemm_ws: the narrow residual projections (out / o / down: N = 2048) split K over
    more blocks and sum the splits in a second kernel; results against float64, the accumulate
    form onto a strided y slice (rows of y wider than N)."""
    print(f"[gemm split] M={M} K={K} N={N} acc={accumulate}", flush=True)
    W = q8(230 + K // 64 + N, K, N)
    x = normal(231 + M, (M, K))
    y0 = normal(232 + M, (M, N + 64))
    yd = dev(y0)
    q35.q8_gemm(dev(x), q8_dev(W, q35.Q35_KN).tiled(), yd[:, 64:], accumulate=accumulate, split_k=True)
    y = host(yd)
    ref = x.astype(np.float64) @ W.dequant()
    if accumulate:
        ref = ref + y0[:, 64:].astype(np.float64)
    assert rel_l2(y[:, 64:], ref) <= 1e-5
    np.testing.assert_array_equal(y[:, :64], y0[:, :64])


def mb_layout_np(W):
    """The Q35_KN_MB records of a host Q8F [K][N] matrix, rebuilt from the layout's definition:
    per (cb, ks) 2048 bytes, lane l = 16 g + c holds q + 128 of rows 32 ks + 8 g + j (j < 8) for
    columns 64 cb + 16 t + c, t < 4, as [t][j]; scales transposed to [N/64][K]."""
    K, N = W.q.shape
    u = (W.q.astype(np.int16) + 128).astype(np.uint8)            # [K][N]
    v = u.reshape(K // 32, 4, 8, N // 64, 4, 16)                 # [ks][g][j][cb][t][c]
    rec = v.transpose(3, 0, 1, 5, 4, 2)                          # [cb][ks][g][c][t][j]
    return rec.reshape(N // 64, K // 32, 2048), np.ascontiguousarray(W.s.T)


@pytest.mark.parametrize("layout", ["kn", "tiled"])
def test_pack_mb_layout_exact(layout):
    K, N = 256, 384
    W = q8(240, K, N)
    Wd = q8_dev(W, q35.Q35_KN)
    if layout == "tiled":
        Wd = Wd.tiled()
    Wm = Wd.mb()
    qm, sm = mb_layout_np(W)
    np.testing.assert_array_equal(host(Wm.q).view(np.uint8), qm)
    np.testing.assert_array_equal(host(Wm.scale), sm)


@pytest.mark.parametrize("K,N", [(2048, 6144), (6144, 2048), (2048, 512), (4096, 2048), (64, 128), (2048, 8192)])
@pytest.mark.parametrize("M", [1, 5, 130, 512])
def test_q8_gemm_mb(M, K, N):
    """Q35_KN_MB on the f16 matrix cores (int8 exact in f16, x * scale as hi + lo halves) against
    float64, whole-matrix and per-row."""
    print(f"[gemm mb] M={M} K={K} N={N}", flush=True)
    W = q8(250 + K // 64 + N, K, N)
    x = normal(251 + M, (M, K))
    y = host(q35.q8_gemm(dev(x), q8_dev(W, q35.Q35_KN).tiled().mb()))
    ref = x.astype(np.float64) @ W.dequant()
    assert rel_l2(y, ref) <= 1e-5
    for r in range(M):
        assert rel_l2(y[r], ref[r]) <= 1e-5, r


def test_q8_gemm_mb_row_magnitudes_and_zero_rows():
    """Rows from 1e-30 to 1e+20 (the power of two follows each row's largest |x|), rows of zeros,
    a row with one outlier 1e6 x its other entries, scales of very different sizes per block."""
    M, K, N = 40, 2048, 1024
    rng = np.random.default_rng(5)
    W = q8(260, K, N)
    W.s[:, ::3] *= 1e-3  # block scales spanning 1e3 within a row of weights
    x = normal(261, (M, K))
    mags = 10.0 ** rng.uniform(-30, 20, M)
    x = (x * mags[:, None]).astype(np.float32)
    x[3] = 0.0
    x[17] = 0.0
    x[8, 100] *= 1e6
    y = host(q35.q8_gemm(dev(x), q8_dev(W, q35.Q35_KN).mb()))
    ref = x.astype(np.float64) @ W.dequant()
    for r in range(M):
        if not np.any(x[r]):
            np.testing.assert_array_equal(y[r], 0.0)
        else:
            assert rel_l2(y[r], ref[r]) <= 1e-5, (r, mags[r])


@pytest.mark.parametrize("accumulate", [False, True])
@pytest.mark.parametrize("K,N", [(2048, 2048), (6144, 2048), (4096, 2048)])
@pytest.mark.parametrize("M", [130, 512])
def test_q8_gemm_mb_split_k_strided(M, K, N, accumulate):
    """The MB path's split-K launches and the residual add into a strided y slice."""
    print(f"[gemm mb split] M={M} K={K} N={N} acc={accumulate}", flush=True)
    W = q8(270 + K // 64 + N, K, N)
    xf = normal(271 + M, (M, K + 64))
    y0 = normal(272 + M, (M, N + 64))
    yd = dev(y0)
    q35.q8_gemm(dev(xf)[:, 64:], q8_dev(W, q35.Q35_KN).tiled().mb(), yd[:, 64:], accumulate=accumulate)
    y = host(yd)
    ref = xf[:, 64:].astype(np.float64) @ W.dequant()
    if accumulate:
        ref = ref + y0[:, 64:].astype(np.float64)
    assert rel_l2(y[:, 64:], ref) <= 1e-5
    np.testing.assert_array_equal(y[:, :64], y0[:, :64])


# ---------------------------------------------------------------- Gated DeltaNet prompt path

def test_gate_proj_prompt_input_rule():
    """beta = sigmoid(x.W_b); g = -e^A_log * softplus(x.W_a + dt_bias), identity branch when the
    softplus INPUT exceeds 20 (text_modules.rs:587-592)."""
    T, H, nh = 37, 2048, 16
    x = normal(230, (T, H))
    wb, wa = normal(231, (H, nh), 0.02), normal(232, (H, nh), 0.02)
    a_log = normal(233, (nh,), 0.5)
    dtb = np.linspace(-5, 30, nh).astype(np.float32)  # some heads past 20
    out = host(q35.gate_proj_prompt(dev(x), dev(wb), dev(wa), dev(a_log), dev(dtb)))
    b = x.astype(np.float64) @ wb
    a = x.astype(np.float64) @ wa + dtb
    sp = np.where(a > 20, a, np.log1p(np.exp(np.minimum(a, 80))))
    ref = np.concatenate([1 / (1 + np.exp(-b)), -np.exp(a_log.astype(np.float64)) * sp], axis=1)
    assert (a > 20).any() and (a < 20).any()
    np.testing.assert_allclose(out, ref, rtol=2e-5, atol=1e-6)


@pytest.mark.parametrize("T,warm", [(1, True), (3, False), (64, False), (100, True), (257, True)])
def test_gated_delta_rule_prefill_matches_recurrent_steps(T, warm):
    """C2 shapes (16 heads, dk = dv = 128); warm: start from non-zero conv / recurrent states
    (a prompt that continues a conversation)."""
    print(f"[delta rule prefill] T={T} warm={warm}", flush=True)
    nh, dk, dv = 16, 128, 128
    kd = nh * dk
    conv_dim = 2 * kd + nh * dv
    mixed = normal(240, (T, conv_dim))
    beta = (1 / (1 + np.exp(-normal(241, (T, nh)).astype(np.float64)))).astype(np.float32)
    g = (-np.log1p(np.exp(normal(242, (T, nh)).astype(np.float64)))).astype(np.float32)
    bg = np.concatenate([beta, g], axis=1)
    cw = normal(243, (conv_dim, 4), 0.5)
    S0 = normal(244, (nh, dk, dv), 0.1) if warm else np.zeros((nh, dk, dv), np.float32)
    cs0 = normal(245, (conv_dim, 3)) if warm else np.zeros((conv_dim, 3), np.float32)
    S_d, cs_d = dev(S0), dev(cs0)
    out = host(q35.gated_delta_rule_prefill(dev(mixed), dev(bg), cs_d, dev(cw), S_d, nh))
    S_h, cs_h = S0.copy(), cs0.copy()
    ref = np.empty((T, nh * dv), np.float32)
    for t in range(T):
        conv, cs_h = O.conv_update(mixed[t], cs_h, cw)
        o, S_h = O.gated_delta_step(conv[:kd].reshape(nh, dk), conv[kd:2 * kd].reshape(nh, dk),
                                    conv[2 * kd:].reshape(nh, dv), g[t], beta[t], S_h)
        ref[t] = o.reshape(-1)
    e_out, e_S = rel_l2(out, ref), rel_l2(host(S_d), S_h)
    print(f"out rel-L2 {e_out:.2e}  state rel-L2 {e_S:.2e}", flush=True)
    assert e_out <= 1e-5
    assert e_S <= 1e-4
    np.testing.assert_array_equal(host(cs_d), cs_h)


# ---------------------------------------------------------------- attention prompt path

@pytest.mark.parametrize("T,p0", [(1, 0), (17, 0), (100, 0), (33, 40), (64, 0), (130, 300), (5, 500)])
def test_attention_core_prefill(T, p0):
    """C3 head layout (8 q heads, 2 kv heads, 256 dims, RoPE on 64, theta 1e7): rows at
    positions p0..p0+T-1 attend causally to the cache rows 0..p0+t.  The cases cover one and many
    16-key tiles per wave, a ragged last tile and a long cached context before a short prompt."""
    print(f"[attention prefill] T={T} p0={p0}", flush=True)
    d = q35.dims_2b()
    nh, nkv, hd = d.attn_heads, d.kv_heads, d.head_dim
    tmax = p0 + T + 5
    kc = normal(250, (nkv, tmax, hd))
    vc = normal(251, (nkv, tmax, hd))
    qg = normal(252, (T, nh * 2 * hd))
    kn, vn = normal(253, (T, nkv * hd)), normal(254, (T, nkv * hd))
    qw, kw = normal(255, (hd,), 0.1), normal(256, (hd,), 0.1)
    cs, sn = q35.rope_tables(d, tmax)
    kc_d, vc_d = dev(kc), dev(vc)
    out = host(q35.attention_core_prefill(d, dev(qg), dev(kn), dev(vn), dev(qw), dev(kw), kc_d, vc_d, p0, dev(cs),
                                          dev(sn)))
    qs = []
    for t in range(T):
        c, s = O.rope_cos_sin(p0 + t)
        qs.append(np.stack([O.apply_rope(O.rmsnorm(qg[t, h * 2 * hd:h * 2 * hd + hd], qw), c, s) for h in range(nh)]))
        kc[:, p0 + t] = np.stack([O.apply_rope(O.rmsnorm(kn[t, g * hd:(g + 1) * hd], kw), c, s) for g in range(nkv)])
        vc[:, p0 + t] = vn[t].reshape(nkv, hd)
    for t in range(T):
        att = O.attention_core(qs[t], kc, vc, p0 + t + 1).astype(np.float64).reshape(-1)
        gate = qg[t].reshape(nh, 2 * hd)[:, hd:].reshape(-1).astype(np.float64)
        assert rel_l2(out[t], att / (1 + np.exp(-gate))) <= 1e-5, t
    kc_g, vc_g = host(kc_d), host(vc_d)
    np.testing.assert_allclose(kc_g[:, p0:p0 + T], kc[:, p0:p0 + T], rtol=1e-5, atol=1e-5)
    np.testing.assert_array_equal(vc_g[:, p0:p0 + T], vc[:, p0:p0 + T])
    np.testing.assert_array_equal(kc_g[:, :p0], kc[:, :p0])
    np.testing.assert_array_equal(kc_g[:, p0 + T:], kc[:, p0 + T:])


# ---------------------------------------------------------------- whole model

def hybrid_dims():
    """4-layer hybrid (3 Gated DeltaNet + 1 attention) whose greedy ids do not collapse."""
    return q35.make_dims(hidden=512, ffn=1536, vocab=8192, n_layers=4, lin_heads=4, attn_heads=4, kv_heads=2)


def oracle_model(d, seed, tmax):
    return O.Model(O.cfg_from_dims(d), lambda name, n: q35.synth_model_tensor(d, seed, name, n), tmax)


@pytest.mark.parametrize("n_prompt", [5, 64, 150])
@pytest.mark.parametrize("mode", ["persistent", "graph"])
def test_model_prefill_then_decode_matches_oracle(mode, n_prompt):
    print(f"[model prefill] mode={mode} prompt={n_prompt}", flush=True)
    d = hybrid_dims()
    seed, tmax = 3, 256
    prompt = np.random.default_rng(n_prompt).integers(0, d.vocab, n_prompt).astype(np.int32)
    rt, margins = oracle_model(d, seed, tmax).generate(prompt, 30)
    m = q35.TextForCausalLM(d, seed=seed, tmax=tmax)
    toks, _ = m.generate(prompt, 30, mode=mode, prefill=True)
    m.check()
    print("tokens", toks[:10], "min margin", margins.min(), flush=True)
    np.testing.assert_array_equal(toks, rt)
    m.close()


def test_model_prefill_states_match_token_by_token():
    """After a 150-token prompt, the prompt path's recurrent / conv states and KV rows equal
    those of feeding the prompt one decode step at a time."""
    d = hybrid_dims()
    prompt = np.random.default_rng(11).integers(0, d.vocab, 150).astype(np.int32)
    a = q35.TextForCausalLM(d, seed=3, tmax=200)
    a.generate(prompt, 0, mode="persistent")
    a.check()
    b = q35.TextForCausalLM(d, seed=3, tmax=200)
    b.generate(prompt, 0, mode="persistent", prefill=True)
    b.check()
    for l in range(d.n_layers):
        if (l + 1) % d.full_interval == 0:
            for nm in ("k_cache", "v_cache"):
                ta = a.tensor(f"layers.{l}.self_attn.{nm}", np.float32)
                tb = b.tensor(f"layers.{l}.self_attn.{nm}", np.float32)
                assert rel_l2(tb, ta) <= 1e-5, (l, nm)
        else:
            S_a = a.tensor(f"layers.{l}.linear_attn.recurrent_state", np.float32)
            S_b = b.tensor(f"layers.{l}.linear_attn.recurrent_state", np.float32)
            assert rel_l2(S_b, S_a) <= 1e-4, l
            c_a = a.tensor(f"layers.{l}.linear_attn.conv_state", np.float32)
            c_b = b.tensor(f"layers.{l}.linear_attn.conv_state", np.float32)
            assert rel_l2(c_b, c_a) <= 1e-5, l
    assert int(a.tensor("token", np.int32)[0]) == int(b.tensor("token", np.int32)[0])
    assert a.position() == b.position() == 150
    a.close()
    b.close()


def test_model_prefill_continuation_and_second_turn():
    """A prompt split over two prefill calls, then decoding, then a second prompt (a chat turn)
    through the prompt path: the ids equal the oracle's run of the same token sequence."""
    d = hybrid_dims()
    seed, tmax = 3, 300
    rng = np.random.default_rng(7)
    p1 = rng.integers(0, d.vocab, 90).astype(np.int32)
    p2 = rng.integers(0, d.vocab, 41).astype(np.int32)
    ref = oracle_model(d, seed, tmax)
    r1, _ = ref.generate(p1, 20)
    r2, _ = ref.generate(np.concatenate([[r1[-1]], p2]), 15)
    m = q35.TextForCausalLM(d, seed=seed, tmax=tmax)
    m.prefill(p1[:37])
    g1, _ = m.generate(p1[37:], 20, mode="persistent", prefill=True)
    m.check()
    np.testing.assert_array_equal(g1, r1)
    g2, _ = m.generate(np.concatenate([[g1[-1]], p2]), 15, mode="persistent", prefill=True)
    m.check()
    np.testing.assert_array_equal(g2, r2)
    m.close()


def test_model_prefill_longer_than_one_pass():
    """An 1100-token prompt in one prefill call runs as two passes over the same prompt-path
    buffers (1024 + 76 tokens): the ids after it equal the oracle's token-by-token run, and the
    recurrent / conv states and KV rows equal those of feeding the prompt one decode step at a
    time."""
    d = hybrid_dims()
    seed, tmax, n = 3, 1200, 1100
    prompt = np.random.default_rng(21).integers(0, d.vocab, n).astype(np.int32)
    print(f"[long prefill] prompt={n} tmax={tmax}", flush=True)
    rt, margins = oracle_model(d, seed, tmax).generate(prompt, 12)
    a = q35.TextForCausalLM(d, seed=seed, tmax=tmax)
    toks, _ = a.generate(prompt, 12, mode="persistent", prefill=True)
    a.check()
    print("tokens", toks[:8], "min margin", margins.min(), flush=True)
    np.testing.assert_array_equal(toks, rt)
    a.reset()
    a.prefill(prompt)
    b = q35.TextForCausalLM(d, seed=seed, tmax=tmax)
    b.generate(prompt, 0, mode="persistent")
    b.check()
    assert a.position() == b.position() == n
    for l in range(d.n_layers):
        if (l + 1) % d.full_interval == 0:
            for nm in ("k_cache", "v_cache"):
                ta = a.tensor(f"layers.{l}.self_attn.{nm}", np.float32)
                tb = b.tensor(f"layers.{l}.self_attn.{nm}", np.float32)
                assert rel_l2(ta, tb) <= 1e-5, (l, nm)
        else:
            S_a = a.tensor(f"layers.{l}.linear_attn.recurrent_state", np.float32)
            S_b = b.tensor(f"layers.{l}.linear_attn.recurrent_state", np.float32)
            assert rel_l2(S_a, S_b) <= 1e-4, l
            c_a = a.tensor(f"layers.{l}.linear_attn.conv_state", np.float32)
            c_b = b.tensor(f"layers.{l}.linear_attn.conv_state", np.float32)
            assert rel_l2(c_a, c_b) <= 1e-5, l
    assert int(a.tensor("token", np.int32)[0]) == int(b.tensor("token", np.int32)[0])
    a.close()
    b.close()


def test_prompt_path_rejects_unsupported_head_dims():
    """The prompt path's chunked rule is built for 128 x 128 heads: with a value head of 64 the
    model prefill and the batched prompt path report Q35_E_SHAPE before launching anything, and
    the model still decodes token by token afterwards."""
    d = q35.make_dims(hidden=512, ffn=1536, vocab=8192, n_layers=4, lin_heads=4, lin_dv=64, attn_heads=4, kv_heads=2)
    prompt = np.random.default_rng(5).integers(0, d.vocab, 40).astype(np.int32)
    m = q35.TextForCausalLM(d, seed=3, tmax=128)
    with pytest.raises(q35.Q35Error) as e:
        m.prefill(prompt)
    assert e.value.code == Q35_E_SHAPE
    with pytest.raises(q35.Q35Error) as e:
        m.generate(prompt, 4, mode="graph", prefill=True)
    assert e.value.code == Q35_E_SHAPE
    b = q35.BatchDecoder(m, 2, tmax=128)
    with pytest.raises(q35.Q35Error) as e:
        b.generate([prompt, prompt[:17]], 4, prefill=True)
    assert e.value.code == Q35_E_SHAPE
    b.close()
    m.reset()
    rt, _ = oracle_model(d, 3, 128).generate(prompt, 6)
    toks, _ = m.generate(prompt, 6, mode="graph")
    m.check()
    np.testing.assert_array_equal(toks, rt)
    m.close()


def test_2b_prefill_matches_golden_512():
    """The benchmarked workload with its prompt through the prompt path: the 2B-shaped model
    (weights seed 0), the 512-token prompt prefilled on the matrix cores, then 512 greedy steps
    of the persistent kernel; all 513 ids equal the oracle's token-by-token run."""
    print("[model 2b prefill vs golden 512+512]", flush=True)
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "e2e_2b_seed0.npz"))
    prompt, want, margins = g["prompt"], g["tokens"], g["margins"]
    m = q35.TextForCausalLM(q35.dims_2b(), seed=int(g["seed"]), tmax=len(prompt) + len(want) + 64)
    toks, _ = m.generate(prompt, len(want) - 1, mode="persistent", prefill=True)
    m.check()
    m.close()
    bad = np.flatnonzero(toks != want)
    if bad.size:
        i = int(bad[0])
        pytest.fail(f"{bad.size} ids differ; first at step {i}: got {toks[i]}, oracle {want[i]} "
                    f"(oracle margin there {margins[i]:.3g})")
