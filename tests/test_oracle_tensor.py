"""Pinning of the oracle's tensor-level functions (kernels.rs restatements) on the CPU.

Each check is chosen so that a plausible restatement mistake fails it: a transposed operand or
wrong scale index (numpy float64 dequant-matmul in a different loop structure, one-hot inputs),
a dropped row (linearity + one-hot), a wrong tie rule (planted maxima / ties).
"""
import numpy as np
import pytest

import oracle as O
from conftest import rel_l2


def dq(W):
    return W.dequant()


@pytest.mark.parametrize("rows,cols", [(64, 64), (3, 128), (17, 192), (128, 256)])
def test_quantize_properties(rows, cols, rng):
    w = rng.standard_normal((rows, cols)).astype(np.float32) * 0.02
    w[0, :64] = 0.0  # an all-zero block
    W = O.quantize(w)
    assert W.s[0, 0] == 0.0 and np.all(W.q[0, :64] == 0)
    blocks = w.reshape(rows, cols // 64, 64)
    amax = np.abs(blocks).max(axis=2)
    np.testing.assert_array_equal(W.s, (amax / np.float32(127.0)).astype(np.float32))
    qb = W.q.reshape(rows, cols // 64, 64).astype(np.int32)
    nz = amax > 0
    # the largest magnitude of every non-zero block maps to +-127, signs are preserved
    assert np.all(np.abs(qb).max(axis=2)[nz] == 127)
    assert np.all(np.sign(qb) * np.sign(blocks) >= 0)
    # reconstruction error at most half a step
    err = np.abs(dq(W).reshape(rows, cols // 64, 64) - blocks)
    assert np.all(err <= W.s[..., None].astype(np.float64) * 0.5 * (1 + 1e-6) + 1e-30)


def test_quantize_known_answer():
    # block = k/64 * 1.27 for k = 0..63: amax = 1.25015625, scale = amax/127, q = round(w/scale)
    w = (np.arange(64, dtype=np.float32) / np.float32(64.0) * np.float32(1.27)).reshape(1, 64)
    W = O.quantize(w)
    sc = np.float32(w.max()) / np.float32(127.0)
    expect = np.clip(np.sign(w / sc) * np.floor(np.abs(w / sc) + 0.5), -127, 127).astype(np.int8)
    np.testing.assert_array_equal(W.q, expect)
    assert W.q[0, 63] == 127 and W.q[0, 0] == 0
    # round half away from zero: a value exactly half a step above a grid point
    w2 = np.zeros((1, 64), np.float32)
    w2[0, 0] = 127.0
    w2[0, 1] = 2.5
    w2[0, 2] = -2.5
    W2 = O.quantize(w2)
    assert W2.s[0, 0] == 1.0 and W2.q[0, 1] == 3 and W2.q[0, 2] == -3


@pytest.mark.parametrize("K,N,M", [(64, 64, 1), (100, 192, 3), (256, 512, 2), (2048, 512, 1)])
def test_gemv_kn_vs_float64(K, N, M, rng):
    W = O.quantize(rng.standard_normal((K, N)).astype(np.float32) * 0.02)
    x = rng.standard_normal((M, K)).astype(np.float32)
    y = O.gemv_kn(x, W)
    ref = x.astype(np.float64) @ dq(W)
    assert rel_l2(y, ref) < 1e-6


def test_gemv_kn_one_hot_rows(rng):
    K, N = 128, 256
    W = O.quantize(rng.standard_normal((K, N)).astype(np.float32))
    for k in (0, 1, 63, 64, 127):
        x = np.zeros(K, np.float32)
        x[k] = 1.0
        y = O.gemv_kn(x, W)[0]
        np.testing.assert_array_equal(y, (W.q[k].astype(np.float32) * np.repeat(W.s[k], 64)).astype(np.float32))


def test_gemv_kn_linearity(rng):
    K, N = 192, 128
    W = O.quantize(rng.standard_normal((K, N)).astype(np.float32))
    x1 = rng.standard_normal(K).astype(np.float32)
    x2 = rng.standard_normal(K).astype(np.float32)
    y = O.gemv_kn(2.0 * x1 - 0.5 * x2, W)
    y12 = 2.0 * O.gemv_kn(x1, W).astype(np.float64) - 0.5 * O.gemv_kn(x2, W)
    assert rel_l2(y, y12) < 1e-6


def test_rowdrop_emulation_matches_reference_split_rule(rng):
    # kernels.rs:504 -> for N=2048, K=2048: splits = min(25000//2048, 2048//80) = 12, chunk 170,
    # each split sums 8*floor(170/8) = 168 rows, so rows 168,169 of every split (24 rows) and the
    # tail rows 2040..2047 (8 rows) are skipped: 32 rows.
    K, N = 2048, 2048
    assert O.lib().orc_gemv_num_splits(K, N) == 12
    assert O.lib().orc_gemv_num_splits(2048, 6144) == 4
    assert O.lib().orc_gemv_num_splits(6144, 2048) == 12
    assert O.lib().orc_gemv_num_splits(2048, 512) == 25
    W = O.quantize(rng.standard_normal((K, N)).astype(np.float32) * 0.02)
    x = rng.standard_normal(K).astype(np.float32)
    dropped = [s * 170 + r for s in range(12) for r in (168, 169)] + list(range(2040, 2048))
    assert len(dropped) == 32
    x0 = x.copy()
    x0[dropped] = 0.0
    np.testing.assert_allclose(O.gemv_kn(x, W, rowdrop=True), O.gemv_kn(x0, W), rtol=1e-6, atol=1e-6)
    # full-K vs row-drop differ by ~sqrt(32/2048) in relative L2
    r = rel_l2(O.gemv_kn(x, W, rowdrop=True), O.gemv_kn(x, W))
    assert 0.05 < r < 0.3


@pytest.mark.parametrize("N,K,M", [(64, 64, 1), (300, 128, 2), (1024, 2048, 1)])
def test_gemv_nk_vs_float64(N, K, M, rng):
    W = O.quantize(rng.standard_normal((N, K)).astype(np.float32) * 0.02)
    x = rng.standard_normal((M, K)).astype(np.float32)
    y, y64 = O.gemv_nk(x, W)
    ref = x.astype(np.float64) @ dq(W).T
    assert rel_l2(y, ref) < 1e-6
    assert rel_l2(y64, ref) < 1e-12


def test_lm_head_is_dot_with_embedding_rows(rng):
    V, D = 500, 256
    E = O.quantize(rng.standard_normal((V, D)).astype(np.float32) * 0.02)
    h = rng.standard_normal(D).astype(np.float32)
    ids = np.array([0, 7, 499, 250], np.int32)
    rows = O.embedding(E, ids)
    logits, _ = O.gemv_nk(h, E)
    np.testing.assert_allclose(logits[0, ids], rows.astype(np.float64) @ h.astype(np.float64), rtol=1e-6)


def test_embedding_exact(rng):
    V, D = 50, 128
    E = O.quantize(rng.standard_normal((V, D)).astype(np.float32))
    ids = np.array([3, 0, 49, 3], np.int32)
    out = O.embedding(E, ids)
    ref = (E.q[ids].astype(np.float32) * np.repeat(E.s[ids], 64, axis=1)).astype(np.float32)
    np.testing.assert_array_equal(out, ref)


def test_argmax_planted_and_ties(rng):
    V = 248320
    base = rng.standard_normal(V).astype(np.float32)
    for idx in (0, 31039, 31040, V - 1, 123457):
        v = base.copy()
        v[idx] = 100.0
        assert O.argmax(v) == idx == int(np.argmax(v))
        assert O.argmax_reference_order(v) == idx
    v = base.copy()
    v[[5000, 70000, 200000]] = 50.0
    assert O.argmax(v) == 5000 == int(np.argmax(v))


def test_argmax_reference_tie_order():
    """kernels.rs:298-371: unit p = i mod c (c = n/8) keeps the first strict maximum of
    p, p + c, ...; thread t keeps the first of units t, t + 256, ...; thread 0 the first of the
    256 threads.  Known answers for exact ties, on both the literal two-kernel restatement and
    the product's key order."""
    V = 248320
    c = V // 8
    cases = [
        ([255, 256], 256),        # unit 256 feeds thread 0, unit 255 thread 255
        ([5, 5 + c], 5),          # same unit: the first in its scan
        ([1, c], c),              # unit 0 (thread 0) beats unit 1
        ([c + 3, 2 * c + 3, 3], 3),
        ([512, 256], 256),        # thread 0 scans unit 256 before unit 512
        ([257, 1], 1),            # thread 1 scans unit 1 before unit 257
        ([V - 1, 255], V - 1),    # unit c-1 = 31039 sits on thread 63, which beats thread 255
        ([V - 1, 31039], 31039),
    ]
    for idx, want in cases:
        v = np.zeros(V, np.float32)
        v[idx] = 1.0
        assert O.argmax_reference_order(v) == want, idx
        assert O.argmax(v) == want, idx
    v = np.zeros(V, np.float32)  # all equal: unit 0, thread 0
    assert O.argmax_reference_order(v) == 0 == O.argmax(v)


@pytest.mark.parametrize("n", [2048, 4096, 8 * 300, 8 * 31040])
def test_argmax_key_order_equals_two_stage_scan(n):
    """The product's argmax order (a closed-form key per index) equals the literal simulation of
    the reference's two kernels on inputs full of exact ties (values from a set of 3)."""
    g = np.random.default_rng(n)
    for trial in range(12):
        v = g.integers(0, 3, n).astype(np.float32)
        if trial % 3 == 0:
            v[g.integers(0, n, 5)] = 7.0  # a few tied maxima only
        assert O.argmax(v) == O.argmax_reference_order(v)


def test_argmax_tail_and_nan():
    """Values past 8*(n/8), which the reference never reads, are read here: a strict maximum
    there wins; on a tie the indices the reference reads come first.  NaN is never picked."""
    n = 2048 + 5
    v = np.zeros(n, np.float32)
    v[n - 2] = 3.0
    assert O.argmax(v) == n - 2
    v[700] = 3.0
    assert O.argmax(v) == 700
    w = np.arange(10, dtype=np.float32)
    w[9] = np.nan
    assert O.argmax(w) == 8
    assert O.argmax(np.full(5, np.nan, np.float32)) == 0


def test_gate_proj_closed_form(rng):
    K, nh = 256, 16
    x = rng.standard_normal(K).astype(np.float32)
    wb = rng.standard_normal((K, nh)).astype(np.float32) * 0.05
    wa = rng.standard_normal((K, nh)).astype(np.float32) * 0.05
    a_log = np.log(rng.uniform(0.01, 16, nh)).astype(np.float32)
    dtb = np.ones(nh, np.float32)
    dtb[3] = 40.0  # softplus threshold branch: result is x_gate itself
    out = O.gate_proj(x, wb, wa, a_log, dtb)
    b = x.astype(np.float64) @ wb
    a = x.astype(np.float64) @ wa + dtb
    beta = 1 / (1 + np.exp(-b))
    sp = np.where(a > 20, a, np.log1p(np.exp(a)))
    g = -np.exp(a_log.astype(np.float64)) * sp
    np.testing.assert_allclose(out[:nh], beta, rtol=2e-6)
    np.testing.assert_allclose(out[nh:], g, rtol=2e-5)
    assert abs(out[nh + 3] / (-np.exp(a_log[3])) - a[3]) < 1e-4


def test_f32_dequant_timing_path_matches_checker(rng):
    """The CPU-baseline timing path (f32 dequantised matrix, f32 accumulation) computes the same
    matvecs as the double-accumulated checker to f32 accuracy, in both layouts."""
    K, N, M = 512, 320, 3
    W = O.quantize(rng.standard_normal((K, N)).astype(np.float32) * 0.05)
    E = O.quantize(rng.standard_normal((N, K)).astype(np.float32) * 0.05)
    x = rng.standard_normal((M, K)).astype(np.float32)
    ref_kn = O.gemv_kn(x, W)
    ref_nk, _ = O.gemv_nk(x, E)
    try:
        O.set_f32_dequant(True)
        got_kn = O.gemv_kn(x, W)
        got_nk, got64 = O.gemv_nk(x, E)
    finally:
        O.set_f32_dequant(False)
    assert rel_l2(got_kn, ref_kn) <= 1e-5 and rel_l2(got_nk, ref_nk) <= 1e-5
    np.testing.assert_array_equal(got64, got_nk.astype(np.float64))
    assert not np.array_equal(got_kn, ref_kn)  # it really is the other (f32) path
