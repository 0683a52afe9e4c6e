"""GPU parity of the tensor-level kernels (kernels.rs surface) against the oracle.
Tolerance: rel-L2 <= 1e-5 for the f32-accumulated matvecs; bit-exact for embedding and argmax."""
import numpy as np
import pytest
import torch

import oracle as O
import q35
from conftest import rel_l2
from gpu_util import dev, host, normal, q8, q8_dev

pytestmark = pytest.mark.gpu

TOL = 1e-5

# decode projection shapes, (N out, K in); the reference stores each as KN [K][N]
C1_SHAPES = [(6144, 2048), (2048, 6144), (4096, 2048), (512, 2048), (2048, 4096), (8192, 2048), (2048, 2048)]


@pytest.mark.parametrize("M", [1, 8])
@pytest.mark.parametrize("N,K", C1_SHAPES)
def test_q8_gemv_kn_projection_shapes(N, K, M):
    print(f"[gemv_kn] N={N} K={K} M={M}", flush=True)
    W = q8(1000 + N + K, K, N)
    x = normal(7, (M, K))
    y = host(q35.q8_gemv(dev(x), q8_dev(W, q35.Q35_KN)))
    assert rel_l2(y, O.gemv_kn(x, W)) <= TOL


@pytest.mark.parametrize("M", [1, 8])
@pytest.mark.parametrize("N,K", C1_SHAPES)
def test_q8_gemv_nk_projection_shapes(N, K, M):
    print(f"[gemv_nk] N={N} K={K} M={M}", flush=True)
    W = q8(2000 + N + K, N, K)
    x = normal(8, (M, K))
    y = host(q35.q8_gemv(dev(x), q8_dev(W, q35.Q35_NK)))
    ref, _ = O.gemv_nk(x, W)
    assert rel_l2(y, ref) <= TOL


@pytest.mark.parametrize("N,K,M", [(64, 64, 1), (192, 100, 3), (320, 48, 2), (64, 4096, 5), (1024, 16, 8),
                                   (256, 2048, 13), (131072, 64, 1)])
def test_q8_gemv_kn_odd_shapes(N, K, M):
    print(f"[gemv_kn odd] N={N} K={K} M={M}", flush=True)
    W = q8(3000 + N + K, K, N, sigma=1.0)
    x = normal(9, (M, K))
    y = host(q35.q8_gemv_partial_sum(dev(x), q8_dev(W, q35.Q35_KN)))
    assert rel_l2(y, O.gemv_kn(x, W)) <= TOL


@pytest.mark.parametrize("M", [1, 8])
@pytest.mark.parametrize("N,K", C1_SHAPES)
def test_q8_gemv_kn_tiled_projection_shapes(N, K, M):
    print(f"[gemv_kn tiled] N={N} K={K} M={M}", flush=True)
    W = q8(1000 + N + K, K, N)
    x = normal(7, (M, K))
    y = host(q35.q8_gemv(dev(x), q8_dev(W, q35.Q35_KN).tiled()))
    assert rel_l2(y, O.gemv_kn(x, W)) <= TOL


@pytest.mark.parametrize("N,K,M", [(64, 64, 1), (192, 100, 3), (320, 48, 2), (1024, 16, 8), (6400, 2048, 1)])
def test_q8_gemv_kn_tiled_odd_shapes(N, K, M):
    """N not a multiple of the 256-column tile: the padded columns must not reach the output."""
    print(f"[gemv_kn tiled odd] N={N} K={K} M={M}", flush=True)
    W = q8(3000 + N + K, K, N, sigma=1.0)
    x = normal(9, (M, K))
    y = host(q35.q8_gemv(dev(x), q8_dev(W, q35.Q35_KN).tiled()))
    assert y.shape == (M, N)
    assert rel_l2(y, O.gemv_kn(x, W)) <= TOL


@pytest.mark.parametrize("M", [1, 8])
@pytest.mark.parametrize("N,K", C1_SHAPES)
def test_q8_gemv_kn_panel_projection_shapes(N, K, M):
    print(f"[gemv_kn panel] N={N} K={K} M={M}", flush=True)
    W = q8(1000 + N + K, K, N)
    x = normal(7, (M, K))
    y = host(q35.q8_gemv(dev(x), q8_dev(W, q35.Q35_KN).panel()))
    assert rel_l2(y, O.gemv_kn(x, W)) <= TOL


@pytest.mark.parametrize("N,K,M", [(64, 64, 1), (192, 100, 3), (320, 48, 2), (1024, 16, 8), (64, 4096, 5),
                                   (256, 513, 13), (128, 9000, 1), (512, 8193, 2), (64, 1, 4), (131072, 64, 1)])
def test_q8_gemv_kn_panel_odd_shapes(N, K, M):
    """K not a multiple of the block's 512 rows, K past one pass of rows in flight (> 8192 at M=1,
    > 4096 at M=2), a single row, and M spanning several launches of 8 rows."""
    print(f"[gemv_kn panel odd] N={N} K={K} M={M}", flush=True)
    W = q8(3000 + N + K, K, N, sigma=1.0)
    x = normal(9, (M, K))
    y = host(q35.q8_gemv_partial_sum(dev(x), q8_dev(W, q35.Q35_KN).panel()))
    assert y.shape == (M, N)
    assert rel_l2(y, O.gemv_kn(x, W)) <= TOL


def test_q8_gemv_layouts_deterministic_and_reusable():
    """Repeated calls give bit-identical outputs in every KN layout (fixed summation orders;
    the split-K accumulators and tile counters are left zero by each call, so a workspace is
    reused), and one-hot inputs select exact dequantised rows."""
    N, K = 2048, 6144
    W = q8(77, K, N, sigma=1.0)  # |q * scale| >= 2^-9: exact on the 2^-32 fixed-point grid too
    x = dev(normal(78, (3, K)))
    for lay in ("kn", "tiled", "panel"):
        Wd = q8_dev(W, q35.Q35_KN)
        Wd = Wd.tiled() if lay == "tiled" else (Wd.panel() if lay == "panel" else Wd)
        a = host(q35.q8_gemv(x, Wd))
        b = host(q35.q8_gemv(x, Wd))
        np.testing.assert_array_equal(a, b, err_msg=lay)
        e = np.zeros((1, K), np.float32)
        e[0, 4321] = 1.0
        row = host(q35.q8_gemv(dev(e), Wd))[0]
        np.testing.assert_array_equal(row, W.q[4321].astype(np.float32) * np.repeat(W.s[4321], 64), err_msg=lay)


@pytest.mark.parametrize("N,K,M", [(1, 64, 1), (17, 128, 2), (33, 1088, 3), (100, 8192, 1), (4097, 6144, 8)])
def test_q8_gemv_nk_odd_shapes(N, K, M):
    print(f"[gemv_nk odd] N={N} K={K} M={M}", flush=True)
    W = q8(4000 + N + K, N, K, sigma=1.0)
    x = normal(10, (M, K))
    y = host(q35.q8_gemv(dev(x), q8_dev(W, q35.Q35_NK)))
    ref, _ = O.gemv_nk(x, W)
    assert rel_l2(y, ref) <= TOL


def test_q8_gemv_kn_one_hot_exact():
    K, N = 256, 512
    W = q8(11, K, N, sigma=1.0)
    x = np.zeros((4, K), np.float32)
    for i, k in enumerate((0, 63, 128, 255)):
        x[i, k] = 1.0
    y = host(q35.q8_gemv(dev(x), q8_dev(W, q35.Q35_KN)))
    np.testing.assert_array_equal(y, O.gemv_kn(x, W))


@pytest.mark.parametrize("M", [1, 8])
def test_lm_head_full_vocab(M):
    V, D = 248320, 2048
    print(f"[lm_head] V={V} D={D} M={M}", flush=True)
    E = q8(12, V, D)
    h = normal(13, (M, D))
    y = host(q35.q8_lm_head(dev(h), q8_dev(E, q35.Q35_NK)))
    ref, _ = O.gemv_nk(h, E)
    assert rel_l2(y, ref) <= TOL


def test_lm_head_kn_layout_full_vocab():
    """lm_head-sized matrix in the projection (KN) layout, M=1 (the other C1 layout)."""
    V, D = 248320, 2048
    W = q8(14, D, V)
    x = normal(15, (1, D))
    y = host(q35.q8_gemv(dev(x), q8_dev(W, q35.Q35_KN)))
    assert rel_l2(y, O.gemv_kn(x, W)) <= TOL


def test_embedding_lookup_exact():
    V, D = 248320, 2048
    E = q8(16, V, D)
    ids = np.array([0, 1, 248319, 123456, 0], np.int32)
    out = host(q35.q8_embedding_lookup(q8_dev(E, q35.Q35_NK), dev(ids)))
    np.testing.assert_array_equal(out, O.embedding(E, ids))


@pytest.mark.parametrize("B", [1, 5])
def test_gate_proj(B):
    K, nh = 2048, 16
    x = normal(17, (B, K))
    wb, wa = normal(18, (K, nh), 0.02), normal(19, (K, nh), 0.02)
    a_log = np.log(q35.synth_uniform(0, 20, nh, 0.01, 16.0)).astype(np.float32)
    dtb = np.ones(nh, np.float32)
    dtb[0] = 30.0
    beta, g = q35.gate_proj(dev(x), dev(wb), dev(wa), dev(a_log), dev(dtb))
    beta, g = host(beta), host(g)
    for b in range(B):
        ref = O.gate_proj(x[b], wb, wa, a_log, dtb)
        assert rel_l2(beta[b], ref[:nh]) <= TOL
        assert rel_l2(g[b], ref[nh:]) <= TOL


def test_argmax_exact_and_ties():
    V = 248320
    base = normal(21, (V,))
    for idx in (0, 31039, 31040, V - 1, 99999):
        v = base.copy()
        v[idx] = 50.0
        assert int(host(q35.argmax(dev(v)))[0]) == idx
    v = base.copy()
    v[[7, 140000, 200001]] = 60.0
    assert int(host(q35.argmax(dev(v)))[0]) == 7 == O.argmax(v)
    for n in (1, 63, 1000, 3_000_001):
        w = normal(22, (n,))
        assert int(host(q35.argmax(dev(w)))[0]) == O.argmax(w)


def test_argmax_reference_tie_order_bit_exact():
    """Exact ties resolve as the reference's two-stage argmax does (kernels.rs:298-371), checked
    against the oracle's literal restatement of those two kernels."""
    V = 248320
    c = V // 8
    for idx in ([255, 256], [5, 5 + c], [1, c], [512, 256], [257, 1], [V - 1, 255], [V - 1, 31039],
                [c + 3, 2 * c + 3, 3]):
        v = np.zeros(V, np.float32)
        v[idx] = 1.0
        want = O.argmax_reference_order(v)
        assert int(host(q35.argmax(dev(v)))[0]) == want, idx
    v = np.zeros(V, np.float32)
    assert int(host(q35.argmax(dev(v)))[0]) == 0 == O.argmax_reference_order(v)
    g = np.random.default_rng(7)
    for n in (2048, 4096, V):
        for trial in range(6):
            w = g.integers(0, 3, n).astype(np.float32)
            if trial % 2:
                w[g.integers(0, n, 4)] = 9.0
            assert int(host(q35.argmax(dev(w)))[0]) == O.argmax_reference_order(w) == O.argmax(w), (n, trial)
    # the n mod 8 values the reference never reads: read here, after all others on ties
    w = np.zeros(2053, np.float32)
    w[2051] = 2.0
    assert int(host(q35.argmax(dev(w)))[0]) == 2051 == O.argmax(w)
    w[9] = 2.0
    assert int(host(q35.argmax(dev(w)))[0]) == 9 == O.argmax(w)
