"""The batched decode's projection kernel on its own (q35_q8_gemv_mb: f16 matrix cores, x * scale
as f16 hi + lo), row by row against the oracle's Q8F matvec (orc_q8_gemv_kn) at rel-L2 <= 1e-5,
at B = 8, 16 and 32 rows, for every prologue the batched step uses: RMSNorm (the qkvz / qkv and
gate|up projections, through the direct path with split factors), the gated RMSNorm (out_proj),
SwiGLU (down_proj) and the plain input (o_proj after the attention merge), with and without the
residual add; both split-K hand-offs on a reused workspace, and the counted one's range guard."""
import ctypes

import numpy as np
import pytest
import torch

import oracle as O
import q35
from conftest import rel_l2
from gpu_util import dev, host, normal, q8, q8_dev
from q35 import _lib as L

pytestmark = pytest.mark.gpu
EPS = 1e-6


def silu(v):
    v = v.astype(np.float64)
    return (v / (1.0 + np.exp(-v))).astype(np.float32)


def run(x, prologue, Wm, N, norm_w=None, z=None, group=0, y0=None, ws=None):
    """q35_q8_gemv_mb over the rows of x (device tensors; y0: rows to add into; ws: a workspace
    to reuse, else a fresh zeroed one)."""
    M = x.shape[0]
    y = y0.clone() if y0 is not None else torch.zeros((M, N), dtype=torch.float32, device="cuda")
    nb = L.lib().q35_q8_gemv_mb_ws_bytes(M, Wm.desc())
    if ws is None:
        ws = torch.zeros(nb // 4 + 64, dtype=torch.float32, device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    L.check(L.lib().q35_q8_gemv_mb(x.data_ptr(), M, x.shape[1], prologue,
                                   norm_w.data_ptr() if norm_w is not None else None,
                                   z.data_ptr() if z is not None else None, z.shape[1] if z is not None else 0, group,
                                   ctypes.c_float(EPS), Wm.desc(), y.data_ptr(), N, 1 if y0 is not None else 0,
                                   ws.data_ptr(), ws.numel() * 4, st))
    L.check(L.lib().q35_workspace_status(ws.data_ptr(), st))
    return host(y)


def check_rows(out, exp):
    for r in range(exp.shape[0]):
        assert rel_l2(out[r], exp[r]) <= 1e-5, r


def mb_matrix(stream, K, N):
    W = q8(stream, K, N)
    return W, q8_dev(W, q35.Q35_KN).mb()


@pytest.mark.parametrize("B", [8, 16, 32])
def test_batched_projection_rms(B):
    """in_proj_qkv|in_proj_z shape [2048 -> 8192] and gate|up [2048 -> 12288 as 6144] with the
    input RMSNorm (1 + w) formed from the raw residual rows."""
    print(f"[batched projection rms] B={B}", flush=True)
    for K, N, s in ((2048, 8192, 300), (2048, 6144, 310)):
        W, Wm = mb_matrix(s, K, N)
        x = normal(s + 1, (B, K), 3.0)
        w = normal(s + 2, (K,), 0.1)
        out = run(dev(x), L.Q35_MB_RMS, Wm, N, norm_w=dev(w))
        xn = np.stack([O.rmsnorm(x[r], w, EPS) for r in range(B)])
        check_rows(out, O.gemv_kn(xn, W))


@pytest.mark.parametrize("B", [8, 16, 32])
def test_batched_projection_gated_norm_with_residual_add(B):
    """out_proj [2048 -> 2048] on RMSNormGated(o, z) per 128-wide head, added into residual rows."""
    print(f"[batched projection gated] B={B}", flush=True)
    K, N, G = 2048, 2048, 128
    W, Wm = mb_matrix(320, K, N)
    o, z = normal(321, (B, K)), normal(322, (B, K))
    w = normal(323, (G,), 0.1) + 1.0
    h0 = normal(324, (B, N))
    out = run(dev(o), L.Q35_MB_GATED, Wm, N, norm_w=dev(w), z=dev(z), group=G, y0=dev(h0))
    xn = np.stack([np.concatenate([O.rmsnorm_gated(o[r, g:g + G], z[r, g:g + G], w, EPS) for g in range(0, K, G)])
                   for r in range(B)])
    check_rows(out, h0 + O.gemv_kn(xn, W))


@pytest.mark.parametrize("B", [8, 16, 32])
def test_batched_projection_swiglu(B):
    """down_proj [6144 -> 2048] on up * silu(gate) from [gate | up] rows, with and without the
    residual add."""
    print(f"[batched projection swiglu] B={B}", flush=True)
    K, N = 6144, 2048
    W, Wm = mb_matrix(330, K, N)
    gu = normal(331, (B, 2 * K))
    xin = gu[:, K:] * silu(gu[:, :K])
    exp = O.gemv_kn(xin, W)
    check_rows(run(dev(gu), L.Q35_MB_SWIGLU, Wm, N), exp)
    h0 = normal(332, (B, N))
    check_rows(run(dev(gu), L.Q35_MB_SWIGLU, Wm, N, y0=dev(h0)), h0 + exp)


@pytest.mark.parametrize("B", [8, 16, 32])
def test_batched_projection_plain(B):
    """o_proj [4096 -> 2048] on the merged attention output rows (plain input), added into
    residual rows, and k_proj [2048 -> 512]."""
    print(f"[batched projection plain] B={B}", flush=True)
    for K, N, s, add in ((4096, 2048, 340, True), (2048, 512, 345, False)):
        W, Wm = mb_matrix(s, K, N)
        x = normal(s + 1, (B, K))
        h0 = normal(s + 2, (B, N))
        out = run(dev(x), L.Q35_MB_PLAIN, Wm, N, y0=dev(h0) if add else None)
        check_rows(out, (h0 if add else 0) + O.gemv_kn(x, W))


@pytest.mark.parametrize("K,N,B", [(2048, 2048, 8), (2048, 512, 8), (2048, 6144, 16), (6144, 2048, 32)])
def test_batched_projection_workspace_reuse(K, N, B):
    """Three calls in a row on one workspace give the same bits as a call on a fresh one: the
    split-K hand-off leaves its counters and counted fixed-point words zero (out_proj and k/v at
    B = 8 hand off through counted words, gate|up at B = 16 and down at B = 32 through partials
    and an arrival counter)."""
    print(f"[batched projection reuse] K={K} N={N} B={B}", flush=True)
    W, Wm = mb_matrix(350 + B, K, N)
    x = normal(351 + B, (B, K))
    h0 = normal(352 + B, (B, N))
    ref = run(dev(x), L.Q35_MB_PLAIN, Wm, N, y0=dev(h0))
    check_rows(ref, h0 + O.gemv_kn(x, W))
    nb = L.lib().q35_q8_gemv_mb_ws_bytes(B, Wm.desc())
    ws = torch.zeros(nb // 4 + 64, dtype=torch.float32, device="cuda")
    for i in range(3):
        out = run(dev(x), L.Q35_MB_PLAIN, Wm, N, y0=dev(h0), ws=ws)
        np.testing.assert_array_equal(out, ref, err_msg=f"call {i}")


@pytest.mark.parametrize("bad", [np.nan, np.inf, 1e12])
def test_batched_projection_counted_range_is_reported(bad):
    """out_proj at B = 8 (a counted split-K hand-off): a row holding NaN / Inf, or a value whose
    partial sums leave the counted words' range (|partial| < 2^22, the persistent step kernel's
    bound), is reported as Q35_E_RANGE through the workspace; the offending contributions count
    as zero, so every word still completes and is cleared, and the next call on the same
    workspace gives the same bits as a call on a fresh one."""
    print(f"[batched projection range] bad={bad}", flush=True)
    K, N, B = 2048, 2048, 8
    W, Wm = mb_matrix(360, K, N)
    x = normal(361, (B, K))
    x[5, 9] = bad
    nb = L.lib().q35_q8_gemv_mb_ws_bytes(B, Wm.desc())
    ws = torch.zeros(nb // 4 + 64, dtype=torch.float32, device="cuda")
    y = torch.zeros((B, N), dtype=torch.float32, device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    L.check(L.lib().q35_q8_gemv_mb(dev(x).data_ptr(), B, K, L.Q35_MB_PLAIN, None, None, 0, 0, ctypes.c_float(EPS),
                                   Wm.desc(), y.data_ptr(), N, 0, ws.data_ptr(), ws.numel() * 4, st))
    assert L.lib().q35_workspace_status(ws.data_ptr(), st) == L.Q35_E_RANGE
    good = normal(362, (B, K))
    fresh = run(dev(good), L.Q35_MB_PLAIN, Wm, N)
    check_rows(fresh, O.gemv_kn(good, W))
    np.testing.assert_array_equal(run(dev(good), L.Q35_MB_PLAIN, Wm, N, ws=ws), fresh)
