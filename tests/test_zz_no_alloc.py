"""q35_q8_gemv_noalloc (the allocation-free matvec, scratch in a fixed device array) against the
workspace entry point q35_q8_gemv, called through the C ABI: identical outputs (the same kernels
and summation order), within rel-L2 1e-5 of the oracle, on two calls in a row with the second
smaller, in every layout; sizes beyond the fixed scratch are rejected."""
import numpy as np
import pytest
import torch

import oracle as O
import q35
from conftest import rel_l2
from gpu_util import dev, host, normal, q8, q8_dev

pytestmark = pytest.mark.gpu

L = q35._lib


def _gemv_ws(x, W):
    """Reference call: q35_q8_gemv with a fresh zeroed workspace."""
    M, K = x.shape
    y = torch.empty(M, W.cols if W.layout != L.Q35_NK else W.rows, device="cuda")
    d = W.desc()
    ws = torch.zeros(max(1, L.lib().q35_q8_gemv_ws_bytes(M, d)), dtype=torch.uint8, device="cuda")
    L.check(L.lib().q35_q8_gemv(x.data_ptr(), M, d, y.data_ptr(), ws.data_ptr(), ws.numel(),
                                torch.cuda.current_stream().cuda_stream))
    return host(y)


def _gemv_noalloc(x, W):
    M, K = x.shape
    y = torch.empty(M, W.cols if W.layout != L.Q35_NK else W.rows, device="cuda")
    L.check(L.lib().q35_q8_gemv_noalloc(x.data_ptr(), M, W.desc(), y.data_ptr(),
                                        torch.cuda.current_stream().cuda_stream))
    return host(y)


@pytest.mark.parametrize("layout", ["kn", "tiled", "panel", "nk"])
def test_noalloc_matches_workspace_entry_point(layout):
    print(f"[noalloc] layout={layout}", flush=True)
    for call, (N, K, M) in enumerate([(8192, 2048, 8), (2048, 6144, 3)]):  # second call smaller
        if layout == "nk":
            W = q8(5000 + call, N, K)
            Wd = q8_dev(W, L.Q35_NK)
        else:
            W = q8(5000 + call, K, N)
            Wd = q8_dev(W, L.Q35_KN)
            Wd = Wd.tiled() if layout == "tiled" else (Wd.panel() if layout == "panel" else Wd)
        xh = normal(5100 + call, (M, K))
        x = dev(xh)
        got = _gemv_noalloc(x, Wd)
        want = _gemv_ws(x, Wd)
        np.testing.assert_array_equal(got, want)
        ref = O.gemv_nk(xh, W)[0] if layout == "nk" else O.gemv_kn(xh, W)
        assert rel_l2(got, ref) <= 1e-5


def test_noalloc_repeated_calls_stay_exact():
    """The scratch is left zero by every call: many calls of mixed sizes keep matching."""
    shapes = [(6144, 2048, 1), (512, 2048, 8), (6144, 2048, 1), (16384, 256, 8), (2048, 2048, 2)]
    for i, (N, K, M) in enumerate(shapes):
        W = q8(5200 + i, K, N)
        Wd = q8_dev(W, L.Q35_KN).tiled()
        x = dev(normal(5300 + i, (M, K)))
        np.testing.assert_array_equal(_gemv_noalloc(x, Wd), _gemv_ws(x, Wd), err_msg=str((N, K, M)))


def test_noalloc_rejects_sizes_beyond_its_scratch():
    W = q8(5400, 64, 16448)  # N = 16448 > 131072 / 8 at M = 8: rejected before any GPU work
    Wd = q8_dev(W, L.Q35_KN)
    x = torch.zeros(8, 64, device="cuda")
    y = torch.empty(8, 16448, device="cuda")
    rc = L.lib().q35_q8_gemv_noalloc(x.data_ptr(), 8, Wd.desc(), y.data_ptr(), torch.cuda.current_stream().cuda_stream)
    assert rc == L.Q35_E_SHAPE and b"131072" in L.lib().q35_last_error()
