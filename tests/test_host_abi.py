"""CPU-only checks of libq35.so: it loads, exports every entry point include/q35.h declares,
its host utilities (generator, quantiser, rope tables) agree with the oracle, and argument
validation returns error codes without touching a GPU."""
import ctypes
import os
import re

import numpy as np
import pytest
import torch

import oracle as O
import q35
from q35 import _lib as L

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "q35.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(q35_[a-z0-9_]+)\s*\(", text)))


def test_exports_every_declared_symbol():
    names = declared_functions()
    assert len(names) >= 25
    lib = ctypes.CDLL(L.LIB_PATH)
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    # and the Python binding covers the whole header
    assert set(names) <= set(L.PROTOTYPES), set(names) - set(L.PROTOTYPES)


def test_dims_2b():
    d = q35.dims_2b()
    assert (d.hidden, d.ffn, d.vocab, d.n_layers, d.full_interval) == (2048, 6144, 248320, 24, 4)
    assert (d.lin_heads, d.lin_dk, d.lin_dv, d.conv_k) == (16, 128, 128, 4)
    assert (d.attn_heads, d.kv_heads, d.head_dim, d.rot_dim) == (8, 2, 256, 64)
    assert d.eps == np.float32(1e-6) and d.theta == np.float32(1e7)


def test_synth_normal_statistics_and_slicing():
    a = q35.synth_normal(0, 7, 200001, 1.0)
    assert abs(a.mean()) < 0.01 and abs(a.std() - 1.0) < 0.01
    # any slice regenerates the same values (counter-based generator)
    b = q35.synth_normal(0, 7, 1001, 1.0, offset=99999)
    np.testing.assert_array_equal(a[99999:101000], b)
    # different stream / seed -> different values
    assert not np.array_equal(a[:100], q35.synth_normal(0, 8, 100)[:100])
    assert not np.array_equal(a[:100], q35.synth_normal(1, 7, 100)[:100])
    s = q35.synth_normal(0, 7, 1000, 0.02)
    np.testing.assert_allclose(s, (a[:1000].astype(np.float64) * 0.02).astype(np.float32), rtol=1e-6)


def test_synth_uniform():
    u = q35.synth_uniform(3, 1, 100000, 0.01, 16.0)
    assert u.min() > 0.01 and u.max() < 16.0 and abs(u.mean() - 8.005) < 0.1


@pytest.mark.parametrize("rows,cols", [(1, 64), (7, 192), (300, 2048)])
def test_product_quantizer_matches_oracle(rows, cols, rng):
    w = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    w[0, :64] = 0
    if rows > 1:
        w[1, 64 % cols:] *= 1e-30  # tiny (denormal-range) blocks
    q, s = q35.quantize_q8f(w)
    W = O.quantize(w)
    np.testing.assert_array_equal(q, W.q)
    np.testing.assert_array_equal(s, W.s)


def test_synth_model_tensor_init_rules():
    d = q35.make_dims(hidden=256, ffn=512, vocab=1000, n_layers=4, lin_heads=4, attn_heads=4, kv_heads=2)
    z = q35.synth_model_tensor(d, 0, "layers.0.input_layernorm", 256)
    assert np.all(z == 0)
    assert np.all(q35.synth_model_tensor(d, 0, "layers.0.linear_attn.dt_bias", 4) == 1)
    assert np.all(q35.synth_model_tensor(d, 0, "layers.0.linear_attn.norm", 128) == 1)
    al = q35.synth_model_tensor(d, 0, "layers.1.linear_attn.a_log", 4)
    assert np.all(al > np.log(0.01)) and np.all(al < np.log(16.0))
    w = q35.synth_model_tensor(d, 0, "layers.3.self_attn.q_proj", 256 * 4 * 256 * 2)
    assert abs(w.std() - 0.02) < 0.001
    sid = L.lib().q35_synth_stream_id(b"layers.3.self_attn.q_proj")
    np.testing.assert_array_equal(w, q35.synth_normal(0, sid, w.size, 0.02))
    with pytest.raises(q35.Q35Error):
        q35.synth_model_tensor(d, 0, "layers.3.linear_attn.in_proj_qkv", 10)  # layer 3 is full attention
    with pytest.raises(q35.Q35Error):
        q35.synth_model_tensor(d, 0, "embed_tokens", 5)


def test_rope_tables_match_oracle():
    d = q35.dims_2b()
    c, s = q35.rope_tables(d, 4096)
    for pos in (0, 1, 511, 4095):
        oc, os_ = O.rope_cos_sin(pos, 64, 1e7)
        np.testing.assert_array_equal(c[pos], oc)
        np.testing.assert_array_equal(s[pos], os_)


def test_argument_validation_without_gpu():
    lib = L.lib()
    x = ctypes.c_void_p(16)
    bad = L.Q8F(16, 16, 64, 100, L.Q35_KN)  # cols not a multiple of 64
    assert lib.q35_q8_gemv(x, 1, bad, x, x, 1 << 20, None) == L.Q35_E_SHAPE
    assert b"multiple of 64" in lib.q35_last_error()
    assert lib.q35_q8_gemv(x, 1, L.Q8F(None, 16, 64, 64, L.Q35_KN), x, x, 1 << 20, None) == L.Q35_E_ARG
    assert lib.q35_q8_gemv(x, 1, L.Q8F(17, 16, 64, 64, L.Q35_KN), x, x, 1 << 20, None) == L.Q35_E_ALIGN
    assert lib.q35_q8_gemv(x, 0, L.Q8F(16, 16, 64, 64, L.Q35_KN), x, x, 1 << 20, None) == L.Q35_E_SHAPE
    assert lib.q35_q8_gemv(x, 1, L.Q8F(16, 16, 64, 64, 7), x, x, 1 << 20, None) == L.Q35_E_ARG
    assert lib.q35_q8_gemv(x, 1, L.Q8F(16, 16, 64, 64, L.Q35_KN), x, x, 16, None) == L.Q35_E_WS
    assert lib.q35_q8_lm_head(x, 1, L.Q8F(16, 16, 64, 64, L.Q35_KN), x, None) == L.Q35_E_ARG
    d = q35.make_dims(head_dim=128)
    assert lib.q35_layer_ws_bytes(ctypes.byref(q35.dims_2b()), 1, 1024) > 0
    h = ctypes.c_void_p()
    assert lib.q35_model_create_synthetic(ctypes.byref(d), 0, 16, ctypes.byref(h)) == L.Q35_E_SHAPE
    assert lib.q35_gate_proj(x, 1, 64, x, x, x, x, 48, x, None) == L.Q35_E_SHAPE  # 2*48 does not divide 256


@pytest.mark.parametrize("K,N", [(3, 64), (5, 256), (2, 320), (7, 704)])
def test_pack_kn_tiled_layout(K, N):
    """Q35_KN -> Q35_KN_TILED: element (k, n) lands at [n // 256][k][n % 256], scale block b at
    [b // 4][k][b % 4]; the tile's columns past N are zero."""
    rng = np.random.default_rng(K * 1000 + N)
    q = rng.integers(-127, 128, size=(K, N), dtype=np.int8)
    s = rng.random((K, N // 64), dtype=np.float32) + 0.5
    t = q35.Q8FTensor(torch.from_numpy(q), torch.from_numpy(s), q35.Q35_KN).tiled()
    assert t.layout == q35.Q35_KN_TILED and t.shape == (K, N) and t.in_dim == K and t.out_dim == N
    qt, st = t.q.numpy(), t.scale.numpy()
    nt = (N + 255) // 256
    assert qt.shape == (nt, K, 256) and st.shape == (nt, K, 4)
    for n in range(N):
        np.testing.assert_array_equal(qt[n // 256, :, n % 256], q[:, n])
    for b in range(N // 64):
        np.testing.assert_array_equal(st[b // 4, :, b % 4], s[:, b])
    assert not qt[nt - 1, :, N - (nt - 1) * 256:].any()
    assert not st[nt - 1, :, N // 64 - (nt - 1) * 4:].any()
