"""GPU parity of the layer-level entry points (text_modules.rs surface) against the oracle.
Tolerances: rel-L2 <= 1e-5 for outputs, <= 1e-4 for the DeltaNet recurrent state; the conv state
and the KV-cache rows are copies and must match bit for bit (KV rows: post-RoPE k to 1e-6)."""
import numpy as np
import pytest
import torch

import oracle as O
import q35
from conftest import rel_l2
from gpu_util import dev, host, normal, q8, q8_dev
from q35._lib import Q35_E_RANGE

pytestmark = pytest.mark.gpu


def softplus(x):
    return np.log1p(np.exp(x))


@pytest.mark.parametrize("fused", [True, False])
@pytest.mark.parametrize("B", [1, 32])
def test_gated_delta_rule_decode_c2(B, fused):
    """C2: 16 heads, dk = dv = 128, S ~ N(0, 0.1), beta = sigmoid(N(0,1)), decay = exp(-softplus(N(0,1))).
    fused: the conv state is advanced by the step kernel's last block of each head (with a
    workspace) or by a second kernel (without)."""
    print(f"[delta rule] B={B} fused={fused}", flush=True)
    nh, dk, dv = 16, 128, 128
    conv_dim = 2 * nh * dk + nh * dv
    S0 = normal(30, (B, nh, dk, dv), 0.1)
    cs0 = normal(31, (B, conv_dim, 3))
    cw = normal(32, (conv_dim, 4), 0.02)
    S_d, cs_d = dev(S0), dev(cs0)
    S_h, cs_h = S0.copy(), cs0.copy()
    for step in range(3):
        mixed = normal(33 + step, (B, conv_dim))
        beta = (1 / (1 + np.exp(-normal(40 + step, (B, nh)).astype(np.float64)))).astype(np.float32)
        g = (-softplus(normal(50 + step, (B, nh)).astype(np.float64))).astype(np.float32)
        bg = np.concatenate([beta, g], axis=1)
        out = host(q35.gated_delta_rule_decode(dev(mixed), dev(bg), cs_d, dev(cw), S_d, nh, dk, dv, fused=fused))
        kd = nh * dk
        for b in range(B):
            conv, cs_h[b] = O.conv_update(mixed[b], cs_h[b], cw)
            ref, S_h[b] = O.gated_delta_step(conv[:kd].reshape(nh, dk), conv[kd:2 * kd].reshape(nh, dk),
                                             conv[2 * kd:].reshape(nh, dv), g[b], beta[b], S_h[b])
            assert rel_l2(out[b], ref.reshape(-1)) <= 1e-5, (step, b)
        np.testing.assert_array_equal(host(cs_d), cs_h)
        assert rel_l2(host(S_d), S_h) <= 1e-4


def _gdn_module(d, seed=0):
    H, nh, dk, dv = d.hidden, d.lin_heads, d.lin_dk, d.lin_dv
    conv_dim = 2 * nh * dk + nh * dv
    Wqkv, Wz, Wo = q8(60, H, conv_dim), q8(61, H, nh * dv), q8(62, nh * dv, H)
    wb, wa = normal(63, (H, nh), 0.02), normal(64, (H, nh), 0.02)
    a_log = np.log(q35.synth_uniform(0, 65, nh, 0.01, 16.0)).astype(np.float32)
    dtb = np.ones(nh, np.float32)
    cw = normal(66, (conv_dim, 4), 0.5)
    nw = (1.0 + normal(67, (dv,), 0.1)).astype(np.float32)
    gpu = q35.GatedDeltaNet(d, q8_dev(Wqkv, q35.Q35_KN), q8_dev(Wz, q35.Q35_KN), q8_dev(Wo, q35.Q35_KN), dev(wb),
                            dev(wa), dev(a_log), dev(dtb), dev(cw), dev(nw))
    ref = O.GdnLayer(Wqkv, Wz, Wo, wb, wa, a_log, dtb, cw, nw)
    return gpu, ref, conv_dim


@pytest.mark.parametrize("B", [1, 3, 9])
def test_gated_deltanet_module(B):
    print(f"[gdn module] B={B}", flush=True)
    d = q35.dims_2b()
    cfg = O.cfg_from_dims(d)
    gpu, ref, conv_dim = _gdn_module(d)
    S0 = normal(68, (B, d.lin_heads, 128, 128), 0.1)
    cs0 = normal(69, (B, conv_dim, 3))
    S_d, cs_d = dev(S0), dev(cs0)
    S_h, cs_h = S0.copy(), cs0.copy()
    for step in range(2):
        x = normal(70 + step, (B, d.hidden))
        out = host(gpu.forward(dev(x), cs_d, S_d))
        exp = O.gdn_decode(cfg, ref, x, cs_h, S_h)
        assert rel_l2(out, exp) <= 1e-5, step
        # the conv state holds in_proj_qkv outputs (f32-accumulated matvec), not exact copies
        assert rel_l2(host(cs_d), cs_h) <= 1e-5
        assert rel_l2(host(S_d), S_h) <= 1e-4


@pytest.mark.parametrize("B,T", [(1, 1), (1, 1024), (1, 8192), (1, 32768), (16, 1024), (16, 8192), (16, 32768)])
def test_attention_core_decode_c3(B, T):
    """C3: 8 q heads, 2 kv heads, head_dim 256, partial RoPE 64 (theta 1e7), q/k RMSNorm,
    KV cache ~ N(0,1), sigmoid gate; the new token goes to position T-1."""
    print(f"[attention core] B={B} T={T}", flush=True)
    d = q35.dims_2b()
    nh, nkv, hd = d.attn_heads, d.kv_heads, d.head_dim
    tmax = T
    rng = np.random.default_rng(T * 31 + B)
    kc = rng.standard_normal((B, nkv, tmax, hd), dtype=np.float32)
    vc = rng.standard_normal((B, nkv, tmax, hd), dtype=np.float32)
    qg = normal(80, (B, nh * 2 * hd))
    kn, vn = normal(81, (B, nkv * hd)), normal(82, (B, nkv * hd))
    qw, kw = normal(83, (hd,), 0.1), normal(84, (hd,), 0.1)
    pos = np.full(B, T - 1, np.int32)
    cs, sn = q35.rope_tables(d, tmax)
    kc_d, vc_d = dev(kc), dev(vc)
    out = host(q35.attention_core_decode(d, dev(qg), dev(kn), dev(vn), dev(qw), dev(kw), kc_d, vc_d, dev(pos),
                                         dev(cs), dev(sn)))
    c, s = O.rope_cos_sin(T - 1)
    for b in range(B):
        q = np.stack([O.apply_rope(O.rmsnorm(qg[b, h * 2 * hd:h * 2 * hd + hd], qw), c, s) for h in range(nh)])
        k = np.stack([O.apply_rope(O.rmsnorm(kn[b, h * hd:(h + 1) * hd], kw), c, s) for h in range(nkv)])
        kc[b, :, T - 1] = k
        vc[b, :, T - 1] = vn[b].reshape(nkv, hd)
        att = O.attention_core(q, kc[b], vc[b], T).astype(np.float64).reshape(-1)
        gate = qg[b].reshape(nh, 2 * hd)[:, hd:].reshape(-1).astype(np.float64)
        ref = att / (1 + np.exp(-gate))
        assert rel_l2(out[b], ref) <= 1e-5, b
    kc_g = host(kc_d)
    np.testing.assert_allclose(kc_g[:, :, T - 1], kc[:, :, T - 1], rtol=1e-6, atol=1e-6)
    np.testing.assert_array_equal(host(vc_d)[:, :, T - 1], vc[:, :, T - 1])
    if T > 1:
        np.testing.assert_array_equal(kc_g[:, :, :T - 1], kc[:, :, :T - 1])


def test_attention_module_ragged_positions():
    d = q35.dims_2b()
    cfg = O.cfg_from_dims(d)
    H, nh, nkv, hd = d.hidden, d.attn_heads, d.kv_heads, d.head_dim
    Wq, Wk, Wv, Wo = q8(90, H, nh * hd * 2), q8(91, H, nkv * hd), q8(92, H, nkv * hd), q8(93, nh * hd, H)
    qw, kw = normal(94, (hd,), 0.1), normal(95, (hd,), 0.1)
    gpu = q35.Attention(d, *(q8_dev(W, q35.Q35_KN) for W in (Wq, Wk, Wv, Wo)), dev(qw), dev(kw))
    ref = O.AttnLayer(Wq, Wk, Wv, Wo, qw, kw)
    B, tmax = 4, 300
    pos = np.array([0, 17, 255, 299], np.int32)
    kc = normal(96, (B, nkv, tmax, hd))
    vc = normal(97, (B, nkv, tmax, hd))
    cs, sn = q35.rope_tables(d, tmax)
    x = normal(98, (B, H))
    kc_d, vc_d = dev(kc), dev(vc)
    out = host(gpu.forward(dev(x), kc_d, vc_d, dev(pos), dev(cs), dev(sn)))
    exp = O.attn_decode(cfg, ref, x, kc, vc, pos)
    assert rel_l2(out, exp) <= 1e-5
    # appended rows are k_proj / v_proj outputs (f32-accumulated); the other rows are untouched
    kc_g, vc_g = host(kc_d), host(vc_d)
    assert rel_l2(kc_g, kc) <= 1e-5 and rel_l2(vc_g, vc) <= 1e-5
    for b, p in enumerate(pos):
        keep = np.ones(tmax, bool)
        keep[p] = False
        np.testing.assert_array_equal(kc_g[b][:, keep], kc[b][:, keep])
        np.testing.assert_array_equal(vc_g[b][:, keep], vc[b][:, keep])


@pytest.mark.parametrize("B", [1, 8, 11])
def test_mlp_module(B):
    d = q35.dims_2b()
    cfg = O.cfg_from_dims(d)
    Wg, Wu, Wd = q8(100, d.hidden, d.ffn), q8(101, d.hidden, d.ffn), q8(102, d.ffn, d.hidden)
    gpu = q35.MLP(d, q8_dev(Wg, q35.Q35_KN), q8_dev(Wu, q35.Q35_KN), q8_dev(Wd, q35.Q35_KN))
    x = normal(103, (B, d.hidden))
    out = host(gpu.forward(dev(x)))
    exp = O.mlp_decode(cfg, O.MlpLayer(Wg, Wu, Wd), x)
    assert rel_l2(out, exp) <= 1e-5


@pytest.mark.parametrize("B", [1, 11])
def test_mlp_module_tiled_weights(B):
    """The layer entry points take Q35_KN_TILED projections, as the model holds them."""
    d = q35.dims_2b()
    cfg = O.cfg_from_dims(d)
    Wg, Wu, Wd = q8(100, d.hidden, d.ffn), q8(101, d.hidden, d.ffn), q8(102, d.ffn, d.hidden)
    gpu = q35.MLP(d, *(q8_dev(W, q35.Q35_KN).tiled() for W in (Wg, Wu, Wd)))
    x = normal(103, (B, d.hidden))
    out = host(gpu.forward(dev(x)))
    exp = O.mlp_decode(cfg, O.MlpLayer(Wg, Wu, Wd), x)
    assert rel_l2(out, exp) <= 1e-5


@pytest.mark.parametrize("bad", [np.nan, np.inf, 1e12])
def test_mlp_fixed_point_range_is_reported(bad):
    """A row holding NaN / Inf, or a value whose products overflow the split-K fixed point
    (1e12 x |w| ~ 1e10 > 2^31), is caught on the device: its contributions are dropped, every
    kernel exits normally and the workspace reports Q35_E_RANGE; the word is then clear, so the
    next good call passes and matches the oracle."""
    print(f"[mlp range guard] bad={bad}", flush=True)
    d = q35.dims_2b()
    cfg = O.cfg_from_dims(d)
    Wg, Wu, Wd = q8(100, d.hidden, d.ffn), q8(101, d.hidden, d.ffn), q8(102, d.ffn, d.hidden)
    gpu = q35.MLP(d, q8_dev(Wg, q35.Q35_KN), q8_dev(Wu, q35.Q35_KN), q8_dev(Wd, q35.Q35_KN))
    x = normal(103, (3, d.hidden))
    x[1, 7] = bad
    with pytest.raises(q35.Q35Error) as ei:
        gpu.forward(dev(x), check=True)
    assert ei.value.code == Q35_E_RANGE
    good = normal(104, (2, d.hidden))
    out = host(gpu.forward(dev(good), check=True))
    assert rel_l2(out, O.mlp_decode(cfg, O.MlpLayer(Wg, Wu, Wd), good)) <= 1e-5


def test_attention_position_outside_cache_is_reported():
    """A position d_pos[b] outside [0, tmax) is caught on the device: that row's cache rows and
    output are untouched, the other rows are computed, and the workspace reports Q35_E_SHAPE
    (then clears, so the next good call passes)."""
    print("[attention position guard]", flush=True)
    d = q35.dims_2b()
    nh, nkv, hd = d.attn_heads, d.kv_heads, d.head_dim
    B, tmax = 3, 64
    rng = np.random.default_rng(5)
    kc = rng.standard_normal((B, nkv, tmax, hd), dtype=np.float32)
    vc = rng.standard_normal((B, nkv, tmax, hd), dtype=np.float32)
    qg = normal(70, (B, nh * 2 * hd))
    kn, vn = normal(71, (B, nkv * hd)), normal(72, (B, nkv * hd))
    qw, kw = normal(73, (hd,), 0.1), normal(74, (hd,), 0.1)
    cs, sn = q35.rope_tables(d, tmax)
    kc_d, vc_d = dev(kc), dev(vc)
    pos = np.array([tmax - 1, tmax, 5], np.int32)
    with pytest.raises(q35.Q35Error) as ei:
        q35.attention_core_decode(d, dev(qg), dev(kn), dev(vn), dev(qw), dev(kw), kc_d, vc_d, dev(pos), dev(cs),
                                  dev(sn), check=True)
    assert ei.value.code == q35._lib.Q35_E_SHAPE
    kc_g, vc_g = host(kc_d), host(vc_d)
    np.testing.assert_array_equal(kc_g[1], kc[1])
    np.testing.assert_array_equal(vc_g[1], vc[1])
    # the good rows went ahead: their new rows differ from the old contents
    assert not np.array_equal(kc_g[0, :, tmax - 1], kc[0, :, tmax - 1])
    assert not np.array_equal(kc_g[2, :, 5], kc[2, :, 5])
    # cleared: a call with valid positions reports nothing
    pos2 = np.array([3, 4, 5], np.int32)
    q35.attention_core_decode(d, dev(qg), dev(kn), dev(vn), dev(qw), dev(kw), kc_d, vc_d, dev(pos2), dev(cs),
                              dev(sn), check=True)
    pos3 = np.array([-1, 0, 1], np.int32)
    with pytest.raises(q35.Q35Error):
        q35.attention_core_decode(d, dev(qg), dev(kn), dev(vn), dev(qw), dev(kw), kc_d, vc_d, dev(pos3), dev(cs),
                                  dev(sn), check=True)
