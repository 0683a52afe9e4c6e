"""Pinning of the oracle's module-level functions (text_modules.rs restatements) on the CPU:
closed forms in numpy float64, special cases that reduce to a textbook result, and
cross-algorithm identities (chunked delta rule == sequential recurrent steps)."""
import zlib

import numpy as np
import pytest

import oracle as O
from conftest import rel_l2


def silu(v):
    return v / (1 + np.exp(-v))


def test_rmsnorm_closed_form(rng):
    x = rng.standard_normal(2048).astype(np.float32) * 3
    w = rng.standard_normal(2048).astype(np.float32) * 0.1
    out = O.rmsnorm(x, w)
    xd = x.astype(np.float64)
    ref = xd / np.sqrt(np.mean(xd * xd) + 1e-6) * (1 + w)
    np.testing.assert_allclose(out, ref, rtol=2e-6, atol=1e-7)
    # w = 0 (the reference init) gives unit RMS
    y = O.rmsnorm(x, np.zeros_like(w)).astype(np.float64)
    assert abs(np.sqrt(np.mean(y * y)) - 1.0) < 1e-5


def test_rmsnorm_gated_closed_form(rng):
    x = rng.standard_normal(128).astype(np.float32)
    z = rng.standard_normal(128).astype(np.float32)
    w = rng.uniform(0.5, 1.5, 128).astype(np.float32)
    out = O.rmsnorm_gated(x, z, w)
    xd = x.astype(np.float64)
    ref = w * (xd / np.sqrt(np.mean(xd * xd) + 1e-6)) * silu(z.astype(np.float64))
    np.testing.assert_allclose(out, ref, rtol=3e-6, atol=1e-7)


def test_l2norm(rng):
    x = rng.standard_normal(128).astype(np.float32)
    y = O.l2norm(x).astype(np.float64)
    assert abs(np.linalg.norm(y) - 1) < 1e-6
    np.testing.assert_allclose(y, x / np.sqrt(np.sum(x.astype(np.float64) ** 2) + 1e-6), rtol=1e-6)


def test_conv_update_one_hot_taps(rng):
    C, k = 8, 4
    x = rng.standard_normal(C).astype(np.float32)
    st = rng.standard_normal((C, k - 1)).astype(np.float32)
    xcat = np.concatenate([st, x[:, None]], axis=1)
    for j in range(k):
        w = np.zeros((C, k), np.float32)
        w[:, j] = 1.0
        out, new = O.conv_update(x, st, w)
        np.testing.assert_allclose(out, silu(xcat[:, j].astype(np.float64)), rtol=1e-6)
        np.testing.assert_array_equal(new, xcat[:, 1:])
    w = rng.standard_normal((C, k)).astype(np.float32)
    out, _ = O.conv_update(x, st, w)
    np.testing.assert_allclose(out, silu(np.sum(w.astype(np.float64) * xcat, axis=1)), rtol=1e-6)


def delta_step_np(q, k, v, g, beta, S):
    """numpy float64 delta rule written from the update equations."""
    H, dk = q.shape
    out = np.zeros_like(v, dtype=np.float64)
    S = S.astype(np.float64).copy()
    for h in range(H):
        qh = q[h] / np.sqrt(np.sum(q[h].astype(np.float64) ** 2) + 1e-6) / np.sqrt(dk)
        kh = k[h] / np.sqrt(np.sum(k[h].astype(np.float64) ** 2) + 1e-6)
        Sd = S[h] * np.exp(g[h])
        delta = (v[h] - kh @ Sd) * beta[h]
        S[h] = Sd + np.outer(kh, delta)
        out[h] = qh @ S[h]
    return out, S


def test_delta_step_vs_numpy(rng):
    H, dk, dv = 4, 128, 128
    q, k = rng.standard_normal((2, H, dk)).astype(np.float32)
    v = rng.standard_normal((H, dv)).astype(np.float32)
    g = -np.log1p(np.exp(rng.standard_normal(H))).astype(np.float32)
    beta = (1 / (1 + np.exp(-rng.standard_normal(H)))).astype(np.float32)
    S = (rng.standard_normal((H, dk, dv)) * 0.1).astype(np.float32)
    out, S2 = O.gated_delta_step(q, k, v, g, beta, S)
    ro, rS = delta_step_np(q, k, v, g, beta, S)
    assert rel_l2(out, ro) < 1e-6
    assert rel_l2(S2, rS) < 1e-6


def test_delta_step_special_cases(rng):
    H, dk, dv = 2, 128, 128
    q, k = rng.standard_normal((2, H, dk)).astype(np.float32)
    v = rng.standard_normal((H, dv)).astype(np.float32)
    S = rng.standard_normal((H, dk, dv)).astype(np.float32)
    g = np.array([-0.3, -1.2], np.float32)
    # beta = 0: pure decay
    _, S2 = O.gated_delta_step(q, k, v, g, np.zeros(H, np.float32), S)
    np.testing.assert_allclose(S2, S * np.exp(g)[:, None, None], rtol=1e-6)
    # full decay and beta = 1: state becomes k_hat (outer) v
    _, S3 = O.gated_delta_step(q, k, v, np.full(H, -1e4, np.float32), np.ones(H, np.float32), S)
    kh = k / np.linalg.norm(k.astype(np.float64), axis=1, keepdims=True)
    np.testing.assert_allclose(S3, np.einsum("hi,hj->hij", kh, v), rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("T,chunk", [(1, 64), (5, 4), (100, 64), (130, 64)])
def test_chunked_equals_recurrent(T, chunk, rng):
    H, dk, dv = 2, 128, 128
    q = rng.standard_normal((T, H, dk)).astype(np.float32)
    k = rng.standard_normal((T, H, dk)).astype(np.float32)
    v = rng.standard_normal((T, H, dv)).astype(np.float32)
    g = -np.log1p(np.exp(rng.standard_normal((T, H)))).astype(np.float32)
    beta = (1 / (1 + np.exp(-rng.standard_normal((T, H))))).astype(np.float32)
    S0 = (rng.standard_normal((H, dk, dv)) * 0.1).astype(np.float32)
    out_c, S_c = O.gated_delta_chunked(q, k, v, g, beta, S0, chunk)
    S = S0.copy()
    outs = []
    for t in range(T):
        o, S = O.gated_delta_step(q[t], k[t], v[t], g[t], beta[t], S)
        outs.append(o)
    assert rel_l2(out_c, np.stack(outs)) < 1e-5
    assert rel_l2(S_c, S) < 1e-5


def test_rope_properties(rng):
    c0, s0 = O.rope_cos_sin(0)
    assert np.all(c0 == 1.0) and np.all(s0 == 0.0)
    x = rng.standard_normal(256).astype(np.float32)
    np.testing.assert_array_equal(O.apply_rope(x, c0, s0), x)
    for pos in (1, 17, 1000, 32767):
        c, s = O.rope_cos_sin(pos)
        y = O.apply_rope(x, c, s)
        np.testing.assert_array_equal(y[64:], x[64:])
        # complex rotation of (x_i, x_{i+32}) by angle pos * theta^(-2i/64)
        # f32 exponent as the reference builds it, exp rounded once to f32 (glibc expf is
        # correctly rounded; numpy's float32 exp is not always)
        sf = np.float32(-np.log(np.float64(np.float32(1e7)))).astype(np.float32) / np.float32(64.0)
        inv = np.exp((np.float32(2) * np.arange(32, dtype=np.float32) * sf).astype(np.float64)).astype(np.float32)
        ang = np.float32(pos) * inv
        z = (x[:32] + 1j * x[32:64]) * np.exp(1j * ang.astype(np.float64))
        np.testing.assert_allclose(y[:32], z.real, rtol=1e-5, atol=1e-5)
        np.testing.assert_allclose(y[32:64], z.imag, rtol=1e-5, atol=1e-5)
        np.testing.assert_allclose(np.hypot(y[:32], y[32:64]), np.hypot(x[:32], x[32:64]), rtol=1e-5)


def test_attention_core(rng):
    nh, nkv, d, tmax = 8, 2, 256, 64
    q = rng.standard_normal((nh, d)).astype(np.float32)
    kc = rng.standard_normal((nkv, tmax, d)).astype(np.float32)
    vc = rng.standard_normal((nkv, tmax, d)).astype(np.float32)
    # T = 1: softmax over one token -> the mapped kv head's value row
    out = O.attention_core(q, kc, vc, 1)
    for h in range(nh):
        np.testing.assert_allclose(out[h], vc[h // 4, 0], rtol=1e-6)
    # constant keys -> uniform weights -> mean of V
    kconst = np.repeat(kc[:, :1], tmax, axis=1)
    out = O.attention_core(q, kconst, vc, 40)
    for h in range(nh):
        np.testing.assert_allclose(out[h], vc[h // 4, :40].astype(np.float64).mean(0), rtol=1e-5, atol=1e-6)
    # general: float64 softmax with GQA map h -> h // (nh / nkv)
    T = 50
    out = O.attention_core(q, kc, vc, T)
    for h in range(nh):
        g = h // (nh // nkv)
        s = kc[g, :T].astype(np.float64) @ q[h] / 16.0
        p = np.exp(s - s.max())
        p /= p.sum()
        np.testing.assert_allclose(out[h], p @ vc[g, :T], rtol=1e-5, atol=1e-6)


def _mk_gdn(rng, H=256, nh=4, dk=128, dv=128):
    conv_dim = 2 * nh * dk + nh * dv
    W = lambda r, c: O.quantize(rng.standard_normal((r, c)).astype(np.float32) * 0.05)
    layer = O.GdnLayer(W(H, conv_dim), W(H, nh * dv), W(nh * dv, H),
                       rng.standard_normal((H, nh)).astype(np.float32) * 0.05,
                       rng.standard_normal((H, nh)).astype(np.float32) * 0.05,
                       np.log(rng.uniform(0.01, 16, nh)).astype(np.float32), np.ones(nh, np.float32),
                       rng.standard_normal((conv_dim, 4)).astype(np.float32) * 0.5,
                       rng.uniform(0.5, 1.5, dv).astype(np.float32))
    return layer, conv_dim


def test_gdn_layer_wiring(rng):
    """orc_gdn_decode == the pinned pieces composed in the reference's order (text_modules.rs:484-667)."""
    H, nh, dk, dv = 256, 4, 128, 128
    cfg = O.Cfg(hidden=H, ffn=512, vocab=1000, n_layers=1, full_interval=4, lin_heads=nh, lin_dk=dk, lin_dv=dv,
                conv_k=4, attn_heads=8, kv_heads=2, head_dim=256, rot_dim=64, eps=1e-6, theta=1e7)
    layer, conv_dim = _mk_gdn(rng, H, nh, dk, dv)
    qkvW, zW, outW, wb, wa, alog, dtb, cw, nw = layer.keep
    x = rng.standard_normal((1, H)).astype(np.float32)
    cs = rng.standard_normal((1, conv_dim, 3)).astype(np.float32)
    S = (rng.standard_normal((1, nh, dk, dv)) * 0.1).astype(np.float32)
    cs_ref, S_ref = cs[0].copy(), S[0].copy()
    out = O.gdn_decode(cfg, layer, x, cs, S)
    mixed = O.gemv_kn(x, qkvW)[0]
    z = O.gemv_kn(x, zW)[0]
    conv, cs_ref = O.conv_update(mixed, cs_ref, cw)
    bg = O.gate_proj(x[0], wb, wa, alog, dtb)
    kd = nh * dk
    core, S_ref = O.gated_delta_step(conv[:kd].reshape(nh, dk), conv[kd:2 * kd].reshape(nh, dk),
                                     conv[2 * kd:].reshape(nh, dv), bg[nh:], bg[:nh], S_ref)
    normed = np.concatenate([O.rmsnorm_gated(core[h], z[h * dv:(h + 1) * dv], nw) for h in range(nh)])
    ref = O.gemv_kn(normed, outW)[0]
    np.testing.assert_allclose(out[0], ref, rtol=1e-6, atol=1e-7)
    np.testing.assert_array_equal(cs[0], cs_ref)
    np.testing.assert_allclose(S[0], S_ref, rtol=1e-6, atol=1e-7)


def test_attn_layer_wiring(rng):
    """orc_attn_decode == pinned pieces in the order of text_modules.rs:842-944, incl. the
    per-head [query | gate] split of q_proj and the post-RoPE key append."""
    H, nh, nkv, d, tmax = 256, 8, 2, 256, 16
    cfg = O.Cfg(hidden=H, ffn=512, vocab=1000, n_layers=1, full_interval=1, lin_heads=4, lin_dk=128, lin_dv=128,
                conv_k=4, attn_heads=nh, kv_heads=nkv, head_dim=d, rot_dim=64, eps=1e-6, theta=1e7)
    W = lambda r, c: O.quantize(rng.standard_normal((r, c)).astype(np.float32) * 0.05)
    qn = rng.standard_normal(d).astype(np.float32) * 0.1
    kn = rng.standard_normal(d).astype(np.float32) * 0.1
    layer = O.AttnLayer(W(H, nh * d * 2), W(H, nkv * d), W(H, nkv * d), W(nh * d, H), qn, kn)
    qW, kW, vW, oW = layer.keep[:4]
    x = rng.standard_normal((1, H)).astype(np.float32)
    pos = 5
    kc = rng.standard_normal((1, nkv, tmax, d)).astype(np.float32)
    vc = rng.standard_normal((1, nkv, tmax, d)).astype(np.float32)
    kc0, vc0 = kc[0].copy(), vc[0].copy()
    out = O.attn_decode(cfg, layer, x, kc, vc, [pos])
    qg = O.gemv_kn(x, qW)[0].reshape(nh, 2 * d)
    c, s = O.rope_cos_sin(pos)
    q = np.stack([O.apply_rope(O.rmsnorm(qg[h, :d], qn), c, s) for h in range(nh)])
    gate = qg[:, d:].reshape(-1)
    k = O.gemv_kn(x, kW)[0].reshape(nkv, d)
    k = np.stack([O.apply_rope(O.rmsnorm(k[h], kn), c, s) for h in range(nkv)])
    v = O.gemv_kn(x, vW)[0].reshape(nkv, d)
    kc0[:, pos] = k
    vc0[:, pos] = v
    att = O.attention_core(q, kc0, vc0, pos + 1).reshape(-1)
    att = att * (1 / (1 + np.exp(-gate.astype(np.float64))))
    ref = O.gemv_kn(att.astype(np.float32), oW)[0]
    np.testing.assert_allclose(out[0], ref, rtol=1e-5, atol=1e-6)
    np.testing.assert_array_equal(kc[0], kc0)
    np.testing.assert_array_equal(vc[0], vc0)


def test_model_step_wiring():
    """orc_model_step == the pinned layer forwards composed as model.rs:27-84,113-129 and
    text_modules.rs:1053-1085 write it: h = embed(token); per layer h += mixer(RMSNorm(h)),
    h += MLP(RMSNorm(h)); logits = tied lm_head(RMSNorm(h)); token = argmax.  Two linear layers
    and one full-attention layer (full_interval 3), three consecutive tokens."""
    H, F, V, nh, dk, dv = 256, 512, 640, 2, 128, 128
    cfg = O.Cfg(hidden=H, ffn=F, vocab=V, n_layers=3, full_interval=3, lin_heads=nh, lin_dk=dk, lin_dv=dv,
                conv_k=4, attn_heads=4, kv_heads=2, head_dim=256, rot_dim=64, eps=1e-6, theta=1e7)
    tmax = 8
    vals = {}

    def get(name, n):
        if name not in vals:
            g = np.random.default_rng(zlib.crc32(name.encode()))
            if name.endswith("norm") and "linear_attn" not in name:
                v = g.standard_normal(n) * 0.1          # RMSNorm weights (applied as 1 + w)
            elif name.endswith("linear_attn.norm"):
                v = g.uniform(0.5, 1.5, n)
            elif name.endswith("a_log"):
                v = np.log(g.uniform(0.01, 16, n))
            elif name.endswith("dt_bias"):
                v = np.ones(n)
            else:
                v = g.standard_normal(n) * 0.05
            vals[name] = v.astype(np.float32)
        return vals[name]

    m = O.Model(cfg, get, tmax)
    conv_dim = 2 * nh * dk + nh * dv
    q8 = lambda name, r, c: O.quantize(get(name, r * c).reshape(r, c))
    E = q8("embed_tokens", V, H)
    layers, states = [], []
    for l in range(3):
        p = f"layers.{l}."
        if (l + 1) % 3:
            a = p + "linear_attn."
            layers.append(O.GdnLayer(q8(a + "in_proj_qkv", H, conv_dim), q8(a + "in_proj_z", H, nh * dv),
                                     q8(a + "out_proj", nh * dv, H), get(a + "in_proj_b", H * nh).reshape(H, nh),
                                     get(a + "in_proj_a", H * nh).reshape(H, nh), get(a + "a_log", nh),
                                     get(a + "dt_bias", nh), get(a + "conv1d", conv_dim * 4).reshape(conv_dim, 4),
                                     get(a + "norm", dv)))
            states.append([np.zeros((1, conv_dim, 3), np.float32), np.zeros((1, nh, dk, dv), np.float32)])
        else:
            a = p + "self_attn."
            layers.append(O.AttnLayer(q8(a + "q_proj", H, 4 * 256 * 2), q8(a + "k_proj", H, 2 * 256),
                                      q8(a + "v_proj", H, 2 * 256), q8(a + "o_proj", 4 * 256, H),
                                      get(a + "q_norm", 256), get(a + "k_norm", 256)))
            states.append([np.zeros((1, 2, tmax, 256), np.float32), np.zeros((1, 2, tmax, 256), np.float32)])
    mlps = [O.MlpLayer(q8(f"layers.{l}.mlp.gate_proj", H, F), q8(f"layers.{l}.mlp.up_proj", H, F),
                       q8(f"layers.{l}.mlp.down_proj", F, H)) for l in range(3)]
    tok = 17
    for pos in range(3):
        got, _, logits = m.step(tok, want_logits=True)
        h = O.embedding(E, [tok])[0].astype(np.float32)
        for l in range(3):
            x = O.rmsnorm(h, get(f"layers.{l}.input_layernorm", H))[None]
            if (l + 1) % 3:
                mix = O.gdn_decode(cfg, layers[l], x, states[l][0], states[l][1])[0]
            else:
                mix = O.attn_decode(cfg, layers[l], x, states[l][0], states[l][1], [pos])[0]
            h = (h + mix).astype(np.float32)
            x2 = O.rmsnorm(h, get(f"layers.{l}.post_attention_layernorm", H))[None]
            h = (h + O.mlp_decode(cfg, mlps[l], x2)[0]).astype(np.float32)
        ref, _ = O.gemv_nk(O.rmsnorm(h, get("norm", H))[None], E)
        np.testing.assert_allclose(logits, ref[0], rtol=1e-5, atol=1e-6)
        assert got == O.argmax(ref[0])
        tok = got


@pytest.mark.parametrize("B", [1, 3])
def test_mlp_decode_closed_form(B, rng):
    """orc_mlp_decode == down(silu(x Wg) * (x Wu)) (text_modules.rs:1000-1011) in numpy float64
    from the dequantised weights.  Gate and up are drawn with different scales and a shifted
    gate, so swapping them or putting the SiLU on `up` moves the result far outside the bar
    (checked below on the same data)."""
    H, F = 256, 384
    cfg = O.Cfg(hidden=H, ffn=F, vocab=1000, n_layers=1, full_interval=4, lin_heads=2, lin_dk=128, lin_dv=128,
                conv_k=4, attn_heads=8, kv_heads=2, head_dim=256, rot_dim=64, eps=1e-6, theta=1e7)
    Wg = O.quantize((rng.standard_normal((H, F)) * 0.08 + 0.01).astype(np.float32))
    Wu = O.quantize((rng.standard_normal((H, F)) * 0.03).astype(np.float32))
    Wd = O.quantize((rng.standard_normal((F, H)) * 0.05).astype(np.float32))
    x = rng.standard_normal((B, H)).astype(np.float32)
    out = O.mlp_decode(cfg, O.MlpLayer(Wg, Wu, Wd), x)
    xd = x.astype(np.float64)
    g, u = xd @ Wg.dequant(), xd @ Wu.dequant()
    ref = (u * silu(g)) @ Wd.dequant()
    assert out.shape == (B, H)
    assert rel_l2(out, ref) <= 1e-5
    # the plausible mistakes are far outside that bar on these inputs
    assert rel_l2((g * silu(u)) @ Wd.dequant(), ref) > 0.1      # gate and up swapped
    assert rel_l2((silu(u) * silu(g)) @ Wd.dequant(), ref) > 0.1  # SiLU on both
    assert rel_l2((u * g) @ Wd.dequant(), ref) > 0.1            # SiLU dropped


def test_mlp_decode_gate_closed():
    """Known answer: a gate row pushing every gate pre-activation to -60 makes silu(gate) ~ 0
    (|silu(-60)| < 6e-25), so the output vanishes whatever `up` holds; with the roles swapped
    it would not."""
    H, F = 128, 256
    cfg = O.Cfg(hidden=H, ffn=F, vocab=1000, n_layers=1, full_interval=4, lin_heads=2, lin_dk=128, lin_dv=128,
                conv_k=4, attn_heads=8, kv_heads=2, head_dim=256, rot_dim=64, eps=1e-6, theta=1e7)
    x = np.zeros((1, H), np.float32)
    x[0, 0] = 1.0
    wg = np.zeros((H, F), np.float32)
    wg[0, :] = -60.0
    wu = np.full((H, F), 0.5, np.float32)
    wd = np.full((F, H), 0.25, np.float32)
    out = O.mlp_decode(cfg, O.MlpLayer(O.quantize(wg), O.quantize(wu), O.quantize(wd)), x)
    assert np.max(np.abs(out)) < 1e-20
    swapped = O.mlp_decode(cfg, O.MlpLayer(O.quantize(wu), O.quantize(wg), O.quantize(wd)), x)
    assert np.max(np.abs(swapped)) > 1.0
