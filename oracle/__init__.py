"""ctypes binding of the CPU restatement (oracle/liboracle.so) — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use this module, and
only as the checker; the product (qwen-3.5_amd/) never imports it.  Function-level pinning is
described in oracle/oracle.h and exercised by tests/test_oracle_*.py.
"""
import ctypes
import os

import numpy as np

_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_DIR, "liboracle.so")

c_i32, c_i64, c_f32, c_vp = ctypes.c_int32, ctypes.c_int64, ctypes.c_float, ctypes.c_void_p


class Q8(ctypes.Structure):
    _fields_ = [("q", c_vp), ("s", c_vp), ("rows", c_i32), ("cols", c_i32)]


class Cfg(ctypes.Structure):
    _fields_ = [(n, c_i32) for n in ("hidden", "ffn", "vocab", "n_layers", "full_interval", "lin_heads", "lin_dk",
                                     "lin_dv", "conv_k", "attn_heads", "kv_heads", "head_dim", "rot_dim")] + \
               [("eps", c_f32), ("theta", c_f32)]


class GdnW(ctypes.Structure):
    _fields_ = [("qkv", Q8), ("z", Q8), ("out", Q8), ("w_b", c_vp), ("w_a", c_vp), ("a_log", c_vp), ("dt_bias", c_vp),
                ("conv_w", c_vp), ("norm_w", c_vp)]


class AttnW(ctypes.Structure):
    _fields_ = [("q", Q8), ("k", Q8), ("v", Q8), ("o", Q8), ("q_norm", c_vp), ("k_norm", c_vp)]


class MlpW(ctypes.Structure):
    _fields_ = [("gate", Q8), ("up", Q8), ("down", Q8)]


class LayerW(ctypes.Structure):
    _fields_ = [("gdn", GdnW), ("attn", AttnW), ("mlp", MlpW), ("in_norm", c_vp), ("post_norm", c_vp)]


class ModelW(ctypes.Structure):
    _fields_ = [("embed", Q8), ("layers", ctypes.POINTER(LayerW)), ("final_norm", c_vp)]


class CacheC(ctypes.Structure):
    _fields_ = [("conv", ctypes.POINTER(c_vp)), ("rec", ctypes.POINTER(c_vp)), ("kc", ctypes.POINTER(c_vp)),
                ("vc", ctypes.POINTER(c_vp)), ("tmax", c_i32), ("pos", c_i32)]


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} missing: run `make -C oracle`")
        L = ctypes.CDLL(LIB_PATH)
        P = ctypes.POINTER
        sig = {
            "orc_quantize_q8f": (None, [c_vp, c_i64, c_i64, c_vp, c_vp]),
            "orc_q8_gemv_kn": (None, [c_vp, ctypes.c_int, Q8, c_vp, ctypes.c_int]),
            "orc_q8_gemv_nk": (None, [c_vp, ctypes.c_int, Q8, c_vp, c_vp]),
            "orc_embedding_lookup": (None, [Q8, c_vp, ctypes.c_int, c_vp]),
            "orc_gate_proj": (None, [c_vp, ctypes.c_int, c_vp, c_vp, c_vp, c_vp, ctypes.c_int, c_vp]),
            "orc_argmax": (c_i32, [c_vp, c_i64]),
            "orc_argmax_reference_order": (c_i32, [c_vp, c_i64]),
            "orc_gemv_num_splits": (ctypes.c_int, [ctypes.c_int, ctypes.c_int]),
            "orc_rmsnorm": (None, [c_vp, ctypes.c_int, c_vp, c_f32, c_vp]),
            "orc_rmsnorm_gated": (None, [c_vp, c_vp, ctypes.c_int, c_vp, c_f32, c_vp]),
            "orc_conv_update": (None, [c_vp, c_vp, c_vp, ctypes.c_int, ctypes.c_int, c_vp]),
            "orc_l2norm": (None, [c_vp, ctypes.c_int, c_f32, c_vp]),
            "orc_gated_delta_step": (None, [c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, ctypes.c_int, ctypes.c_int,
                                            ctypes.c_int, c_vp]),
            "orc_gated_delta_chunked": (None, [c_vp, c_vp, c_vp, c_vp, c_vp, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                               ctypes.c_int, ctypes.c_int, c_vp, c_vp]),
            "orc_rope_cos_sin": (None, [ctypes.c_int, ctypes.c_int, c_f32, c_vp, c_vp]),
            "orc_apply_rope": (None, [c_vp, ctypes.c_int, c_vp, c_vp]),
            "orc_attention_core": (None, [c_vp, c_vp, c_vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                          ctypes.c_int, c_vp]),
            "orc_gdn_decode": (None, [P(Cfg), P(GdnW), c_vp, ctypes.c_int, c_vp, c_vp, c_vp]),
            "orc_attn_decode": (None, [P(Cfg), P(AttnW), c_vp, ctypes.c_int, c_vp, c_vp, ctypes.c_int, c_vp, c_vp]),
            "orc_mlp_decode": (None, [P(Cfg), P(MlpW), c_vp, ctypes.c_int, c_vp]),
            "orc_model_step": (c_i32, [P(Cfg), P(ModelW), P(CacheC), c_i32, c_vp, P(ctypes.c_double)]),
            "orc_set_f32_dequant": (None, [ctypes.c_int]),
            "orc_set_threads": (None, [ctypes.c_int]),
            "orc_get_threads": (ctypes.c_int, []),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a):
    return a.ctypes.data if a is not None else None


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def cfg_from_dims(d):
    c = Cfg()
    for n, _ in Cfg._fields_:
        setattr(c, n, getattr(d, n) if not isinstance(d, dict) else d[n])
    return c


class Q8Mat:
    """Host Q8F matrix (values [rows][cols] int8, scales [rows][cols/64] f32)."""

    def __init__(self, q, s):
        self.q = np.ascontiguousarray(q, dtype=np.int8)
        self.s = np.ascontiguousarray(s, dtype=np.float32)
        assert self.s.shape == (self.q.shape[0], self.q.shape[1] // 64)

    def c(self):
        return Q8(self.q.ctypes.data, self.s.ctypes.data, self.q.shape[0], self.q.shape[1])

    def dequant(self):
        return (self.q.astype(np.float64) * np.repeat(self.s.astype(np.float64), 64, axis=1))


def quantize(w):
    w = f32(w)
    rows, cols = w.shape
    q = np.empty((rows, cols), np.int8)
    s = np.empty((rows, cols // 64), np.float32)
    lib().orc_quantize_q8f(w.ctypes.data, rows, cols, q.ctypes.data, s.ctypes.data)
    return Q8Mat(q, s)


def gemv_kn(x, W: Q8Mat, rowdrop=False):
    x = f32(x)
    M = x.shape[0] if x.ndim == 2 else 1
    y = np.empty((M, W.q.shape[1]), np.float32)
    lib().orc_q8_gemv_kn(x.ctypes.data, M, W.c(), y.ctypes.data, 1 if rowdrop else 0)
    return y


def gemv_nk(x, W: Q8Mat):
    x = f32(x)
    M = x.shape[0] if x.ndim == 2 else 1
    y = np.empty((M, W.q.shape[0]), np.float32)
    y64 = np.empty((M, W.q.shape[0]), np.float64)
    lib().orc_q8_gemv_nk(x.ctypes.data, M, W.c(), y.ctypes.data, y64.ctypes.data)
    return y, y64


def embedding(W: Q8Mat, ids):
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    out = np.empty((ids.size, W.q.shape[1]), np.float32)
    lib().orc_embedding_lookup(W.c(), ids.ctypes.data, ids.size, out.ctypes.data)
    return out


def gate_proj(x, w_b, w_a, a_log, dt_bias):
    x, w_b, w_a, a_log, dt_bias = map(f32, (x, w_b, w_a, a_log, dt_bias))
    nh = w_b.shape[1]
    out = np.empty(2 * nh, np.float32)
    lib().orc_gate_proj(x.ctypes.data, x.size, w_b.ctypes.data, w_a.ctypes.data, a_log.ctypes.data,
                        dt_bias.ctypes.data, nh, out.ctypes.data)
    return out


def set_f32_dequant(on):
    """CPU-baseline timing path: Q8F matvecs dequantize the matrix to f32 and run an f32 GEMV."""
    lib().orc_set_f32_dequant(1 if on else 0)


def set_threads(n):
    lib().orc_set_threads(int(n))


def get_threads():
    return int(lib().orc_get_threads())


def argmax(v):
    v = f32(v)
    return int(lib().orc_argmax(v.ctypes.data, v.size))


def argmax_reference_order(v):
    v = f32(v)
    return int(lib().orc_argmax_reference_order(v.ctypes.data, v.size))


def rmsnorm(x, w, eps=1e-6):
    x, w = f32(x), f32(w)
    out = np.empty_like(x)
    lib().orc_rmsnorm(x.ctypes.data, x.size, w.ctypes.data, eps, out.ctypes.data)
    return out


def rmsnorm_gated(x, z, w, eps=1e-6):
    x, z, w = f32(x), f32(z), f32(w)
    out = np.empty_like(x)
    lib().orc_rmsnorm_gated(x.ctypes.data, z.ctypes.data, x.size, w.ctypes.data, eps, out.ctypes.data)
    return out


def conv_update(x, state, w):
    """Returns (out, new_state); state [C][k-1], w [C][k]."""
    x, w = f32(x), f32(w)
    st = f32(state).copy()
    out = np.empty_like(x)
    lib().orc_conv_update(x.ctypes.data, st.ctypes.data, w.ctypes.data, x.size, w.shape[1], out.ctypes.data)
    return out, st


def l2norm(x, eps=1e-6):
    x = f32(x)
    out = np.empty_like(x)
    lib().orc_l2norm(x.ctypes.data, x.size, eps, out.ctypes.data)
    return out


def gated_delta_step(q, k, v, g, beta, S):
    """q,k [H][dk] raw; v [H][dv]; g, beta [H]; S [H][dk][dv] -> (out [H][dv], S_new)."""
    q, k, v, g, beta = map(f32, (q, k, v, g, beta))
    S2 = f32(S).copy()
    H, dk = q.shape
    dv = v.shape[1]
    out = np.empty((H, dv), np.float32)
    lib().orc_gated_delta_step(q.ctypes.data, k.ctypes.data, v.ctypes.data, g.ctypes.data, beta.ctypes.data,
                               S2.ctypes.data, H, dk, dv, out.ctypes.data)
    return out, S2


def gated_delta_chunked(q, k, v, g, beta, S, chunk=64):
    """q,k [T][H][dk]; v [T][H][dv]; g, beta [T][H]; S [H][dk][dv] -> (out [T][H][dv], S_new)."""
    q, k, v, g, beta = map(f32, (q, k, v, g, beta))
    S2 = f32(S).copy()
    T, H, dk = q.shape
    dv = v.shape[2]
    out = np.empty((T, H, dv), np.float32)
    lib().orc_gated_delta_chunked(q.ctypes.data, k.ctypes.data, v.ctypes.data, g.ctypes.data, beta.ctypes.data, T, H,
                                  dk, dv, chunk, S2.ctypes.data, out.ctypes.data)
    return out, S2


def rope_cos_sin(pos, rot_dim=64, theta=1e7):
    c = np.empty(rot_dim, np.float32)
    s = np.empty(rot_dim, np.float32)
    lib().orc_rope_cos_sin(pos, rot_dim, theta, c.ctypes.data, s.ctypes.data)
    return c, s


def apply_rope(x, cos, sin):
    x = f32(x).copy()
    lib().orc_apply_rope(x.ctypes.data, cos.size, f32(cos).ctypes.data, f32(sin).ctypes.data)
    return x


def attention_core(q, kc, vc, T):
    """q [nh][d]; kc, vc [nkv][tmax][d] -> [nh][d]."""
    q, kc, vc = f32(q), f32(kc), f32(vc)
    nh, d = q.shape
    nkv, tmax, _ = kc.shape
    out = np.empty((nh, d), np.float32)
    lib().orc_attention_core(q.ctypes.data, kc.ctypes.data, vc.ctypes.data, T, tmax, nh, nkv, d, out.ctypes.data)
    return out


# ---------------------------------------------------------------- layer / model level

class GdnLayer:
    def __init__(self, qkv: Q8Mat, z: Q8Mat, out: Q8Mat, w_b, w_a, a_log, dt_bias, conv_w, norm_w):
        self.keep = [qkv, z, out] + [f32(a) for a in (w_b, w_a, a_log, dt_bias, conv_w, norm_w)]
        _, _, _, w_b, w_a, a_log, dt_bias, conv_w, norm_w = self.keep
        self.c = GdnW(qkv.c(), z.c(), out.c(), _p(w_b), _p(w_a), _p(a_log), _p(dt_bias), _p(conv_w), _p(norm_w))


class AttnLayer:
    def __init__(self, q: Q8Mat, k: Q8Mat, v: Q8Mat, o: Q8Mat, q_norm, k_norm):
        self.keep = [q, k, v, o, f32(q_norm), f32(k_norm)]
        self.c = AttnW(q.c(), k.c(), v.c(), o.c(), _p(self.keep[4]), _p(self.keep[5]))


class MlpLayer:
    def __init__(self, gate: Q8Mat, up: Q8Mat, down: Q8Mat):
        self.keep = [gate, up, down]
        self.c = MlpW(gate.c(), up.c(), down.c())


def gdn_decode(cfg, layer: GdnLayer, x, conv_state, rec_state):
    x = f32(x)
    B = x.shape[0]
    out = np.empty_like(x)
    lib().orc_gdn_decode(ctypes.byref(cfg), ctypes.byref(layer.c), x.ctypes.data, B, conv_state.ctypes.data,
                         rec_state.ctypes.data, out.ctypes.data)
    return out


def attn_decode(cfg, layer: AttnLayer, x, kc, vc, pos):
    x = f32(x)
    B = x.shape[0]
    pos = np.ascontiguousarray(pos, dtype=np.int32)
    out = np.empty_like(x)
    lib().orc_attn_decode(ctypes.byref(cfg), ctypes.byref(layer.c), x.ctypes.data, B, kc.ctypes.data, vc.ctypes.data,
                          kc.shape[2], pos.ctypes.data, out.ctypes.data)
    return out


def mlp_decode(cfg, layer: MlpLayer, x):
    x = f32(x)
    out = np.empty_like(x)
    lib().orc_mlp_decode(ctypes.byref(cfg), ctypes.byref(layer.c), x.ctypes.data, x.shape[0], out.ctypes.data)
    return out


class Model:
    """Host model for orc_model_step.  `get(name)` must return the f32 values of a named tensor
    (the names of the reference's module paths, as the product's synthetic builder uses)."""

    def __init__(self, cfg, get, tmax):
        self.cfg = cfg
        d = cfg
        H, F = d.hidden, d.ffn
        nh, vdim = d.lin_heads, d.lin_heads * d.lin_dv
        conv_dim = 2 * nh * d.lin_dk + vdim
        ah, kvh, hd = d.attn_heads, d.kv_heads, d.head_dim
        self.keep = []

        def q8(name, rows, cols):
            m = quantize(get(name, rows * cols).reshape(rows, cols))
            self.keep.append(m)
            return m

        def fv(name, n):
            a = f32(get(name, n))
            self.keep.append(a)
            return a

        self.embed = q8("embed_tokens", d.vocab, H)
        self.final_norm = fv("norm", H)
        n = d.n_layers
        self.layers = (LayerW * n)()
        self.conv = [None] * n
        self.rec = [None] * n
        self.kc = [None] * n
        self.vc = [None] * n
        for l in range(n):
            p = f"layers.{l}."
            Lw = self.layers[l]
            Lw.in_norm = _p(fv(p + "input_layernorm", H))
            Lw.post_norm = _p(fv(p + "post_attention_layernorm", H))
            if (l + 1) % d.full_interval != 0:
                a = p + "linear_attn."
                g = GdnLayer(q8(a + "in_proj_qkv", H, conv_dim), q8(a + "in_proj_z", H, vdim),
                             q8(a + "out_proj", vdim, H), fv(a + "in_proj_b", H * nh).reshape(H, nh),
                             fv(a + "in_proj_a", H * nh).reshape(H, nh), fv(a + "a_log", nh), fv(a + "dt_bias", nh),
                             fv(a + "conv1d", conv_dim * d.conv_k).reshape(conv_dim, d.conv_k),
                             fv(a + "norm", d.lin_dv))
                self.keep.append(g)
                Lw.gdn = g.c
                self.conv[l] = np.zeros((conv_dim, d.conv_k - 1), np.float32)
                self.rec[l] = np.zeros((nh, d.lin_dk, d.lin_dv), np.float32)
            else:
                a = p + "self_attn."
                at = AttnLayer(q8(a + "q_proj", H, ah * hd * 2), q8(a + "k_proj", H, kvh * hd),
                               q8(a + "v_proj", H, kvh * hd), q8(a + "o_proj", ah * hd, H), fv(a + "q_norm", hd),
                               fv(a + "k_norm", hd))
                self.keep.append(at)
                Lw.attn = at.c
                self.kc[l] = np.zeros((kvh, tmax, hd), np.float32)
                self.vc[l] = np.zeros((kvh, tmax, hd), np.float32)
            m = p + "mlp."
            ml = MlpLayer(q8(m + "gate_proj", H, F), q8(m + "up_proj", H, F), q8(m + "down_proj", F, H))
            self.keep.append(ml)
            Lw.mlp = ml.c
        self.mw = ModelW(self.embed.c(), self.layers, _p(self.final_norm))
        arr = lambda xs: (c_vp * n)(*[(_p(x) if x is not None else None) for x in xs])
        self.cache = CacheC(arr(self.conv), arr(self.rec), arr(self.kc), arr(self.vc), tmax, 0)

    def set_position(self, pos):
        """Set the cache length (tokens already cached) without running them: the caches keep
        whatever they hold.  Used to time a step at a given context; results are then not a
        real continuation."""
        self.cache.pos = int(pos)

    def step(self, token, want_logits=False):
        if not 0 <= self.cache.pos < self.cache.tmax:
            raise ValueError(f"oracle model: position {self.cache.pos} outside the cache of {self.cache.tmax} tokens")
        logits = np.empty(self.cfg.vocab, np.float32) if want_logits else None
        margin = ctypes.c_double(0.0)
        t = lib().orc_model_step(ctypes.byref(self.cfg), ctypes.byref(self.mw), ctypes.byref(self.cache), int(token),
                                 _p(logits), ctypes.byref(margin))
        return int(t), margin.value, logits

    def generate(self, prompt, n_new):
        """(tokens[n_new+1], margins[n_new+1]) with the product's generate() semantics."""
        toks, margins = [], []
        t = None
        for i, tok in enumerate(prompt):
            t, mg, _ = self.step(tok)
        toks.append(t)
        margins.append(mg)
        for _ in range(n_new):
            t, mg, _ = self.step(t)
            toks.append(t)
            margins.append(mg)
        return np.array(toks, np.int32), np.array(margins)
