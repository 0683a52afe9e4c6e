// extern "C" entry points for the tensor-level (kernels.rs) and layer-level (text_modules.rs)
// surface.  Argument checking lives here; kernels assume validated shapes.
//
// Workspace layout of every entry point: [completion counters (kCounterBytes)]
// [fixed-point accumulators][f32 scratch].  Counters and accumulators must be zero when a call
// starts and are zero again when it completes, so a workspace can be reused by later calls of
// the same entry point on the same stream.
#include "q35_host.h"

#include <algorithm>
#include <cmath>
#include <cstring>

namespace q35 {

namespace {
thread_local std::string g_err;

inline hipStream_t S(void* s) { return static_cast<hipStream_t>(s); }

int check_q8f(const q35_q8f& W, const char* what) {
  if (!W.q || !W.scale) return fail(Q35_E_ARG, std::string(what) + ": null Q8F pointer");
  if (W.rows < 1 || W.cols < 64 || (W.cols % 64) != 0)
    return fail(Q35_E_SHAPE, std::string(what) + ": Q8F cols must be a positive multiple of 64");
  if (W.layout != Q35_KN && W.layout != Q35_NK && W.layout != Q35_KN_TILED && W.layout != Q35_KN_PANEL)
    return fail(Q35_E_ARG, std::string(what) + ": bad layout");
  if ((reinterpret_cast<uintptr_t>(W.q) & 15) != 0) return fail(Q35_E_ALIGN, std::string(what) + ": q not 16-byte aligned");
  return Q35_OK;
}

// Projection weights of the layer entry points: [K][N] storage, row-major or tiled.
int check_kn(const q35_q8f& W, const char* what) {
  const int rc = check_q8f(W, what);
  if (rc) return rc;
  if (W.layout == Q35_NK || W.layout == Q35_KN_PANEL)
    return fail(Q35_E_ARG, std::string(what) + ": layer projections must be Q35_KN or Q35_KN_TILED");
  return Q35_OK;
}

// NK rows of x handled per launch: LDS holds MR*K floats.
int nk_group(int K) { return nk_max_rows(K); }

MvSeg seg_of(const q35_q8f& W, fx_t* acc, int ldacc) {
  return MvSeg{W.q, W.scale, acc, W.cols, ldacc, W.layout == Q35_KN_TILED ? 1 : 0};
}

// Bump allocator over a workspace region.
struct Carver {
  char* p;
  size_t left;
  template <class T>
  T* take(size_t n) {
    const size_t b = align256(n * sizeof(T));
    if (b > left) return nullptr;
    T* r = reinterpret_cast<T*>(p);
    p += b; left -= b;
    return r;
  }
};

struct LayerDims {
  int H, F, nh, dk, dv, key_dim, vdim, conv_dim, ah, kvh, hd;
};
LayerDims ldims(const q35_dims& d) {
  LayerDims L;
  L.H = d.hidden; L.F = d.ffn; L.nh = d.lin_heads; L.dk = d.lin_dk; L.dv = d.lin_dv;
  L.key_dim = L.nh * L.dk; L.vdim = L.nh * L.dv; L.conv_dim = 2 * L.key_dim + L.vdim;
  L.ah = d.attn_heads; L.kvh = d.kv_heads; L.hd = d.head_dim;
  return L;
}

// accumulator bytes of the three layer calls (each region 256-byte aligned)
size_t acc_bytes(const q35_dims& d, int B) {
  const LayerDims L = ldims(d);
  auto a = [](size_t n) { return align256(n * sizeof(fx_t)); };
  const size_t gdn = a((size_t)B * (L.conv_dim + L.vdim)) + a((size_t)B * 2 * L.nh) + a((size_t)B * L.H);
  const size_t att = a((size_t)B * (L.ah * L.hd * 2 + 2 * L.kvh * L.hd)) + a((size_t)B * L.H);
  const size_t mlp = a((size_t)B * 2 * L.F) + a((size_t)B * L.H);
  return std::max(gdn, std::max(att, mlp));
}

size_t scratch_bytes(const q35_dims& d, int B, int tmax) {
  const LayerDims L = ldims(d);
  const size_t gdn = align256((size_t)B * L.vdim * 4);
  const size_t att = (attn_ws_bytes(B, L.ah, L.kvh, L.hd, tmax) - kCounterBytes) + align256((size_t)B * L.ah * L.hd * 4);
  return std::max(gdn, att);
}

}  // namespace

void set_error(const std::string& msg) { g_err = msg; }
int fail(int code, const std::string& msg) {
  g_err = msg;
  return code;
}

int validate_dims(const q35_dims& d) {
  if (d.hidden < 64 || d.hidden % 64 || d.ffn < 64 || d.ffn % 64 || d.vocab < 1 || d.n_layers < 1 || d.full_interval < 1)
    return fail(Q35_E_SHAPE, "dims: hidden/ffn must be multiples of 64, vocab/n_layers/full_interval >= 1");
  if (d.lin_dk != 128 || d.lin_dv % 32 || d.conv_k != 4 || d.lin_heads < 1 || (256 % (2 * d.lin_heads)) != 0)
    return fail(Q35_E_SHAPE, "dims: linear heads need dk=128, dv%32==0, conv_k=4, 2*heads | 256");
  if (d.head_dim != 256 || d.kv_heads < 1 || d.attn_heads % d.kv_heads || d.attn_heads / d.kv_heads > 4 ||
      d.rot_dim < 2 || d.rot_dim > d.head_dim || d.rot_dim % 2)
    return fail(Q35_E_SHAPE, "dims: attention needs head_dim=256, heads/kv_heads in 1..4, even rot_dim");
  if ((d.lin_heads * d.lin_dv) % 64 || (d.attn_heads * d.head_dim) % 64) return fail(Q35_E_SHAPE, "dims: widths % 64");
  return Q35_OK;
}

}  // namespace q35

using namespace q35;

extern "C" {

const char* q35_last_error(void) { return g_err.c_str(); }

q35_dims q35_dims_qwen35_2b(void) {
  q35_dims d;
  d.hidden = 2048; d.ffn = 6144; d.vocab = 248320; d.n_layers = 24; d.full_interval = 4;
  d.lin_heads = 16; d.lin_dk = 128; d.lin_dv = 128; d.conv_k = 4;
  d.attn_heads = 8; d.kv_heads = 2; d.head_dim = 256; d.rot_dim = 64;
  d.eps = 1e-6f; d.theta = 1e7f;
  return d;
}

size_t q35_q8_gemv_ws_bytes(int32_t M, q35_q8f W) {
  if (W.layout == Q35_KN_PANEL) return 0;
  if (W.layout == Q35_NK) return kCounterBytes;
  const int m = std::max(1, std::min<int>(M, 8));
  return kCounterBytes + align256((size_t)m * W.cols * sizeof(fx_t));
}

int q35_q8_gemv(const float* x, int32_t M, q35_q8f W, float* y, void* ws, size_t ws_bytes, void* stream) {
  int rc = check_q8f(W, "q8_gemv");
  if (rc) return rc;
  if (!x || !y) return fail(Q35_E_ARG, "q8_gemv: null x or y");
  if (M < 1 || M > 64) return fail(Q35_E_SHAPE, "q8_gemv: M must be in [1, 64]");
  if (W.layout == Q35_KN_PANEL) {  // one launch per 8 rows, no workspace
    const int K = W.rows, N = W.cols;
    for (int m0 = 0; m0 < M; m0 += 8)
      if ((rc = mvp_launch(W.q, W.scale, K, N, x + (size_t)m0 * K, K, std::min(8, M - m0), y + (size_t)m0 * N, N,
                           S(stream))))
        return rc;
    return Q35_OK;
  }
  if (W.layout != Q35_NK) {  // split-K with fixed-point sums; one launch per 8 rows
    const int K = W.rows, N = W.cols;
    if (!ws || ws_bytes < q35_q8_gemv_ws_bytes(M, W)) return fail(Q35_E_WS, "q8_gemv: workspace too small");
    fx_t* acc = reinterpret_cast<fx_t*>(ws_scratch(ws));
    for (int m0 = 0; m0 < M; m0 += 8) {
      MvCall c;
      c.err = ws_counters(ws) + kWsErrWord;
      c.K = K; c.M = std::min(8, M - m0); c.nseg = 1;
      c.seg[0] = seg_of(W, acc, N);
      c.pro = PRO_PLAIN; c.x = x + (size_t)m0 * K; c.ldx = K;
      c.y_out = y + (size_t)m0 * N; c.ldy = N; c.tile_ctr = ws_counters(ws);
      if ((rc = mv_kn_launch(c, S(stream)))) return rc;
    }
    return Q35_OK;
  }
  const int N = W.rows, K = W.cols;
  const int g = nk_group(K);
  for (int m0 = 0; m0 < M; m0 += g) {
    NkCall c;
    c.q = W.q; c.s = W.scale; c.N = N; c.K = K; c.M = std::min(g, M - m0);
    c.x = x + (size_t)m0 * K; c.ldx = K; c.y = y + (size_t)m0 * N; c.ldy = N;
    rc = nk_launch(c, ws, ws_bytes, S(stream));
    if (rc) return rc;
  }
  return Q35_OK;
}

int q35_q8_gemv_partial_sum(const float* x, int32_t M, q35_q8f W, float* y, void* ws, size_t ws_bytes, void* stream) {
  return q35_q8_gemv(x, M, W, y, ws, ws_bytes, stream);
}

int q35_q8_lm_head(const float* h, int32_t M, q35_q8f E, float* logits, void* stream) {
  int rc = check_q8f(E, "q8_lm_head");
  if (rc) return rc;
  if (E.layout != Q35_NK) return fail(Q35_E_ARG, "q8_lm_head: embedding table must be Q35_NK");
  if (!h || !logits) return fail(Q35_E_ARG, "q8_lm_head: null pointer");
  if (M < 1 || M > 64) return fail(Q35_E_SHAPE, "q8_lm_head: M must be in [1, 64]");
  const int N = E.rows, K = E.cols;
  const int g = nk_group(K);
  for (int m0 = 0; m0 < M; m0 += g) {
    NkCall c;
    c.q = E.q; c.s = E.scale; c.N = N; c.K = K; c.M = std::min(g, M - m0);
    c.x = h + (size_t)m0 * K; c.ldx = K; c.y = logits + (size_t)m0 * N; c.ldy = N;
    rc = nk_launch(c, nullptr, 0, S(stream));
    if (rc) return rc;
  }
  return Q35_OK;
}

int q35_q8_embedding_lookup(q35_q8f table, const int32_t* ids, int32_t n, float* out, void* stream) {
  int rc = check_q8f(table, "q8_embedding_lookup");
  if (rc) return rc;
  if (table.layout != Q35_NK) return fail(Q35_E_ARG, "q8_embedding_lookup: table must be Q35_NK ([V][D])");
  return embed_launch(table.q, table.scale, table.rows, table.cols, ids, n, out, S(stream));
}

int q35_gate_proj(const float* x, int32_t B, int32_t in_dim, const float* w_b, const float* w_a,
                  const float* a_log, const float* dt_bias, int32_t n_heads, float* out, void* stream) {
  return gate_proj_simple_launch(x, B, in_dim, w_b, w_a, a_log, dt_bias, n_heads, out, S(stream));
}

size_t q35_argmax_ws_bytes(int64_t n) { return argmax_ws_bytes(n); }

int q35_argmax(const float* logits, int64_t n, int32_t* out, void* ws, size_t ws_bytes, void* stream) {
  return argmax_launch(logits, n, out, ws, ws_bytes, S(stream));
}

int q35_workspace_status(void* ws, void* stream) {
  if (!ws) return fail(Q35_E_ARG, "workspace_status: null workspace");
  hipStream_t st = S(stream);
  uint32_t* word = ws_counters(ws) + kWsErrWord;
  uint32_t v = 0;
  Q35_HIP_TRY(hipStreamSynchronize(st));
  Q35_HIP_TRY(hipMemcpy(&v, word, sizeof(v), hipMemcpyDeviceToHost));
  if (v == 0) return Q35_OK;
  const uint32_t zero = 0;
  Q35_HIP_TRY(hipMemcpy(word, &zero, sizeof(zero), hipMemcpyHostToDevice));
  if (v & kWsErrPos)
    return fail(Q35_E_SHAPE, "attention: a row's position d_pos[b] was outside [0, tmax); that row was skipped");
  if (v & kWsErrRange)
    return fail(Q35_E_RANGE, "a value for a fixed-point sum was not finite or |v| >= 2^31 (NaN / Inf or overflowing "
                             "inputs); it was dropped and the outputs are invalid");
  return fail(Q35_E_HIP, "workspace: unknown error bits " + std::to_string(v));
}

size_t q35_layer_ws_bytes(const q35_dims* d, int32_t B, int32_t tmax) {
  if (!d || B < 1) return 0;
  return kCounterBytes + acc_bytes(*d, B) + scratch_bytes(*d, B, std::max(1, tmax));
}

int q35_gated_deltanet_decode(const q35_dims* d, const q35_gdn_weights* w, const float* x, int32_t B,
                              float* conv_state, float* rec_state, float* out, void* ws, size_t ws_bytes,
                              void* stream) {
  if (!d || !w || !x || !conv_state || !rec_state || !out) return fail(Q35_E_ARG, "gated_deltanet_decode: null pointer");
  int rc = validate_dims(*d);
  if (rc) return rc;
  if (B < 1) return fail(Q35_E_SHAPE, "gated_deltanet_decode: B must be >= 1");
  const LayerDims L = ldims(*d);
  if ((rc = check_kn(w->in_proj_qkv, "in_proj_qkv")) || (rc = check_kn(w->in_proj_z, "in_proj_z")) ||
      (rc = check_kn(w->out_proj, "out_proj")))
    return rc;
  if (w->in_proj_qkv.rows != L.H || w->in_proj_qkv.cols != L.conv_dim || w->in_proj_z.rows != L.H ||
      w->in_proj_z.cols != L.vdim || w->out_proj.rows != L.vdim || w->out_proj.cols != L.H)
    return fail(Q35_E_SHAPE, "gated_deltanet_decode: projection shapes do not match dims");
  if (!w->in_proj_b || !w->in_proj_a || !w->a_log || !w->dt_bias || !w->conv_w || !w->norm_w)
    return fail(Q35_E_ARG, "gated_deltanet_decode: null f32 weight");
  if (!ws || ws_bytes < q35_layer_ws_bytes(d, B, 1)) return fail(Q35_E_WS, "gated_deltanet_decode: workspace too small");
  Carver ac{ws_scratch(ws), acc_bytes(*d, B)};
  Carver sc{ws_scratch(ws) + acc_bytes(*d, B), ws_bytes - kCounterBytes - acc_bytes(*d, B)};
  const int ldq = L.conv_dim + L.vdim;
  fx_t* qkvz = ac.take<fx_t>((size_t)B * ldq);
  fx_t* ba = ac.take<fx_t>((size_t)B * 2 * L.nh);
  fx_t* y = ac.take<fx_t>((size_t)B * L.H);
  float* o = sc.take<float>((size_t)B * L.vdim);
  hipStream_t st = S(stream);
  for (int b0 = 0; b0 < B; b0 += 8) {  // in_proj_qkv | in_proj_z | in_proj_b,a (text_modules.rs:497-508,569-576)
    MvCall c;
    c.err = ws_counters(ws) + kWsErrWord;
    c.K = L.H; c.M = std::min(8, B - b0); c.nseg = 2;
    c.seg[0] = seg_of(w->in_proj_qkv, qkvz + (size_t)b0 * ldq, ldq);
    c.seg[1] = seg_of(w->in_proj_z, qkvz + (size_t)b0 * ldq + L.conv_dim, ldq);
    c.pro = PRO_PLAIN; c.x = x + (size_t)b0 * L.H; c.ldx = L.H;
    c.aux_wb = w->in_proj_b; c.aux_wa = w->in_proj_a; c.aux_nh = L.nh;
    c.aux_acc = ba + (size_t)b0 * 2 * L.nh; c.aux_ldo = 2 * L.nh;
    if ((rc = mv_kn_launch(c, st))) return rc;
  }
  GdnCall g;  // conv update, l2norm, recurrent delta rule (:515-530, :627-652)
  g.qkv_f = qkvz; g.ld_qkv = ldq; g.ba_f = ba; g.ld_bg = 2 * L.nh; g.a_log = w->a_log; g.dt_bias = w->dt_bias;
  g.conv_state = conv_state; g.conv_w = w->conv_w; g.S = rec_state; g.o = o; g.ld_o = L.vdim;
  g.B = B; g.nh = L.nh; g.dk = L.dk; g.dv = L.dv; g.conv_k = d->conv_k;
  if ((rc = gdn_step_launch(g, st))) return rc;
  for (int b0 = 0; b0 < B; b0 += 8) {  // gated RMSNorm + out_proj (:654-663); conv state advance
    MvCall c;
    c.err = ws_counters(ws) + kWsErrWord;
    c.K = L.vdim; c.M = std::min(8, B - b0); c.nseg = 1;
    c.seg[0] = seg_of(w->out_proj, y + (size_t)b0 * L.H, L.H);
    c.pro = PRO_GATED; c.x = o + (size_t)b0 * L.vdim; c.ldx = L.vdim;
    c.x2f = qkvz + (size_t)b0 * ldq + L.conv_dim; c.ldx2 = ldq;
    c.pw = w->norm_w; c.group = L.dv; c.eps = d->eps;
    c.cs_state = conv_state + (size_t)b0 * L.conv_dim * 3; c.cs_x = qkvz + (size_t)b0 * ldq;
    c.cs_ch = L.conv_dim; c.cs_ldx = ldq; c.cs_B = c.M;
    if ((rc = mv_kn_launch(c, st))) return rc;
  }
  if ((rc = fx_to_f32_launch(y, (int64_t)B * L.H, out, true, st))) return rc;
  if ((rc = fx_zero_launch(qkvz, (int64_t)B * ldq, st))) return rc;
  return fx_zero_launch(ba, (int64_t)B * 2 * L.nh, st);
}

int q35_attention_decode(const q35_dims* d, const q35_attn_weights* w, const float* x, int32_t B, float* k_cache,
                         float* v_cache, int32_t tmax, const int32_t* d_pos, const float* rope_cos,
                         const float* rope_sin, float* out, void* ws, size_t ws_bytes, void* stream) {
  if (!d || !w || !x || !k_cache || !v_cache || !d_pos || !rope_cos || !rope_sin || !out)
    return fail(Q35_E_ARG, "attention_decode: null pointer");
  int rc = validate_dims(*d);
  if (rc) return rc;
  if (B < 1 || tmax < 1) return fail(Q35_E_SHAPE, "attention_decode: B and tmax must be >= 1");
  const LayerDims L = ldims(*d);
  if ((rc = check_kn(w->q_proj, "q_proj")) || (rc = check_kn(w->k_proj, "k_proj")) ||
      (rc = check_kn(w->v_proj, "v_proj")) || (rc = check_kn(w->o_proj, "o_proj")))
    return rc;
  if (w->q_proj.rows != L.H || w->q_proj.cols != L.ah * L.hd * 2 || w->k_proj.rows != L.H ||
      w->k_proj.cols != L.kvh * L.hd || w->v_proj.rows != L.H || w->v_proj.cols != L.kvh * L.hd ||
      w->o_proj.rows != L.ah * L.hd || w->o_proj.cols != L.H)
    return fail(Q35_E_SHAPE, "attention_decode: projection shapes do not match dims");
  if (!w->q_norm || !w->k_norm) return fail(Q35_E_ARG, "attention_decode: null norm weight");
  if (!ws || ws_bytes < q35_layer_ws_bytes(d, B, tmax)) return fail(Q35_E_WS, "attention_decode: workspace too small");
  const size_t abytes = acc_bytes(*d, B);
  Carver ac{ws_scratch(ws), abytes};
  const int ldqg = L.ah * L.hd * 2, ldo = L.ah * L.hd, LD = ldqg + 2 * L.kvh * L.hd;
  fx_t* qkv = ac.take<fx_t>((size_t)B * LD);
  fx_t* y = ac.take<fx_t>((size_t)B * L.H);
  // scratch after the accumulators: the attention kernel's chunk partials, then its output
  const size_t att_ws = attn_ws_bytes(B, L.ah, L.kvh, L.hd, tmax);
  Carver sc{ws_scratch(ws) + abytes + (att_ws - kCounterBytes), ws_bytes - kCounterBytes - abytes - (att_ws - kCounterBytes)};
  float* att = sc.take<float>((size_t)B * ldo);
  hipStream_t st = S(stream);
  for (int b0 = 0; b0 < B; b0 += 8) {  // q_proj | k_proj | v_proj (text_modules.rs:855-893)
    MvCall c;
    c.err = ws_counters(ws) + kWsErrWord;
    c.K = L.H; c.M = std::min(8, B - b0); c.nseg = 3;
    c.seg[0] = seg_of(w->q_proj, qkv + (size_t)b0 * LD, LD);
    c.seg[1] = seg_of(w->k_proj, qkv + (size_t)b0 * LD + ldqg, LD);
    c.seg[2] = seg_of(w->v_proj, qkv + (size_t)b0 * LD + ldqg + L.kvh * L.hd, LD);
    c.pro = PRO_PLAIN; c.x = x + (size_t)b0 * L.H; c.ldx = L.H;
    if ((rc = mv_kn_launch(c, st))) return rc;
  }
  AttnCall a;  // norms, RoPE, KV append, attention, gate (:860-936)
  a.qg_f = qkv; a.ld_qg = LD; a.k_f = qkv + ldqg; a.v_f = qkv + ldqg + L.kvh * L.hd; a.ld_kv = LD;
  a.qnw = w->q_norm; a.knw = w->k_norm; a.eps = d->eps;
  a.rcos = rope_cos; a.rsin = rope_sin; a.rot = d->rot_dim; a.kc = k_cache; a.vc = v_cache; a.tmax = tmax;
  a.pos = d_pos; a.out = att; a.ld_out = ldo; a.B = B; a.nh = L.ah; a.nkv = L.kvh; a.hd = L.hd;
  // the attention kernel takes [counters | partials]; its partials start right after the accumulators
  if ((rc = attn_launch_split(a, ws_counters(ws), ws_scratch(ws) + abytes, att_ws - kCounterBytes, st))) return rc;
  for (int b0 = 0; b0 < B; b0 += 8) {  // o_proj (:938-942)
    MvCall c;
    c.err = ws_counters(ws) + kWsErrWord;
    c.K = ldo; c.M = std::min(8, B - b0); c.nseg = 1;
    c.seg[0] = seg_of(w->o_proj, y + (size_t)b0 * L.H, L.H);
    c.pro = PRO_PLAIN; c.x = att + (size_t)b0 * ldo; c.ldx = ldo;
    if ((rc = mv_kn_launch(c, st))) return rc;
  }
  if ((rc = fx_to_f32_launch(y, (int64_t)B * L.H, out, true, st))) return rc;
  return fx_zero_launch(qkv, (int64_t)B * LD, st);
}

int q35_mlp_decode(const q35_dims* d, const q35_mlp_weights* w, const float* x, int32_t B, float* out, void* ws,
                   size_t ws_bytes, void* stream) {
  if (!d || !w || !x || !out) return fail(Q35_E_ARG, "mlp_decode: null pointer");
  int rc = validate_dims(*d);
  if (rc) return rc;
  if (B < 1) return fail(Q35_E_SHAPE, "mlp_decode: B must be >= 1");
  const LayerDims L = ldims(*d);
  if ((rc = check_kn(w->gate_proj, "gate_proj")) || (rc = check_kn(w->up_proj, "up_proj")) ||
      (rc = check_kn(w->down_proj, "down_proj")))
    return rc;
  if (w->gate_proj.rows != L.H || w->gate_proj.cols != L.F || w->up_proj.rows != L.H || w->up_proj.cols != L.F ||
      w->down_proj.rows != L.F || w->down_proj.cols != L.H)
    return fail(Q35_E_SHAPE, "mlp_decode: projection shapes do not match dims");
  if (!ws || ws_bytes < q35_layer_ws_bytes(d, B, 1)) return fail(Q35_E_WS, "mlp_decode: workspace too small");
  Carver ac{ws_scratch(ws), acc_bytes(*d, B)};
  fx_t* gu = ac.take<fx_t>((size_t)B * 2 * L.F);
  fx_t* y = ac.take<fx_t>((size_t)B * L.H);
  hipStream_t st = S(stream);
  for (int b0 = 0; b0 < B; b0 += 8) {  // gate_proj | up_proj (text_modules.rs:1003-1004)
    MvCall c;
    c.err = ws_counters(ws) + kWsErrWord;
    c.K = L.H; c.M = std::min(8, B - b0); c.nseg = 2;
    c.seg[0] = seg_of(w->gate_proj, gu + (size_t)b0 * 2 * L.F, 2 * L.F);
    c.seg[1] = seg_of(w->up_proj, gu + (size_t)b0 * 2 * L.F + L.F, 2 * L.F);
    c.pro = PRO_PLAIN; c.x = x + (size_t)b0 * L.H; c.ldx = L.H;
    if ((rc = mv_kn_launch(c, st))) return rc;
  }
  for (int b0 = 0; b0 < B; b0 += 8) {  // up * silu(gate) -> down_proj (:1005)
    MvCall c;
    c.err = ws_counters(ws) + kWsErrWord;
    c.K = L.F; c.M = std::min(8, B - b0); c.nseg = 1;
    c.seg[0] = seg_of(w->down_proj, y + (size_t)b0 * L.H, L.H);
    c.pro = PRO_SWIGLU; c.xf = gu + (size_t)b0 * 2 * L.F; c.ldx = 2 * L.F; c.swiglu_off = L.F;
    if ((rc = mv_kn_launch(c, st))) return rc;
  }
  if ((rc = fx_to_f32_launch(y, (int64_t)B * L.H, out, true, st))) return rc;
  return fx_zero_launch(gu, (int64_t)B * 2 * L.F, st);
}

int q35_gated_delta_rule_decode(const float* mixed_qkv, int32_t B, const float* beta_g, float* conv_state,
                                const float* conv_w, float* rec_state, float* core_out, int32_t lin_heads,
                                int32_t lin_dk, int32_t lin_dv, void* ws, size_t ws_bytes, void* stream) {
  if (!mixed_qkv || !beta_g || !conv_state || !conv_w || !rec_state || !core_out)
    return fail(Q35_E_ARG, "gated_delta_rule_decode: null pointer");
  if (B < 1 || lin_heads < 1) return fail(Q35_E_SHAPE, "gated_delta_rule_decode: B and heads must be >= 1");
  GdnCall g;
  const int conv_dim = 2 * lin_heads * lin_dk + lin_heads * lin_dv;
  g.qkv = mixed_qkv; g.ld_qkv = conv_dim; g.bg = beta_g; g.ld_bg = 2 * lin_heads; g.conv_state = conv_state;
  g.conv_w = conv_w; g.S = rec_state; g.o = core_out; g.ld_o = lin_heads * lin_dv; g.B = B; g.nh = lin_heads;
  g.dk = lin_dk; g.dv = lin_dv; g.conv_k = 4;
  // with a workspace the step kernel advances the conv state itself (one launch)
  const bool fused = ws && ws_bytes >= kCounterBytes && (int64_t)B * lin_heads <= kMaxCounters;
  if (fused) g.head_ctr = ws_counters(ws);
  int rc = gdn_step_launch(g, S(stream));
  if (rc || fused) return rc;
  return conv_shift_launch(conv_state, mixed_qkv, B, conv_dim, S(stream));
}

int q35_attention_core_decode(const q35_dims* d, const float* q_gate, const float* k_new, const float* v_new,
                              int32_t kv_ld, int32_t B, const float* q_norm, const float* k_norm, float* k_cache,
                              float* v_cache, int32_t tmax, const int32_t* d_pos, const float* rope_cos,
                              const float* rope_sin, float* out, void* ws, size_t ws_bytes, void* stream) {
  if (!d) return fail(Q35_E_ARG, "attention_core_decode: null dims");
  int rc = validate_dims(*d);
  if (rc) return rc;
  if (kv_ld < d->kv_heads * d->head_dim) return fail(Q35_E_SHAPE, "attention_core_decode: kv_ld too small");
  AttnCall a;
  a.qg = q_gate; a.ld_qg = d->attn_heads * d->head_dim * 2; a.k = k_new; a.v = v_new; a.ld_kv = kv_ld;
  a.qnw = q_norm; a.knw = k_norm; a.eps = d->eps; a.rcos = rope_cos; a.rsin = rope_sin; a.rot = d->rot_dim;
  a.kc = k_cache; a.vc = v_cache; a.tmax = tmax; a.pos = d_pos; a.out = out; a.ld_out = d->attn_heads * d->head_dim;
  a.B = B; a.nh = d->attn_heads; a.nkv = d->kv_heads; a.hd = d->head_dim;
  return attn_launch(a, ws, ws_bytes, S(stream));
}

// ---------------------------------------------------------------- prompt (seq_len > 1) surface

int q35_q8_gemm(const float* x, int32_t M, int32_t ldx, q35_q8f W, float* y, int32_t ldy, int32_t accumulate,
                void* stream) {
  if (W.layout == Q35_KN_MB) return fail(Q35_E_WS, "q8_gemm: Q35_KN_MB needs q35_q8_gemm_ws with a workspace");
  int rc = check_q8f(W, "q8_gemm");
  if (rc) return rc;
  if (!x || !y) return fail(Q35_E_ARG, "q8_gemm: null pointer");
  if (W.layout == Q35_KN_PANEL) return fail(Q35_E_ARG, "q8_gemm: layout must be Q35_KN, Q35_KN_TILED or Q35_NK");
  const bool nk = W.layout == Q35_NK;
  const int K = nk ? W.cols : W.rows, N = nk ? W.rows : W.cols;
  if (M < 1) return fail(Q35_E_SHAPE, "q8_gemm: M must be >= 1");
  if (K % 64 != 0 || N % 64 != 0) return fail(Q35_E_SHAPE, "q8_gemm: K and N must be multiples of 64");
  if (ldx < K || ldy < N) return fail(Q35_E_SHAPE, "q8_gemm: ldx >= K and ldy >= N required");
  GemmCall c;
  c.x = x; c.ldx = ldx; c.M = M; c.K = K; c.nseg = 1; c.accumulate = accumulate ? 1 : 0;
  c.seg[0] = GemmSeg{W.q, W.scale, y, N, W.layout, ldy};
  return gemm_launch(c, S(stream));
}

size_t q35_q8_gemm_ws_bytes(int32_t M, q35_q8f W) {
  if (M < 1) return 0;
  const int N = W.layout == Q35_NK ? W.rows : W.cols;
  const size_t aux = W.layout == Q35_KN_MB ? gemm_aux_floats(M) : 0;
  return (aux + gemm_part_floats(M, N)) * sizeof(float);
}

int q35_q8_gemm_ws(const float* x, int32_t M, int32_t ldx, q35_q8f W, float* y, int32_t ldy, int32_t accumulate,
                   void* ws, size_t ws_bytes, void* stream) {
  if (!ws) return q35_q8_gemm(x, M, ldx, W, y, ldy, accumulate, stream);
  if (W.layout == Q35_KN_MB) {  // f16 matrix cores: workspace = row / scale maxima, then partials
    if (!W.q || !W.scale || !x || !y) return fail(Q35_E_ARG, "q8_gemm_ws: null pointer");
    const int K = W.rows, N = W.cols;
    if (M < 1 || K < 64 || K % 64 || N < 128 || N % 128)
      return fail(Q35_E_SHAPE, "q8_gemm_ws: Q35_KN_MB needs M >= 1, K a multiple of 64 and N of 128");
    if (ldx < K || ldy < N) return fail(Q35_E_SHAPE, "q8_gemm_ws: ldx >= K and ldy >= N required");
    if ((reinterpret_cast<uintptr_t>(ws) & 15) != 0) return fail(Q35_E_ALIGN, "q8_gemm_ws: workspace not 16-byte aligned");
    const size_t aux = gemm_aux_floats(M);
    if (ws_bytes < aux * sizeof(float)) return fail(Q35_E_WS, "q8_gemm_ws: workspace too small");
    GemmCall c;
    c.x = x; c.ldx = ldx; c.M = M; c.K = K; c.nseg = 1; c.accumulate = accumulate ? 1 : 0;
    c.seg[0] = GemmSeg{W.q, W.scale, y, N, Q35_KN_MB, ldy};
    c.aux = static_cast<float*>(ws);
    c.part = c.aux + aux;
    c.part_floats = ws_bytes / sizeof(float) - aux;
    return gemm_launch(c, S(stream));
  }
  int rc = check_q8f(W, "q8_gemm_ws");
  if (rc) return rc;
  if (!x || !y) return fail(Q35_E_ARG, "q8_gemm_ws: null pointer");
  if (W.layout == Q35_KN_PANEL) return fail(Q35_E_ARG, "q8_gemm_ws: layout must be Q35_KN, Q35_KN_TILED or Q35_NK");
  const bool nk = W.layout == Q35_NK;
  const int K = nk ? W.cols : W.rows, N = nk ? W.rows : W.cols;
  if (M < 1) return fail(Q35_E_SHAPE, "q8_gemm_ws: M must be >= 1");
  if (K % 64 != 0 || N % 64 != 0) return fail(Q35_E_SHAPE, "q8_gemm_ws: K and N must be multiples of 64");
  if (ldx < K || ldy < N) return fail(Q35_E_SHAPE, "q8_gemm_ws: ldx >= K and ldy >= N required");
  if ((reinterpret_cast<uintptr_t>(ws) & 15) != 0) return fail(Q35_E_ALIGN, "q8_gemm_ws: workspace not 16-byte aligned");
  GemmCall c;
  c.x = x; c.ldx = ldx; c.M = M; c.K = K; c.nseg = 1; c.accumulate = accumulate ? 1 : 0;
  c.seg[0] = GemmSeg{W.q, W.scale, y, N, W.layout, ldy};
  c.part = static_cast<float*>(ws);
  c.part_floats = ws_bytes / sizeof(float);
  return gemm_launch(c, S(stream));
}

size_t q35_q8_gemv_mb_ws_bytes(int32_t M, q35_q8f W) {
  if (W.layout != Q35_KN_MB || M < 1 || M > 32 || W.rows < 128 || W.cols < 128) return 0;
  const int K = W.rows, N = W.cols;
  return kCounterBytes + align256(32 * sizeof(fx_t)) + align256((size_t)(N / 64) * sizeof(float)) +
         align256(mb_part_floats(N / 64, K, M) * sizeof(float)) + align256(mb_word_floats(N / 64, M) * sizeof(float));
}

int q35_q8_gemv_mb(const float* x, int32_t M, int32_t ldx, int32_t prologue, const float* norm_w, const float* z,
                   int32_t ldz, int32_t group, float eps, q35_q8f W, float* y, int32_t ldy, int32_t accumulate,
                   void* ws, size_t ws_bytes, void* stream) {
  if (W.layout != Q35_KN_MB) return fail(Q35_E_ARG, "q8_gemv_mb: W must be Q35_KN_MB");
  if (!W.q || !W.scale || !x || !y) return fail(Q35_E_ARG, "q8_gemv_mb: null pointer");
  const int K = W.rows, N = W.cols;
  if (M < 1 || M > 32) return fail(Q35_E_SHAPE, "q8_gemv_mb: M must be in [1, 32]");
  if (K < 128 || K % 128 || N < 128 || N % 128) return fail(Q35_E_SHAPE, "q8_gemv_mb: K and N must be multiples of 128");
  if (prologue < Q35_MB_PLAIN || prologue > Q35_MB_SWIGLU) return fail(Q35_E_ARG, "q8_gemv_mb: bad prologue");
  if ((prologue == Q35_MB_RMS || prologue == Q35_MB_GATED) && !norm_w) return fail(Q35_E_ARG, "q8_gemv_mb: null norm_w");
  if (ldx < (prologue == Q35_MB_SWIGLU ? 2 * K : K) || ldy < N) return fail(Q35_E_SHAPE, "q8_gemv_mb: ldx / ldy too small");
  if (!ws || ws_bytes < q35_q8_gemv_mb_ws_bytes(M, W)) return fail(Q35_E_WS, "q8_gemv_mb: workspace too small");
  hipStream_t st = S(stream);
  uint32_t* ctr = ws_counters(ws);
  const size_t pf = mb_part_floats(N / 64, K, M);
  Carver cv{ws_scratch(ws), ws_bytes - kCounterBytes};
  fx_t* ss = cv.take<fx_t>(32);
  float* f = cv.take<float>((size_t)(N / 64));
  float* part = cv.take<float>(std::max<size_t>(pf, 1));
  const size_t wf = mb_word_floats(N / 64, M);
  float* words = cv.take<float>(wf);
  MbCall c;
  c.M = M; c.K = K; c.x = x; c.ldx = ldx; c.pro = prologue; c.eps = eps; c.add = accumulate ? 1 : 0;
  c.nseg = 1;
  c.seg[0] = MbSeg{W.q, W.scale, y, N, ldy, nullptr};
  c.part = part; c.part_floats = pf; c.ctr = ctr; c.nctr = kMaxCounters; c.err = ctr + kWsErrWord;
  c.words = words; c.word_floats = wf;
  int rc;
  if (prologue == Q35_MB_RMS) {
    if ((rc = mb_row_ss_launch(x, ldx, K, M, ss, c.err, st)) || (rc = mb_split_factor_launch(W.scale, K, N, norm_w, f, st)))
      return rc;
    c.ss = ss; c.pw = norm_w; c.seg[0].f = f;
  } else if (prologue == Q35_MB_GATED) {
    c.z = z; c.ldz = ldz; c.group = group; c.pw = norm_w;
  } else if (prologue == Q35_MB_SWIGLU) {
    c.swiglu_off = K;
  }
  return mb_launch(c, st);
}

int q35_q8f_pack_mb(q35_q8f W, int8_t* q_mb, float* scale_mb, void* stream) {
  if (!W.q || !W.scale || !q_mb || !scale_mb) return fail(Q35_E_ARG, "q8f_pack_mb: null pointer");
  if (W.layout != Q35_KN && W.layout != Q35_KN_TILED) return fail(Q35_E_ARG, "q8f_pack_mb: W must be Q35_KN or Q35_KN_TILED");
  if (W.rows < 32 || W.rows % 32 || W.cols < 64 || W.cols % 64)
    return fail(Q35_E_SHAPE, "q8f_pack_mb: K a multiple of 32 and N of 64 required");
  return mb_convert_launch(W.q, W.scale, W.rows, W.cols, q_mb, scale_mb, S(stream), W.layout == Q35_KN_TILED ? 1 : 0);
}

int q35_gate_proj_prompt(const float* x, int32_t T, int32_t in_dim, const float* w_b, const float* w_a,
                         const float* a_log, const float* dt_bias, int32_t n_heads, float* out, void* stream) {
  return gate_prompt_launch(x, in_dim, T, in_dim, w_b, w_a, a_log, dt_bias, n_heads, out, S(stream));
}

size_t q35_gated_delta_rule_prefill_ws_bytes(int32_t T, int32_t lin_heads) {
  if (T < 1 || lin_heads < 1) return 0;
  const size_t nchunk = (size_t)(T + kGdnChunk - 1) / kGdnChunk;
  return (size_t)lin_heads * nchunk * kGdnScratchPerChunk * sizeof(float);
}

int q35_gated_delta_rule_prefill(const float* mixed_qkv, int32_t T, int32_t ld_qkv, const float* beta_g,
                                 float* conv_state, const float* conv_w, float* rec_state, float* core_out,
                                 int32_t lin_heads, int32_t lin_dk, int32_t lin_dv, void* ws, size_t ws_bytes,
                                 void* stream) {
  if (!mixed_qkv || !beta_g || !conv_state || !conv_w || !rec_state || !core_out || !ws)
    return fail(Q35_E_ARG, "gated_delta_rule_prefill: null pointer");
  if (T < 1 || lin_heads < 1) return fail(Q35_E_SHAPE, "gated_delta_rule_prefill: T and heads must be >= 1");
  if (lin_dk != 128 || lin_dv != 128) return fail(Q35_E_SHAPE, "gated_delta_rule_prefill: head dims must be 128");
  const int key_dim = lin_heads * lin_dk, conv_dim = 2 * key_dim + lin_heads * lin_dv;
  if (ld_qkv < conv_dim) return fail(Q35_E_SHAPE, "gated_delta_rule_prefill: ld_qkv < conv_dim");
  if (ws_bytes < q35_gated_delta_rule_prefill_ws_bytes(T, lin_heads))
    return fail(Q35_E_WS, "gated_delta_rule_prefill: workspace too small");
  GdnPrefill g;
  g.raw = mixed_qkv; g.ld_raw = ld_qkv; g.conv_state = conv_state; g.conv_state_out = conv_state; g.conv_w = conv_w;
  g.bg = beta_g; g.ld_bg = 2 * lin_heads; g.scr = static_cast<float*>(ws); g.S = rec_state; g.out = core_out;
  g.ld_out = lin_heads * lin_dv; g.T = T; g.nh = lin_heads; g.key_dim = key_dim;
  g.nchunk = (T + kGdnChunk - 1) / kGdnChunk; g.qscale = powf((float)lin_dk, -0.5f);
  return gdn_prefill_launch(g, S(stream));
}

size_t q35_attention_prefill_ws_bytes(const q35_dims* d, int32_t T) {
  if (!d || T < 1) return 0;
  return (size_t)T * d->attn_heads * d->head_dim * sizeof(float);
}

int q35_attention_core_prefill(const q35_dims* d, const float* q_gate, int32_t ld_qg, const float* k_new,
                               const float* v_new, int32_t kv_ld, int32_t T, int32_t p0, const float* q_norm,
                               const float* k_norm, float* k_cache, float* v_cache, int32_t tmax,
                               const float* rope_cos, const float* rope_sin, float* out, void* ws, size_t ws_bytes,
                               void* stream) {
  if (!d) return fail(Q35_E_ARG, "attention_core_prefill: null dims");
  int rc = validate_dims(*d);
  if (rc) return rc;
  if (d->head_dim != kHdP) return fail(Q35_E_SHAPE, "attention_core_prefill: head_dim must be 256");
  if (ld_qg < d->attn_heads * d->head_dim * 2 || kv_ld < d->kv_heads * d->head_dim)
    return fail(Q35_E_SHAPE, "attention_core_prefill: row strides too small");
  if (!ws || ws_bytes < q35_attention_prefill_ws_bytes(d, T)) return fail(Q35_E_WS, "attention_core_prefill: workspace too small");
  AttnPrefill a;
  a.qg = q_gate; a.ld_qg = ld_qg; a.k = k_new; a.v = v_new; a.ld_kv = kv_ld; a.qnw = q_norm; a.knw = k_norm;
  a.eps = d->eps; a.rcos = rope_cos; a.rsin = rope_sin; a.rot = d->rot_dim; a.kc = k_cache; a.vc = v_cache;
  a.tmax = tmax; a.p0 = p0; a.T = T; a.nh = d->attn_heads; a.nkv = d->kv_heads; a.qbuf = static_cast<float*>(ws);
  a.out = out; a.ld_out = d->attn_heads * d->head_dim; a.scale = (float)(1.0 / std::sqrt((double)d->head_dim));
  return attn_prefill_launch(a, S(stream));
}

int q35_rope_tables(const q35_dims* d, int32_t tmax, float* cos_host, float* sin_host) {
  if (!d || !cos_host || !sin_host || tmax < 1) return fail(Q35_E_ARG, "rope_tables: bad argument");
  const int rot = d->rot_dim, half = rot / 2;
  const float sf = -std::log(d->theta) / (float)rot;
  for (int i = 0; i < half; ++i) {
    const float inv = std::exp((float)(2 * i) * sf);
    for (int t = 0; t < tmax; ++t) {
      const float ang = (float)t * inv;
      const float c = std::cos(ang), s = std::sin(ang);
      cos_host[(size_t)t * rot + i] = c; cos_host[(size_t)t * rot + i + half] = c;
      sin_host[(size_t)t * rot + i] = s; sin_host[(size_t)t * rot + i + half] = s;
    }
  }
  return Q35_OK;
}

}  // extern "C"
