// Batched greedy decode: B independent sequences through the whole decode step at once, sharing
// one model's weights.  The reference decodes one sequence (kernels.rs:447,683 squeeze to bs = 1);
// here every projection streams its weights once for up to 32 sequences (the matrix-core batch
// kernels of mvb.hip, on an MB-layout copy of the weights built once per model), while each
// sequence keeps its own conv / recurrent states, KV cache, position, prompt, token and history.
// A step:
//   embedding of each row's token (its next prompt id, or its last argmax) -> f32 residual row,
//     with the row's sum of squares for the first RMSNorm
//   per layer: [RMSNorm -> qkv|z (+ DeltaNet gate sums) | q|k|v] -> DeltaNet step / attention
//              (all rows, own positions) -> [gated RMSNorm -> out | o] += residual
//              -> [RMSNorm -> gate|up] -> [SwiGLU -> down] += residual
//   final RMSNorm + lm_head rows -> argmax per row (reference tie order) -> token, position + 1
// Each RMSNorm's per-row statistic is accumulated by the projection that last updated the
// residual rows (fixed point, order-independent), so no kernel re-reads whole rows for it.  The
// step can be captured in a hipGraph (all control data is in device memory).  Prompts are fed
// either through the decode step (rows at their own positions, ragged lengths) or through the
// prompt path one sequence at a time.
#include "model_internal.h"

#include <algorithm>
#include <chrono>
#include <cstring>

namespace q35 {
int batch_embed_f32_launch(const int8_t* q, const float* s, int D, const int32_t* token, const int32_t* prompt, int ldp,
                           const int32_t* plen, const int32_t* pos, float* h, fx_t* ss, fx_t* zero_ptr, int64_t zero_n,
                           uint32_t* err, int B, hipStream_t st);
int batch_argmax_groups(int V);
int batch_argmax_launch(const float* logits, int V, int B, float* pv, int32_t* pi, int32_t* token, int32_t* pos,
                        int32_t* hist, int ldh, hipStream_t st);
}  // namespace q35

struct q35_batch {
  q35_model* m = nullptr;
  int B = 0, tmax = 0;
  std::vector<int32_t> host_pos;  // per row
  std::map<std::string, q35_model::Buf> tensors;
  std::vector<void*> allocs;
  std::vector<float*> conv, rec, kc, vc;  // per layer, [B][...]
  float *h = nullptr;      // residual rows [B][hidden]
  float *proj = nullptr;   // q|k|v|z (linear) or q|k|v (full) projection rows [B][proj_n]
  float *gu = nullptr;     // gate | up rows [B][2 ffn], and a second copy for two split partials
  float *o_raw = nullptr, *attn = nullptr, *logits = nullptr, *pv = nullptr, *part = nullptr, *invf = nullptr;
  float* words = nullptr;  // counted split-K words of the projections (zero between launches)
  _Float16* split16 = nullptr;  // the lm_head's split input rows (hi, lo) of one row group
  q35::fx_t* ss = nullptr;   // RMSNorm statistics [2 layers + 1][B]
  q35::fx_t* gates = nullptr;  // DeltaNet gate sums [layers][B][32] (follows ss)
  int64_t proj_n = 0;
  size_t part_floats = 0, word_floats = 0;
  uint32_t *mb_ctr = nullptr, *gdn_ctr = nullptr;
  int32_t *token = nullptr, *pos = nullptr, *prompt = nullptr, *plen = nullptr, *hist = nullptr, *pi = nullptr;
  int32_t* pinned = nullptr;
  void* ws = nullptr;
  size_t ws_bytes = 0;
  hipStream_t own_stream = nullptr;
  hipGraphExec_t exec = nullptr;
  hipGraph_t graph = nullptr;
};

namespace q35 {
namespace {

constexpr int kRowGroup = 32;  // rows per projection launch
constexpr int kGateLd = 32;    // gate-sum row stride (2 x lin_heads <= 32)
constexpr int kMbCounters = 4096;

int balloc(q35_batch* b, const std::string& name, size_t bytes, void** out) {
  void* p = nullptr;
  hipError_t e = hipMalloc(&p, bytes < 256 ? 256 : bytes);
  if (e != hipSuccess) return fail(Q35_E_NOMEM, "hipMalloc(batch " + name + "): " + hipGetErrorString(e));
  b->allocs.push_back(p);
  b->tensors[name] = {p, bytes};
  *out = p;
  return Q35_OK;
}
template <class T>
int balloc_t(q35_batch* b, const std::string& name, size_t n, T** out) {
  void* p = nullptr;
  const int rc = balloc(b, name, n * sizeof(T), &p);
  *out = static_cast<T*>(p);
  return rc;
}

void bdestroy(q35_batch* b) {
  if (!b) return;
  if (b->exec) (void)hipGraphExecDestroy(b->exec);
  if (b->graph) (void)hipGraphDestroy(b->graph);
  for (void* p : b->allocs) (void)hipFree(p);
  if (b->pinned) (void)hipHostFree(b->pinned);
  if (b->own_stream) (void)hipStreamDestroy(b->own_stream);
  delete b;
}

hipStream_t bpick(q35_batch* b, void* s) { return s ? static_cast<hipStream_t>(s) : b->own_stream; }

// One decode step of all B rows (the launch sequence a graph captures).
int batch_step_launch(q35_batch* bt, hipStream_t st) {
  const q35_model* m = bt->m;
  const q35_dims& d = m->d;
  const int B = bt->B, H = d.hidden, F = d.ffn, NL = d.n_layers;
  const int nh = d.lin_heads, dk = d.lin_dk, dv = d.lin_dv;
  const int key_dim = nh * dk, vdim = nh * dv, conv_dim = 2 * key_dim + vdim, ldq = (int)bt->proj_n;
  const int ah = d.attn_heads, kvh = d.kv_heads, hd = d.head_dim;
  const int ldqg = ah * hd * 2, kvw = kvh * hd;
  int rc;
  std::vector<int32_t> gu_two((B + kRowGroup - 1) / kRowGroup, 0);  // gate|up left two partials
  // embedding rows + the first norm's statistic; clears every other statistic and gate sum
  if ((rc = batch_embed_f32_launch(m->embed.q, m->embed.s, H, bt->token, bt->prompt, bt->tmax, bt->plen, bt->pos, bt->h,
                                   bt->ss, bt->ss + B, (int64_t)2 * NL * B + (int64_t)NL * B * kGateLd,
                                   ws_counters(bt->ws) + kWsErrWord, B, st)))
    return rc;
  auto base = [&](MbCall& c, int M) {
    c.M = M; c.eps = d.eps;
    c.part = bt->part; c.part_floats = bt->part_floats; c.ctr = bt->mb_ctr; c.nctr = kMbCounters;
    c.words = bt->words; c.word_floats = bt->word_floats;
    c.err = ws_counters(bt->ws) + kWsErrWord;
    c.stream_order = true;  // the .qs copies
  };
  for (int l = 0; l < NL; ++l) {
    const q35_model::Layer& L = m->layers[l];
    const q35_model::MbLayer& W = m->mb[l];
    fx_t* ss_in = bt->ss + (size_t)(2 * l) * B;
    fx_t* ss_mid = bt->ss + (size_t)(2 * l + 1) * B;
    fx_t* ss_next = bt->ss + (size_t)(2 * l + 2) * B;
    fx_t* gates = bt->gates + (size_t)l * B * kGateLd;
    for (int r0 = 0; r0 < B; r0 += kRowGroup) {
      MbCall c;
      base(c, std::min(kRowGroup, B - r0));
      c.K = H; c.x = bt->h + (size_t)r0 * H; c.ldx = H; c.pro = MB_PRO_RMS; c.pw = L.in_norm; c.ss = ss_in + r0;
      float* pr = bt->proj + (size_t)r0 * ldq;
      if (!L.full) {
        c.nseg = 2;
        c.seg[0] = MbSeg{W.qkv.qs, W.qkv.s, pr, conv_dim, ldq, W.qkv.f};
        c.seg[1] = MbSeg{W.z.qs, W.z.s, pr + conv_dim, vdim, ldq, W.z.f};
        c.aux_wb = L.w_b; c.aux_wa = L.w_a; c.aux_nh = nh; c.aux_acc = gates + (size_t)r0 * kGateLd; c.aux_ldo = kGateLd;
      } else {
        c.nseg = 3;
        c.seg[0] = MbSeg{W.q.qs, W.q.s, pr, ldqg, ldq, W.q.f};
        c.seg[1] = MbSeg{W.k.qs, W.k.s, pr + ldqg, kvw, ldq, W.k.f};
        c.seg[2] = MbSeg{W.v.qs, W.v.s, pr + ldqg + kvw, kvw, ldq, W.v.f};
      }
      if ((rc = mb_launch(c, st))) return rc;
    }
    if (!L.full) {
      GdnCall g;
      g.qkv = bt->proj; g.ld_qkv = ldq; g.ba_f = gates; g.ld_bg = kGateLd; g.a_log = L.a_log; g.dt_bias = L.dt_bias;
      g.conv_state = bt->conv[l]; g.conv_w = L.conv_w; g.S = bt->rec[l]; g.o = bt->o_raw; g.ld_o = vdim;
      g.B = B; g.nh = nh; g.dk = dk; g.dv = dv; g.conv_k = d.conv_k; g.head_ctr = bt->gdn_ctr;
      if ((rc = gdn_step_launch(g, st))) return rc;
      for (int r0 = 0; r0 < B; r0 += kRowGroup) {
        MbCall c;
        base(c, std::min(kRowGroup, B - r0));
        c.K = vdim; c.x = bt->o_raw + (size_t)r0 * vdim; c.ldx = vdim; c.pro = MB_PRO_GATED;
        c.z = bt->proj + (size_t)r0 * ldq + conv_dim; c.ldz = ldq; c.group = dv; c.pw = L.norm_w;
        c.nseg = 1; c.seg[0] = MbSeg{W.out.qs, W.out.s, bt->h + (size_t)r0 * H, H, H};
        c.add = 1; c.ss_out = ss_mid + r0;
        if ((rc = mb_launch(c, st))) return rc;
      }
    } else {
      AttnCall a;
      a.qg = bt->proj; a.ld_qg = ldq; a.k = bt->proj + ldqg; a.v = bt->proj + ldqg + kvw; a.ld_kv = ldq;
      a.qnw = L.q_norm; a.knw = L.k_norm; a.eps = d.eps;
      a.rcos = m->rope_cos; a.rsin = m->rope_sin; a.rot = d.rot_dim;
      a.kc = bt->kc[l]; a.vc = bt->vc[l]; a.tmax = bt->tmax; a.pos = bt->pos;
      a.out = bt->attn; a.ld_out = ah * hd; a.B = B; a.nh = ah; a.nkv = kvh; a.hd = hd;
      if ((rc = attn_launch(a, bt->ws, bt->ws_bytes, st))) return rc;
      for (int r0 = 0; r0 < B; r0 += kRowGroup) {
        MbCall c;
        base(c, std::min(kRowGroup, B - r0));
        c.K = ah * hd; c.x = bt->attn + (size_t)r0 * ah * hd; c.ldx = ah * hd; c.pro = MB_PRO_PLAIN;
        c.nseg = 1; c.seg[0] = MbSeg{W.o.qs, W.o.s, bt->h + (size_t)r0 * H, H, H};
        c.add = 1; c.ss_out = ss_mid + r0;
        if ((rc = mb_launch(c, st))) return rc;
      }
    }
    for (int r0 = 0; r0 < B; r0 += kRowGroup) {
      MbCall c;
      base(c, std::min(kRowGroup, B - r0));
      c.K = H; c.x = bt->h + (size_t)r0 * H; c.ldx = H; c.pro = MB_PRO_RMS; c.pw = L.post_norm; c.ss = ss_mid + r0;
      float* gu = bt->gu + (size_t)r0 * 2 * F;
      c.nseg = 2;
      c.seg[0] = MbSeg{W.gate.qs, W.gate.s, gu, F, 2 * F, W.gate.f};
      c.seg[1] = MbSeg{W.up.qs, W.up.s, gu + F, F, 2 * F, W.up.f};
      // with two K splits the down projection sums the two partial copies itself (no hand-off)
      c.defer_stride = (int64_t)B * 2 * F;
      c.deferred_out = &gu_two[r0 / kRowGroup];
      if ((rc = mb_launch(c, st))) return rc;
    }
    for (int r0 = 0; r0 < B; r0 += kRowGroup) {
      MbCall c;
      base(c, std::min(kRowGroup, B - r0));
      c.K = F; c.x = bt->gu + (size_t)r0 * 2 * F; c.ldx = 2 * F; c.pro = MB_PRO_SWIGLU; c.swiglu_off = F;
      if (gu_two[r0 / kRowGroup]) {
        c.xsum = 2;
        c.xsstride = (int64_t)B * 2 * F;
      }
      c.nseg = 1; c.seg[0] = MbSeg{W.down.qs, W.down.s, bt->h + (size_t)r0 * H, H, H};
      c.add = 1; c.ss_out = ss_next + r0;
      if ((rc = mb_launch(c, st))) return rc;
    }
  }
  // final RMSNorm and the tied lm_head (model.rs:113-129) for every row
  for (int r0 = 0; r0 < B; r0 += kRowGroup)
    if ((rc = mb_lm_head_launch(m->embed_lm, m->embed_scale_t, d.vocab, H, bt->h + (size_t)r0 * H, H, m->final_norm, d.eps,
                                std::min(kRowGroup, B - r0), bt->split16, bt->invf, bt->logits + (size_t)r0 * d.vocab,
                                d.vocab, st)))
      return rc;
  return batch_argmax_launch(bt->logits, d.vocab, B, bt->pv, bt->pi, bt->token, bt->pos, bt->hist, bt->tmax, st);
}

int bcapture(q35_batch* b, hipStream_t st) {
  if (b->exec) return Q35_OK;
  Q35_HIP_TRY(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
  const int rc = batch_step_launch(b, st);
  hipGraph_t g = nullptr;
  const hipError_t e = hipStreamEndCapture(st, &g);
  if (rc != Q35_OK) { if (g) (void)hipGraphDestroy(g); return rc; }
  if (e != hipSuccess) return fail(Q35_E_HIP, std::string("hipStreamEndCapture: ") + hipGetErrorString(e));
  const hipError_t e2 = hipGraphInstantiate(&b->exec, g, nullptr, nullptr, 0);
  if (e2 != hipSuccess) { (void)hipGraphDestroy(g); return fail(Q35_E_HIP, std::string("hipGraphInstantiate: ") + hipGetErrorString(e2)); }
  b->graph = g;
  return Q35_OK;
}

int bstep(q35_batch* b, int mode, hipStream_t st) {
  for (int r = 0; r < b->B; ++r)
    if (b->host_pos[r] >= b->tmax) return fail(Q35_E_SHAPE, "batch_step: a row's cache is full (position == tmax)");
  if (mode == Q35_LAUNCH_GRAPH) {
    int rc = bcapture(b, st);
    if (rc) return rc;
    Q35_HIP_TRY(hipGraphLaunch(b->exec, st));
  } else {
    const int rc = batch_step_launch(b, st);
    if (rc) return rc;
  }
  for (int r = 0; r < b->B; ++r) b->host_pos[r] += 1;
  return Q35_OK;
}

}  // namespace

// MB-layout copies of every projection (once per model; the tile-major originals stay in use by
// the single-sequence paths).
int ensure_mb(q35_model* m, hipStream_t st) {
  if (!m->mb.empty()) return Q35_OK;
  std::vector<q35_model::MbLayer> mb(m->layers.size());
  int rc;
  // norm_w: the RMSNorm weights of the projection's prologue (its input is normalised in the
  // launch), for the direct path's split factors
  auto conv = [&](const q35_model::Q8& w, const std::string& name, q35_model::Mb& out,
                  const float* norm_w = nullptr) -> int {
    if (!w.q) return Q35_OK;
    int8_t* q = nullptr;
    float* s = nullptr;
    float* f = nullptr;
    float* smax = nullptr;
    int r;
    if ((r = dev_alloc_t(m, "mb." + name, (size_t)w.rows * w.cols, &q)) ||
        (r = dev_alloc_t(m, "mb." + name + ".scale", (size_t)w.rows * (w.cols / 64), &s)) ||
        (r = dev_alloc_t(m, "mb." + name + ".scale_max", 1, &smax)) ||
        (r = mb_convert_launch(w.q, w.s, w.rows, w.cols, q, s, st)) ||
        (r = mb_scale_max_launch(s, (int64_t)w.rows * (w.cols / 64), smax, st)))
      return r;
    if (norm_w && ((r = dev_alloc_t(m, "mb." + name + ".split", (size_t)(w.cols / 64), &f)) ||
                   (r = mb_split_factor_launch(s, w.rows, w.cols, norm_w, f, st))))
      return r;
    out.q = q;
    out.s = s;
    out.f = f;
    out.smax = smax;
    return Q35_OK;
  };
  for (size_t l = 0; l < m->layers.size(); ++l) {
    const q35_model::Layer& L = m->layers[l];
    const std::string p = "layers." + std::to_string(l) + ".";
    q35_model::MbLayer& o = mb[l];
    const float *nin = L.in_norm, *npost = L.post_norm;
    if ((rc = conv(L.qkv, p + "in_proj_qkv", o.qkv, nin)) || (rc = conv(L.z, p + "in_proj_z", o.z, nin)) ||
        (rc = conv(L.out, p + "out_proj", o.out)) || (rc = conv(L.q, p + "q_proj", o.q, nin)) ||
        (rc = conv(L.k, p + "k_proj", o.k, nin)) || (rc = conv(L.v, p + "v_proj", o.v, nin)) ||
        (rc = conv(L.o, p + "o_proj", o.o)) || (rc = conv(L.gate, p + "gate_proj", o.gate, npost)) ||
        (rc = conv(L.up, p + "up_proj", o.up, npost)) || (rc = conv(L.down, p + "down_proj", o.down)))
      return rc;
  }
  float* sT = nullptr;
  int8_t* lm = nullptr;
  if ((rc = dev_alloc_t(m, "mb.embed_scale_t", (size_t)m->d.vocab * (m->d.hidden / 64), &sT)) ||
      (rc = mb_scale_transpose_launch(m->embed.s, m->d.vocab, m->d.hidden, sT, st)) ||
      (rc = dev_alloc_t(m, "mb.embed_lm", mb_lm_table_bytes(m->d.vocab, m->d.hidden), &lm)) ||
      (rc = mb_lm_table_launch(m->embed.q, m->d.vocab, m->d.hidden, lm, st)))
    return rc;
  Q35_HIP_TRY(hipStreamSynchronize(st));
  m->mb = std::move(mb);
  m->embed_scale_t = sT;
  m->embed_lm = lm;
  return Q35_OK;
}

// The batched decode's copies of the projection weights in stream order (the prompt GEMMs keep
// reading the MB order): the bytes only; scales and split factors are shared with the MB copies.
int ensure_mb_stream(q35_model* m, hipStream_t st) {
  int rc;
  if ((rc = ensure_mb(m, st))) return rc;
  for (size_t l = 0; l < m->layers.size(); ++l) {
    const q35_model::Layer& L = m->layers[l];
    q35_model::MbLayer& o = m->mb[l];
    const std::string p = "mb.layers." + std::to_string(l) + ".";
    struct W { const q35_model::Q8* w; q35_model::Mb* mb; const char* name; };
    const W ws[] = {{&L.qkv, &o.qkv, "in_proj_qkv"}, {&L.z, &o.z, "in_proj_z"}, {&L.out, &o.out, "out_proj"},
                    {&L.q, &o.q, "q_proj"},         {&L.k, &o.k, "k_proj"},     {&L.v, &o.v, "v_proj"},
                    {&L.o, &o.o, "o_proj"},         {&L.gate, &o.gate, "gate_proj"}, {&L.up, &o.up, "up_proj"},
                    {&L.down, &o.down, "down_proj"}};
    for (const W& x : ws) {  // named as the MB copy (mb.layers.<l>.<proj>) + ".stream"
      if (!x.mb->q || x.mb->qs) continue;
      const size_t nb = (size_t)x.w->rows * x.w->cols;
      int8_t* qs = nullptr;
      if ((rc = dev_alloc_t(m, p + x.name + ".stream", nb, &qs)) || (rc = mb_stream_launch(x.mb->q, nb, qs, st)))
        return rc;
      x.mb->qs = qs;
    }
  }
  Q35_HIP_TRY(hipStreamSynchronize(st));
  return Q35_OK;
}

namespace {

// The prompt-path view of row r's state.
SeqView row_view(q35_batch* b, int r) {
  const q35_dims& d = b->m->d;
  const size_t conv_n = (size_t)(2 * d.lin_heads * d.lin_dk + d.lin_heads * d.lin_dv) * (d.conv_k - 1);
  const size_t rec_n = (size_t)d.lin_heads * d.lin_dk * d.lin_dv, kv_n = (size_t)d.kv_heads * b->tmax * d.head_dim;
  SeqView v;
  for (size_t l = 0; l < b->conv.size(); ++l) {
    v.conv.push_back(b->conv[l] ? b->conv[l] + r * conv_n : nullptr);
    v.rec.push_back(b->rec[l] ? b->rec[l] + r * rec_n : nullptr);
    v.kc.push_back(b->kc[l] ? b->kc[l] + r * kv_n : nullptr);
    v.vc.push_back(b->vc[l] ? b->vc[l] + r * kv_n : nullptr);
  }
  v.token = b->token + r;
  v.pos = b->pos + r;
  v.hist = b->hist + (size_t)r * b->tmax;
  v.tmax = b->tmax;
  return v;
}

}  // namespace
}  // namespace q35

namespace q35 {
namespace {
// Reads and clears the batch workspace's error word (after the stream is synchronised).
int bcheck(q35_batch* b) {
  uint32_t* word = ws_counters(b->ws) + kWsErrWord;
  uint32_t v = 0;
  Q35_HIP_TRY(hipMemcpy(&v, word, sizeof(v), hipMemcpyDeviceToHost));
  if (v == 0) return Q35_OK;
  const uint32_t zero = 0;
  Q35_HIP_TRY(hipMemcpy(word, &zero, sizeof(zero), hipMemcpyHostToDevice));
  if (v & kWsErrRange)
    return fail(Q35_E_RANGE, "batch step: a value for a fixed-point sum (a norm statistic or gate sum) was not "
                             "finite or |v| >= 2^31; the batch state is invalid until q35_batch_reset");
  if (v & kWsErrPos) return fail(Q35_E_SHAPE, "batch step: an attention position was outside the cache");
  return fail(Q35_E_HIP, "batch step: unknown error bits " + std::to_string(v));
}
}  // namespace
}  // namespace q35

using namespace q35;

extern "C" {

int q35_batch_create(q35_model* m, int32_t B, int32_t tmax, q35_batch** out) {
  if (!m || !out) return fail(Q35_E_ARG, "batch_create: null pointer");
  *out = nullptr;
  if (B < 1 || B > 256) return fail(Q35_E_SHAPE, "batch_create: B must be in [1, 256]");
  if (tmax < 1) return fail(Q35_E_SHAPE, "batch_create: tmax must be >= 1");
  if (tmax > m->tmax) return fail(Q35_E_SHAPE, "batch_create: tmax larger than the model's (its rotary tables)");
  q35_batch* b = new q35_batch();
  b->m = m; b->B = B; b->tmax = tmax;
  b->host_pos.assign(B, 0);
  auto bail = [&](int code) { bdestroy(b); return code; };
  if (hipStreamCreateWithFlags(&b->own_stream, hipStreamNonBlocking) != hipSuccess) return bail(fail(Q35_E_HIP, "hipStreamCreate failed"));
  const q35_dims& d = m->d;
  const int H = d.hidden, F = d.ffn, nh = d.lin_heads, vdim = nh * d.lin_dv, key_dim = nh * d.lin_dk;
  const int conv_dim = 2 * key_dim + vdim, ah = d.attn_heads, kvh = d.kv_heads, hd = d.head_dim;
  if (H % 512 || H > 2048 || F % 128 || vdim % 128 || (ah * hd) % 128 || kvh * hd % 64 || d.lin_dv > 128 ||
      2 * nh > kGateLd)
    return bail(fail(Q35_E_SHAPE, "batch_create: the batched kernels need a hidden size of 512, 1024, 1536 or 2048, ffn, "
                                  "the DeltaNet value width and the attention width multiples of 128, value heads of <= "
                                  "128 and <= 16 DeltaNet heads"));
  int rc;
  if ((rc = ensure_mb_stream(m, b->own_stream))) return bail(rc);
  for (int l = 0; l < d.n_layers; ++l) {
    const std::string p = "layers." + std::to_string(l) + ".";
    float *cs = nullptr, *rs = nullptr, *k = nullptr, *v = nullptr;
    if (!m->layers[l].full) {
      if ((rc = balloc_t(b, p + "linear_attn.conv_state", (size_t)B * conv_dim * (d.conv_k - 1), &cs)) ||
          (rc = balloc_t(b, p + "linear_attn.recurrent_state", (size_t)B * nh * d.lin_dk * d.lin_dv, &rs)))
        return bail(rc);
    } else {
      if ((rc = balloc_t(b, p + "self_attn.k_cache", (size_t)B * kvh * tmax * hd, &k)) ||
          (rc = balloc_t(b, p + "self_attn.v_cache", (size_t)B * kvh * tmax * hd, &v)))
        return bail(rc);
    }
    b->conv.push_back(cs); b->rec.push_back(rs); b->kc.push_back(k); b->vc.push_back(v);
  }
  b->proj_n = std::max<int64_t>(conv_dim + vdim, (int64_t)ah * hd * 2 + 2 * kvh * hd);
  const int G = batch_argmax_groups(d.vocab);
  const int NL = d.n_layers;
  // split-K partials: the largest any projection launch of this batch needs
  const int M0 = std::min(B, kRowGroup);
  const int shapes[6][2] = {{H, conv_dim + vdim}, {vdim, H}, {H, ah * hd * 2 + 2 * kvh * hd}, {ah * hd, H}, {H, 2 * F}, {F, H}};
  for (const auto& kn : shapes) {
    b->part_floats = std::max(b->part_floats, mb_part_floats(kn[1] / 64, kn[0], M0));
    b->word_floats = std::max(b->word_floats, mb_word_floats(kn[1] / 64, M0));
  }
  fx_t* stats = nullptr;
  if ((rc = balloc_t(b, "norm_stats", (size_t)(2 * NL + 1) * B + (size_t)NL * B * kGateLd, &stats))) return bail(rc);
  b->ss = stats;
  b->gates = stats + (size_t)(2 * NL + 1) * B;
  if ((rc = balloc_t(b, "h", (size_t)B * H, &b->h)) || (rc = balloc_t(b, "proj", (size_t)B * b->proj_n, &b->proj)) ||
      (rc = balloc_t(b, "gu", (size_t)2 * B * 2 * F, &b->gu)) || (rc = balloc_t(b, "lm_split16", (size_t)2 * kRowGroup * H, &b->split16)) ||
      (rc = balloc_t(b, "lm_invf", kRowGroup, &b->invf)) ||
      (rc = balloc_t(b, "partials", std::max<size_t>(b->part_floats, 64), &b->part)) ||
      (rc = balloc_t(b, "split_words", std::max<size_t>(b->word_floats, 64), &b->words)) ||
      (rc = balloc_t(b, "mb_counters", kMbCounters, &b->mb_ctr)) ||
      (rc = balloc_t(b, "gdn_counters", (size_t)B * nh, &b->gdn_ctr)) ||
      (rc = balloc_t(b, "o_raw", (size_t)B * vdim, &b->o_raw)) || (rc = balloc_t(b, "attn", (size_t)B * ah * hd, &b->attn)) ||
      (rc = balloc_t(b, "logits", (size_t)B * d.vocab, &b->logits)) || (rc = balloc_t(b, "argmax_pv", (size_t)B * G, &b->pv)) ||
      (rc = balloc_t(b, "argmax_pi", (size_t)B * G, &b->pi)) || (rc = balloc_t(b, "token", B, &b->token)) ||
      (rc = balloc_t(b, "pos", B, &b->pos)) || (rc = balloc_t(b, "prompt", (size_t)B * tmax, &b->prompt)) ||
      (rc = balloc_t(b, "plen", B, &b->plen)) || (rc = balloc_t(b, "hist", (size_t)B * tmax, &b->hist)))
    return bail(rc);
  b->ws_bytes = align256(attn_ws_bytes(B, ah, kvh, hd, tmax));
  if ((rc = balloc(b, "workspace", b->ws_bytes, &b->ws))) return bail(rc);
  if (hipHostMalloc(reinterpret_cast<void**>(&b->pinned), sizeof(int32_t) * 2 * B, hipHostMallocDefault) != hipSuccess)
    return bail(fail(Q35_E_NOMEM, "hipHostMalloc failed"));
  if (hipMemset(b->ws, 0, b->ws_bytes) != hipSuccess) return bail(fail(Q35_E_HIP, "workspace clear"));
  if ((rc = q35_batch_reset(b, nullptr))) return bail(rc);
  if (hipStreamSynchronize(b->own_stream) != hipSuccess) return bail(fail(Q35_E_HIP, "sync"));
  *out = b;
  return Q35_OK;
}

int q35_batch_destroy(q35_batch* b) {
  if (!b) return Q35_OK;
  (void)hipDeviceSynchronize();
  bdestroy(b);
  return Q35_OK;
}

int q35_batch_reset(q35_batch* b, void* stream) {
  if (!b) return fail(Q35_E_ARG, "batch_reset: null batch");
  hipStream_t st = bpick(b, stream);
  for (auto& kv : b->tensors)
    if (kv.first != "workspace") Q35_HIP_TRY(hipMemsetAsync(kv.second.p, 0, kv.second.bytes, st));
  Q35_HIP_TRY(hipMemsetAsync(ws_counters(b->ws) + kWsErrWord, 0, sizeof(uint32_t), st));
  std::fill(b->host_pos.begin(), b->host_pos.end(), 0);
  return Q35_OK;
}

int q35_batch_step(q35_batch* b, int32_t mode, void* stream) {
  if (!b) return fail(Q35_E_ARG, "batch_step: null batch");
  if (mode != Q35_LAUNCH_STREAM && mode != Q35_LAUNCH_GRAPH) return fail(Q35_E_ARG, "batch_step: mode must be stream or graph");
  return bstep(b, mode, bpick(b, stream));
}

int q35_batch_decode(q35_batch* b, int32_t n_steps, int32_t mode, void* stream) {
  if (!b) return fail(Q35_E_ARG, "batch_decode: null batch");
  if (n_steps < 0) return fail(Q35_E_SHAPE, "batch_decode: n_steps must be >= 0");
  for (int i = 0; i < n_steps; ++i) {
    const int rc = q35_batch_step(b, mode, stream);
    if (rc) return rc;
  }
  return Q35_OK;
}

int q35_batch_generate(q35_batch* b, const int32_t* prompts_host, const int32_t* lens_host, int32_t n_new,
                       int32_t* out_tokens_host, int32_t mode, double* decode_seconds_host, void* stream) {
  if (!b || !prompts_host || !lens_host || !out_tokens_host) return fail(Q35_E_ARG, "batch_generate: null pointer");
  const bool gemm_prefill = (mode & Q35_PREFILL_GEMM) != 0;
  mode &= ~Q35_PREFILL_GEMM;
  if (mode != Q35_LAUNCH_STREAM && mode != Q35_LAUNCH_GRAPH) return fail(Q35_E_ARG, "batch_generate: mode must be stream or graph");
  if (n_new < 0) return fail(Q35_E_SHAPE, "batch_generate: n_new must be >= 0");
  const int B = b->B, V = b->m->d.vocab;
  int maxlen = 0;
  int64_t off = 0;
  for (int r = 0; r < B; ++r) {
    if (lens_host[r] < 1) return fail(Q35_E_SHAPE, "batch_generate: every prompt needs >= 1 id");
    maxlen = std::max(maxlen, lens_host[r]);
    for (int i = 0; i < lens_host[r]; ++i)
      if (prompts_host[off + i] < 0 || prompts_host[off + i] >= V) return fail(Q35_E_ARG, "batch_generate: prompt id out of range");
    off += lens_host[r];
  }
  // decode-step feeding runs every row for max(len) + n_new steps; the prompt path exactly n_new
  const int steps = gemm_prefill ? n_new : maxlen - 1 + n_new + 1;
  std::vector<int32_t> start(B);
  for (int r = 0; r < B; ++r) {
    start[r] = b->host_pos[r];
    const int64_t need = (int64_t)start[r] + (gemm_prefill ? lens_host[r] + n_new : steps);
    if (need > b->tmax) return fail(Q35_E_SHAPE, "batch_generate: tmax too small");
  }
  hipStream_t st = bpick(b, stream);
  Q35_HIP_TRY(hipStreamSynchronize(st));
  off = 0;
  for (int r = 0; r < B; ++r) {
    Q35_HIP_TRY(hipMemcpy(b->prompt + (size_t)r * b->tmax + start[r], prompts_host + off, sizeof(int32_t) * lens_host[r],
                          hipMemcpyHostToDevice));
    off += lens_host[r];
    b->pinned[r] = start[r] + lens_host[r];
  }
  Q35_HIP_TRY(hipMemcpy(b->plen, b->pinned, sizeof(int32_t) * B, hipMemcpyHostToDevice));
  int rc;
  if (gemm_prefill) {
    q35_model* m = b->m;
    if ((rc = ensure_prefill(m, st))) return rc;
    for (int r = 0; r < B; ++r) {
      const SeqView v = row_view(b, r);
      for (int done = 0; done < lens_host[r];) {
        const int T = std::min(m->pf_cap, lens_host[r] - done);
        const int p0 = b->host_pos[r];
        if ((rc = prefill_pass(m, v, b->prompt + (size_t)r * b->tmax + p0, T, p0, st))) return rc;
        b->host_pos[r] += T;
        done += T;
      }
    }
  }
  if (mode == Q35_LAUNCH_GRAPH && (rc = bcapture(b, st))) return rc;
  Q35_HIP_TRY(hipStreamSynchronize(st));
  const auto t0 = std::chrono::steady_clock::now();
  for (int i = 0; i < steps; ++i)
    if ((rc = bstep(b, mode, st))) return rc;
  Q35_HIP_TRY(hipStreamSynchronize(st));
  const auto t1 = std::chrono::steady_clock::now();
  if ((rc = bcheck(b))) return rc;
  if (decode_seconds_host) *decode_seconds_host = std::chrono::duration<double>(t1 - t0).count();
  for (int r = 0; r < B; ++r)
    Q35_HIP_TRY(hipMemcpy(out_tokens_host + (size_t)r * (n_new + 1), b->hist + (size_t)r * b->tmax + start[r] + lens_host[r] - 1,
                          sizeof(int32_t) * (n_new + 1), hipMemcpyDeviceToHost));
  return Q35_OK;
}

int q35_batch_position(q35_batch* b, int32_t* pos_out_host) {
  if (!b || !pos_out_host) return fail(Q35_E_ARG, "batch_position: null pointer");
  for (int r = 0; r < b->B; ++r) pos_out_host[r] = b->host_pos[r];
  return Q35_OK;
}

int q35_batch_tensor(q35_batch* b, const char* name, void** dptr, size_t* bytes) {
  if (!b || !name || !dptr) return fail(Q35_E_ARG, "batch_tensor: null pointer");
  auto it = b->tensors.find(name);
  if (it == b->tensors.end()) return fail(Q35_E_ARG, std::string("batch_tensor: unknown tensor ") + name);
  *dptr = it->second.p;
  if (bytes) *bytes = it->second.bytes;
  return Q35_OK;
}

}  // extern "C"
