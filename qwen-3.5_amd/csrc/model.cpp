// The decoder model: weight upload, per-layer caches, the decode step as a fixed sequence of
// fused kernels, hipGraph capture of that sequence, and greedy generation.
//
// One decode step (TextForCausalLM::forward at seq_len 1, model.rs:27-84,113-129, plus the
// greedy argmax of main.rs:131) is 5 launches per layer + 1:
//   linear-attention layer: [input RMSNorm -> in_proj_qkv|in_proj_z|in_proj_b,a] -> DeltaNet step
//                           -> [gated RMSNorm -> out_proj -> +residual; conv-state shift]
//   full-attention layer:   [input RMSNorm -> q|k|v proj] -> attention -> [o_proj -> +residual]
//   MLP:                    [post RMSNorm -> gate|up] -> [SwiGLU -> down -> +residual]
//   head:                   [final RMSNorm -> lm_head -> argmax -> token, pos += 1]
// Matvec outputs are fixed-point accumulators (see fx_add); the residual stream h is one too, so
// residual adds are the projections' own atomics.  Accumulator hygiene: the q|k|v(|z) and gate
// accumulators are zero when a step starts; the gate|up launch clears the projection
// accumulators (read for the last time by the launch before it) and the next layer's first
// launch clears the gate|up accumulator (last read by down_proj).
// The token, the position, the prompt and the token history live in device memory, so the
// captured graph is replayed unchanged for every prompt token and every generated token.
#include "q35_host.h"

#include <atomic>
#include <chrono>
#include <cmath>
#include <cstring>
#include <map>
#include <vector>

#include "model_internal.h"

namespace q35 {

int dev_alloc(q35_model* m, const std::string& name, size_t bytes, void** out) {
  void* p = nullptr;
  hipError_t e = hipMalloc(&p, bytes < 256 ? 256 : bytes);
  if (e != hipSuccess) return fail(Q35_E_NOMEM, "hipMalloc(" + name + "): " + hipGetErrorString(e));
  m->allocs.push_back(p);
  m->tensors[name] = {p, bytes};
  *out = p;
  return Q35_OK;
}

hipStream_t pick(q35_model* m, void* s) { return s ? static_cast<hipStream_t>(s) : m->own_stream; }

namespace {

int launch_step(q35_model* m, hipStream_t st) {
  const q35_dims& d = m->d;
  const int H = d.hidden, F = d.ffn;
  const int nh = d.lin_heads, dk = d.lin_dk, dv = d.lin_dv;
  const int key_dim = nh * dk, vdim = nh * dv, conv_dim = 2 * key_dim + vdim, ldq = conv_dim + vdim;
  const int ah = d.attn_heads, kvh = d.kv_heads, hd = d.head_dim;
  const int ldqg = ah * hd * 2, LDa = ldqg + 2 * kvh * hd;
  int rc;
  for (int l = 0; l < d.n_layers; ++l) {
    const q35_model::Layer& L = m->layers[l];
    MvCall c;
    c.err = ws_counters(m->ws) + kWsErrWord;
    c.K = H; c.M = 1; c.xf = m->h; c.ldx = H; c.pw = L.in_norm; c.eps = d.eps;
    c.zero_ptr = m->acc_gu; c.zero_n = 2 * (int64_t)F;
    if (l == 0) {
      c.pro = PRO_EMBED_RMS;
      c.emb_q = m->embed.q; c.emb_s = m->embed.s; c.token = m->token; c.h_out = m->h;
      c.prompt = m->prompt; c.plen = m->plen; c.pos = m->pos;
    } else {
      c.pro = PRO_RMS;
    }
    if (!L.full) {
      c.nseg = 2;
      c.seg[0] = MvSeg{L.qkv.q, L.qkv.s, m->acc_proj, conv_dim, ldq, 1};
      c.seg[1] = MvSeg{L.z.q, L.z.s, m->acc_proj + conv_dim, vdim, ldq, 1};
      c.aux_wb = L.w_b; c.aux_wa = L.w_a; c.aux_nh = nh; c.aux_acc = m->acc_ba; c.aux_ldo = 2 * nh;
      if ((rc = mv_kn_launch(c, st))) return rc;
      GdnCall g;
      g.qkv_f = m->acc_proj; g.ld_qkv = ldq; g.ba_f = m->acc_ba; g.ld_bg = 2 * nh; g.a_log = L.a_log;
      g.dt_bias = L.dt_bias; g.conv_state = L.conv_state; g.conv_w = L.conv_w; g.S = L.rec; g.o = m->o_raw;
      g.ld_o = vdim; g.B = 1; g.nh = nh; g.dk = dk; g.dv = dv; g.conv_k = d.conv_k;
      if ((rc = gdn_step_launch(g, st))) return rc;
      MvCall c2;
      c2.err = ws_counters(m->ws) + kWsErrWord;
      c2.K = vdim; c2.M = 1; c2.nseg = 1;
      c2.seg[0] = MvSeg{L.out.q, L.out.s, m->h, H, H, 1};
      c2.pro = PRO_GATED; c2.x = m->o_raw; c2.ldx = vdim; c2.x2f = m->acc_proj + conv_dim; c2.ldx2 = ldq;
      c2.pw = L.norm_w; c2.group = dv; c2.eps = d.eps;
      c2.cs_state = L.conv_state; c2.cs_x = m->acc_proj; c2.cs_ch = conv_dim; c2.cs_ldx = ldq; c2.cs_B = 1;
      if ((rc = mv_kn_launch(c2, st))) return rc;
    } else {
      c.nseg = 3;
      c.seg[0] = MvSeg{L.q.q, L.q.s, m->acc_proj, ldqg, LDa, 1};
      c.seg[1] = MvSeg{L.k.q, L.k.s, m->acc_proj + ldqg, kvh * hd, LDa, 1};
      c.seg[2] = MvSeg{L.v.q, L.v.s, m->acc_proj + ldqg + kvh * hd, kvh * hd, LDa, 1};
      if ((rc = mv_kn_launch(c, st))) return rc;
      AttnCall a;
      a.qg_f = m->acc_proj; a.ld_qg = LDa; a.k_f = m->acc_proj + ldqg; a.v_f = m->acc_proj + ldqg + kvh * hd;
      a.ld_kv = LDa; a.qnw = L.q_norm; a.knw = L.k_norm; a.eps = d.eps;
      a.rcos = m->rope_cos; a.rsin = m->rope_sin; a.rot = d.rot_dim;
      a.kc = L.kc; a.vc = L.vc; a.tmax = m->tmax; a.pos = m->pos;
      a.out = m->attn; a.ld_out = ah * hd; a.B = 1; a.nh = ah; a.nkv = kvh; a.hd = hd;
      if ((rc = attn_launch(a, m->ws, m->ws_bytes, st))) return rc;
      MvCall c2;
      c2.err = ws_counters(m->ws) + kWsErrWord;
      c2.K = ah * hd; c2.M = 1; c2.nseg = 1;
      c2.seg[0] = MvSeg{L.o.q, L.o.s, m->h, H, H, 1};
      c2.pro = PRO_PLAIN; c2.x = m->attn; c2.ldx = ah * hd;
      if ((rc = mv_kn_launch(c2, st))) return rc;
    }
    MvCall c3;
    c3.err = ws_counters(m->ws) + kWsErrWord;
    c3.K = H; c3.M = 1; c3.nseg = 2;
    c3.seg[0] = MvSeg{L.gate.q, L.gate.s, m->acc_gu, F, 2 * F, 1};
    c3.seg[1] = MvSeg{L.up.q, L.up.s, m->acc_gu + F, F, 2 * F, 1};
    c3.pro = PRO_RMS; c3.xf = m->h; c3.ldx = H; c3.pw = L.post_norm; c3.eps = d.eps;
    c3.zero_ptr = m->acc_proj; c3.zero_n = m->acc_proj_n + 2 * nh;  // acc_ba follows acc_proj
    if ((rc = mv_kn_launch(c3, st))) return rc;
    MvCall c4;
    c4.err = ws_counters(m->ws) + kWsErrWord;
    c4.K = F; c4.M = 1; c4.nseg = 1;
    c4.seg[0] = MvSeg{L.down.q, L.down.s, m->h, H, H, 1};
    c4.pro = PRO_SWIGLU; c4.xf = m->acc_gu; c4.ldx = 2 * F; c4.swiglu_off = F;
    if ((rc = mv_kn_launch(c4, st))) return rc;
  }
  NkCall n;
  n.q = m->embed.q; n.s = m->embed.s; n.N = d.vocab; n.K = H; n.M = 1;
  n.xf = m->h; n.ldx = H; n.y = m->logits; n.ldy = d.vocab; n.pro = PRO_RMS; n.pw = m->final_norm; n.eps = d.eps;
  n.argmax_out = m->token; n.pos_inc = m->pos; n.hist = m->hist;
  return nk_launch(n, m->ws, m->ws_bytes, st);
}

size_t model_ws_bytes(const q35_dims& d, int tmax) {
  size_t m = attn_ws_bytes(1, d.attn_heads, d.kv_heads, d.head_dim, tmax);
  NkCall n;
  n.N = d.vocab; n.K = d.hidden;
  m = std::max(m, nk_ws_bytes(n));
  return align256(m);
}

// Device tables and scratch of the persistent step kernel.  A model whose shapes the kernel does
// not support still builds; launch mode 2 then reports why.
int setup_persistent(q35_model* m) {
  const q35_dims& d = m->d;
  m->step_grid = step_grid(d.hidden);
  m->step_rc = step_validate(d, m->tmax, m->step_grid);
  if (m->step_rc != Q35_OK) {
    m->step_msg = "persistent step unavailable: " + std::string(q35_last_error());
    return Q35_OK;
  }
  const int grid = m->step_grid, nh = d.lin_heads, kvh = d.kv_heads;
  const int nmax = step_att_nmax(grid, kvh);
  // second copies of every linear-attention layer's recurrent state and conv state
  const size_t rec_n = (size_t)nh * d.lin_dk * d.lin_dv, conv_n = (size_t)(2 * nh * d.lin_dk + nh * d.lin_dv) * 3;
  int n_lin = 0;
  for (int l = 0; l < d.n_layers; ++l) n_lin += m->layers[l].full ? 0 : 1;
  float* alt = nullptr;
  if (n_lin > 0) {
    const int rc0 = dev_alloc_t(m, "step_state_alt", (size_t)n_lin * (rec_n + conv_n), &alt);
    if (rc0) return rc0;
  }
  std::vector<StepLayer> hl(d.n_layers);
  for (int l = 0; l < d.n_layers; ++l) {
    const q35_model::Layer& L = m->layers[l];
    StepLayer& s = hl[l];
    s = StepLayer{};
    s.full = L.full ? 1 : 0;
    s.in_norm = L.in_norm; s.post_norm = L.post_norm;
    s.qkv_q = L.qkv.q; s.qkv_s = L.qkv.s; s.z_q = L.z.q; s.z_s = L.z.s; s.out_q = L.out.q; s.out_s = L.out.s;
    s.w_b = L.w_b; s.w_a = L.w_a; s.a_log = L.a_log; s.dt_bias = L.dt_bias; s.conv_w = L.conv_w; s.norm_w = L.norm_w;
    s.conv_state = L.conv_state; s.rec = L.rec;
    if (!L.full) {
      s.rec_alt = alt;
      s.conv_alt = alt + rec_n;
      alt += rec_n + conv_n;
    }
    s.q_q = L.q.q; s.q_s = L.q.s; s.k_q = L.k.q; s.k_s = L.k.s; s.v_q = L.v.q; s.v_s = L.v.s; s.o_q = L.o.q; s.o_s = L.o.s;
    s.q_norm = L.q_norm; s.k_norm = L.k_norm; s.kc = L.kc; s.vc = L.vc;
    s.gate_q = L.gate.q; s.gate_s = L.gate.s; s.up_q = L.up.q; s.up_s = L.up.s; s.down_q = L.down.q; s.down_s = L.down.s;
  }
  StepLayer* dl = nullptr;
  uint32_t *err = nullptr, *tokseq = nullptr;
  uint64_t *att_ml = nullptr, *att_o = nullptr, *argp = nullptr;
  fx_t *acc = nullptr, *h_sp = nullptr;
  // per layer: projection outputs | gate|up | in_proj_b|a sums (each sum on its own cache line)
  const int64_t gu_off = ((int64_t)m->acc_proj_n + 15) / 16 * 16, ba_off = gu_off + 2 * (int64_t)d.ffn;
  const int64_t acc_stride = ba_off + 2 * (int64_t)nh * kStepBaStride;
  const int64_t acc_par = (int64_t)d.n_layers * acc_stride;
  const int64_t h_n = (int64_t)2 * d.n_layers * 2 * d.hidden;  // per parity: one copy per residual stage
  int rc;
  if ((rc = dev_alloc_t(m, "step_layers", hl.size(), &dl)) ||
      (rc = dev_alloc_t(m, "step_error", 1, &err)) ||
      (rc = dev_alloc_t(m, "step_tokseq", 1, &tokseq)) ||
      (rc = dev_alloc_t(m, "step_acc", (size_t)2 * acc_par, &acc)) ||
      (rc = dev_alloc_t(m, "step_h", (size_t)2 * h_n, &h_sp)) ||
      (rc = dev_alloc_t(m, "step_attn_partial_ml", (size_t)kvh * nmax * 8, &att_ml)) ||
      (rc = dev_alloc_t(m, "step_attn_partial_o", (size_t)kvh * nmax * 4 * 256, &att_o)) ||
      (rc = dev_alloc_t(m, "step_argmax_partial", (size_t)2 * grid, &argp)))
    return rc;
  Q35_HIP_TRY(hipMemcpy(dl, hl.data(), hl.size() * sizeof(StepLayer), hipMemcpyHostToDevice));
  // counted accumulators, tags and the token counter start from zero (a model reset clears them again)
  Q35_HIP_TRY(hipMemset(err, 0, sizeof(uint32_t)));
  Q35_HIP_TRY(hipMemset(tokseq, 0, sizeof(uint32_t)));
  Q35_HIP_TRY(hipMemset(acc, 0, (size_t)2 * acc_par * sizeof(fx_t)));
  Q35_HIP_TRY(hipMemset(h_sp, 0, (size_t)2 * h_n * sizeof(fx_t)));
  Q35_HIP_TRY(hipMemset(att_ml, 0, (size_t)kvh * nmax * 8 * sizeof(uint64_t)));
  Q35_HIP_TRY(hipMemset(att_o, 0, (size_t)kvh * nmax * 4 * 256 * sizeof(uint64_t)));
  Q35_HIP_TRY(hipMemset(argp, 0, (size_t)2 * grid * sizeof(uint64_t)));
  StepArgs& a = m->step_args;
  a.layers = dl; a.n_layers = d.n_layers;
  a.H = d.hidden; a.F = d.ffn; a.V = d.vocab; a.nh = nh; a.dk = d.lin_dk; a.dv = d.lin_dv;
  a.key_dim = nh * d.lin_dk; a.vdim = nh * d.lin_dv; a.conv_dim = 2 * a.key_dim + a.vdim;
  a.ah = d.attn_heads; a.kvh = kvh; a.hd = d.head_dim; a.rot = d.rot_dim; a.tmax = m->tmax;
  a.eps = d.eps;
  a.qscale = powf((float)d.lin_dk, -0.5f);
  a.ascale = (float)(1.0 / sqrt((double)d.head_dim));
  step_plan(d, grid, a.mv);
  a.emb_q = m->embed.q; a.emb_s = m->embed.s; a.final_norm = m->final_norm;
  a.rope_cos = m->rope_cos; a.rope_sin = m->rope_sin;
  // The residual stream gets buffers of its own (a copy per residual stage and token parity) with
  // every 128-byte line on a 256-byte slot: each out / down / o stage adds 256 blocks' partials
  // into it, and 16 consecutive lines took those atomics about 1.8x as long as lines spread this way.
  a.h = h_sp; a.n_res = 2 * d.n_layers; a.acc = acc; a.acc_stride = acc_stride; a.acc_gu_off = gu_off; a.acc_ba_off = ba_off; a.acc_par = acc_par;
  a.att_ml = att_ml; a.att_o = att_o; a.att_nmax = nmax;
  a.logits = m->logits; a.argp = argp; a.tokseq = tokseq;
  a.token = m->token; a.pos = m->pos; a.prompt = m->prompt; a.plen = m->plen; a.hist = m->hist;
  a.tok_host = nullptr;
  a.ord = make_arg_order(d.vocab);
  a.err = err;
  a.ntok = 0;
  a.n_stop = 0;
  for (int j = 0; j < 4; ++j) a.stop_ids[j] = -1;
  return Q35_OK;
}

void destroy(q35_model* m) {
  if (!m) return;
  if (m->exec) (void)hipGraphExecDestroy(m->exec);
  if (m->graph) (void)hipGraphDestroy(m->graph);
  for (void* p : m->allocs) (void)hipFree(p);
  if (m->pinned) (void)hipHostFree(m->pinned);
  if (m->tok_stream) (void)hipHostFree(m->tok_stream);
  if (m->own_stream) (void)hipStreamDestroy(m->own_stream);
  delete m;
}

int capture(q35_model* m, hipStream_t st) {
  if (m->exec) return Q35_OK;
  Q35_HIP_TRY(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
  int rc = launch_step(m, st);
  hipGraph_t g = nullptr;
  hipError_t e = hipStreamEndCapture(st, &g);
  if (rc != Q35_OK) { if (g) (void)hipGraphDestroy(g); return rc; }
  if (e != hipSuccess) return fail(Q35_E_HIP, std::string("hipStreamEndCapture: ") + hipGetErrorString(e));
  e = hipGraphInstantiate(&m->exec, g, nullptr, nullptr, 0);
  if (e != hipSuccess) { (void)hipGraphDestroy(g); return fail(Q35_E_HIP, std::string("hipGraphInstantiate: ") + hipGetErrorString(e)); }
  m->graph = g;
  return Q35_OK;
}

const char* kStepFailed = "persistent step: a wait for another block's results timed out; the model state is invalid until q35_model_reset";
const char* kStepRange = "persistent step: a value to be accumulated in fixed point was not finite or |v| >= 2^22; the model state is invalid until q35_model_reset";

// n consecutive steps in one launch of the persistent kernel.  The barrier base is the number of
// barriers every earlier launch passed; a launch that fails (its error word set) leaves later
// launches as no-ops until a reset, so the base only has to be right while nothing failed.  With
// stop ids the launch may end early (a stopped launch still settles its barrier counters); the
// caller then re-reads the device position (sync_pos).
int persistent(q35_model* m, int n, hipStream_t st, const int32_t* stop_ids = nullptr, int n_stop = 0,
               bool stream_tokens = false) {
  if (m->step_rc != Q35_OK) return fail(m->step_rc, m->step_msg);
  if (m->step_failed) return fail(m->step_fail_code, m->step_fail_msg);
  if ((int64_t)m->host_pos + n > m->tmax) return fail(Q35_E_SHAPE, "model_step: cache full (position == tmax)");
  StepArgs a = m->step_args;
  a.ntok = n;
  a.tok_host = stream_tokens ? m->tok_stream_dev : nullptr;
  a.n_stop = n_stop;
  for (int j = 0; j < n_stop; ++j) a.stop_ids[j] = stop_ids[j];
  int rc = step_launch(a, m->step_grid, st);
  if (rc) return rc;
  m->host_pos += n;
  return Q35_OK;
}

}  // namespace

// ---- prompt path (TextForCausalLM::forward at seq_len > 1, model.rs:27-84,130-138)
constexpr int kPrefillCap = 1024;  // tokens per pass; longer prompts run in passes

SeqView model_view(q35_model* m) {
  SeqView v;
  for (const q35_model::Layer& L : m->layers) {
    v.conv.push_back(L.conv_state);
    v.rec.push_back(L.rec);
    v.kc.push_back(L.kc);
    v.vc.push_back(L.vc);
  }
  v.token = m->token;
  v.pos = m->pos;
  v.hist = m->hist;
  v.tmax = m->tmax;
  return v;
}

int ensure_prefill(q35_model* m, hipStream_t st) {
  int rc;
  {
    // Checked before anything is allocated or launched: the chunked delta rule's state and
    // output strides are fixed at 128 x 128 per head, and every prompt GEMM width (hidden, ffn,
    // conv_dim, value dim, 2 * attn_heads * 256, kv_heads * 256) must be a multiple of 128.
    const q35_dims& d = m->d;
    if (d.lin_dk != 128 || d.lin_dv != 128)
      return fail(Q35_E_SHAPE, "prompt path: linear-attention heads need dk = dv = 128");
    if (d.hidden % 128 || d.ffn % 128)
      return fail(Q35_E_SHAPE, "prompt path: hidden and ffn must be multiples of 128");
  }
  if ((rc = ensure_mb(m, st))) return rc;  // the projections' GEMMs read the MB copies
  if (m->pf_cap > 0) return Q35_OK;
  const q35_dims& d = m->d;
  const int H = d.hidden, F = d.ffn, nh = d.lin_heads, vdim = nh * d.lin_dv, key_dim = nh * d.lin_dk;
  const int conv_dim = 2 * key_dim + vdim, ah = d.attn_heads, kvh = d.kv_heads, hd = d.head_dim;
  const int cap = std::min(kPrefillCap, (m->tmax + kGdnChunk - 1) / kGdnChunk * kGdnChunk);
  const int ldy = std::max({conv_dim + vdim, ah * hd * 2 + 2 * kvh * hd, 2 * F});
  const int lda = std::max({vdim, ah * hd, F});
  const size_t nchunk = (size_t)cap / kGdnChunk;
  if ((rc = dev_alloc_t(m, "prefill_x", (size_t)cap * H, &m->pf_x)) ||
      (rc = dev_alloc_t(m, "prefill_xn", (size_t)cap * H, &m->pf_xn)) ||
      (rc = dev_alloc_t(m, "prefill_y", (size_t)cap * ldy, &m->pf_y)) ||
      (rc = dev_alloc_t(m, "prefill_a", (size_t)cap * lda, &m->pf_a)) ||
      (rc = dev_alloc_t(m, "prefill_core", (size_t)cap * vdim, &m->pf_core)) ||
      (rc = dev_alloc_t(m, "prefill_bg", (size_t)cap * 2 * nh, &m->pf_bg)) ||
      (rc = dev_alloc_t(m, "prefill_q", (size_t)cap * ah * hd, &m->pf_q)) ||
      (rc = dev_alloc_t(m, "prefill_scratch", (size_t)nh * nchunk * kGdnScratchPerChunk, &m->pf_scr)) ||
      (rc = dev_alloc_t(m, "prefill_partials", gemm_part_floats(cap, H), &m->pf_part)) ||
      (rc = dev_alloc_t(m, "prefill_gemm_aux", gemm_aux_floats(cap), &m->pf_aux)) ||
      (rc = dev_alloc_t(m, "prefill_act_max", (size_t)cap, &m->pf_act_max)))
    return rc;
  // gate | up interleaved by 64-column block for the fused SwiGLU: an MB copy keeps each column
  // block's records (K * 64 bytes) and scales (K floats) contiguous, so the two copies are
  // interleaved with strided copies
  for (size_t l = 0; l < m->layers.size(); ++l) {
    q35_model::MbLayer& W = m->mb[l];
    const int K = d.hidden, nb = F / 64;
    const std::string p = "layers." + std::to_string(l) + ".";
    int8_t* q = nullptr;
    float *s = nullptr, *smax = nullptr;
    if ((rc = dev_alloc_t(m, "mb." + p + "gate_up_interleaved", (size_t)2 * F * K, &q)) ||
        (rc = dev_alloc_t(m, "mb." + p + "gate_up_interleaved.scale", (size_t)2 * nb * K, &s)) ||
        (rc = dev_alloc_t(m, "mb." + p + "gate_up_interleaved.scale_max", 1, &smax)))
      return rc;
    const size_t qb = (size_t)K * 64, sb = (size_t)K * sizeof(float);
    Q35_HIP_TRY(hipMemcpy2DAsync(q, 2 * qb, W.gate.q, qb, qb, nb, hipMemcpyDeviceToDevice, st));
    Q35_HIP_TRY(hipMemcpy2DAsync(q + qb, 2 * qb, W.up.q, qb, qb, nb, hipMemcpyDeviceToDevice, st));
    Q35_HIP_TRY(hipMemcpy2DAsync(s, 2 * sb, W.gate.s, sb, sb, nb, hipMemcpyDeviceToDevice, st));
    Q35_HIP_TRY(hipMemcpy2DAsync(s + K, 2 * sb, W.up.s, sb, sb, nb, hipMemcpyDeviceToDevice, st));
    if ((rc = mb_scale_max_launch(s, (int64_t)2 * nb * K, smax, st))) return rc;
    W.gu.q = q;
    W.gu.s = s;
    W.gu.smax = smax;
  }
  m->pf_cap = cap;
  m->pf_ldy = ldy;
  m->pf_lda = lda;
  return Q35_OK;
}

// One pass over T <= pf_cap prompt tokens ids[0..T) at positions p0..p0+T-1: every layer on all
// T rows (GEMM projections on the matrix cores, conv + chunked delta rule, causal attention),
// then the final norm and the tied lm_head for the last row only (the only logits the greedy
// loop reads, main.rs:93-95), whose argmax goes to the token slot and hist[p0+T-1].
int prefill_pass(q35_model* m, const SeqView& v, const int32_t* ids, int T, int p0, hipStream_t st) {
  const q35_dims& d = m->d;
  const int H = d.hidden, F = d.ffn, nh = d.lin_heads, vdim = nh * d.lin_dv, key_dim = nh * d.lin_dk;
  const int conv_dim = 2 * key_dim + vdim, ah = d.attn_heads, kvh = d.kv_heads, hd = d.head_dim;
  const int LDY = m->pf_ldy;
  int rc;
  if ((rc = embed_launch(m->embed.q, m->embed.s, d.vocab, H, ids, T, m->pf_x, st))) return rc;
  // projections on the f16 matrix cores from the MB copies of the weights
  auto seg = [](const q35_model::Q8& w, const q35_model::Mb& mb, float* y, int ldy) {
    return GemmSeg{mb.q, mb.s, y, w.cols, Q35_KN_MB, ldy, mb.smax};
  };
  // The residual projections (out, o, down) leave their K splits in pf_part; the RMSNorm that next
  // reads the residual adds them in (pend splits).  The producers of the GEMM inputs write their
  // row maxima into the GEMMs' scratch (pf_aux).
  int pend = 1;
  const int64_t pstride = (int64_t)T * H;
  for (int l = 0; l < d.n_layers; ++l) {
    const q35_model::Layer& L = m->layers[l];
    const q35_model::MbLayer& W = m->mb[l];
    if ((rc = rms_rows_launch(m->pf_x, H, T, H, L.in_norm, d.eps, m->pf_xn, H, st, m->pf_aux, m->pf_part, pend,
                              pstride, H)))
      return rc;
    pend = 1;
    if (!L.full) {
      GemmCall g;
      g.x = m->pf_xn; g.ldx = H; g.M = T; g.K = H; g.nseg = 2;
      g.seg[0] = seg(L.qkv, W.qkv, m->pf_y, LDY);
      g.seg[1] = seg(L.z, W.z, m->pf_y + conv_dim, LDY);
      g.part = m->pf_part; g.part_floats = gemm_part_floats(m->pf_cap, d.hidden); g.aux = m->pf_aux; g.amax = m->pf_aux;
      if ((rc = gemm_launch(g, st))) return rc;
      if ((rc = gate_prompt_launch(m->pf_xn, H, T, H, L.w_b, L.w_a, L.a_log, L.dt_bias, nh, m->pf_bg, st))) return rc;
      GdnPrefill gp;
      gp.raw = m->pf_y; gp.ld_raw = LDY; gp.conv_state = v.conv[l]; gp.conv_state_out = v.conv[l];
      gp.conv_w = L.conv_w; gp.bg = m->pf_bg; gp.ld_bg = 2 * nh; gp.scr = m->pf_scr; gp.S = v.rec[l];
      gp.out = m->pf_core; gp.ld_out = vdim; gp.T = T; gp.nh = nh; gp.key_dim = key_dim;
      gp.nchunk = (T + kGdnChunk - 1) / kGdnChunk; gp.qscale = powf((float)d.lin_dk, -0.5f);
      if ((rc = gdn_prefill_launch(gp, st))) return rc;
      if ((rc = gated_norm_rows_launch(m->pf_core, vdim, m->pf_y + conv_dim, LDY, L.norm_w, T, nh, d.eps, m->pf_a, vdim, st,
                                       m->pf_aux)))
        return rc;
      GemmCall o;
      o.x = m->pf_a; o.ldx = vdim; o.M = T; o.K = vdim; o.nseg = 1; o.accumulate = 1;
      o.seg[0] = seg(L.out, W.out, m->pf_x, H);
      o.defer_reduce = 1; o.ksplit_out = &pend;
      o.part = m->pf_part; o.part_floats = gemm_part_floats(m->pf_cap, d.hidden); o.aux = m->pf_aux; o.amax = m->pf_aux;
      if ((rc = gemm_launch(o, st))) return rc;
    } else {
      const int qw = ah * hd * 2, kvw = kvh * hd;
      GemmCall g;
      g.x = m->pf_xn; g.ldx = H; g.M = T; g.K = H; g.nseg = 3;
      g.seg[0] = seg(L.q, W.q, m->pf_y, LDY);
      g.seg[1] = seg(L.k, W.k, m->pf_y + qw, LDY);
      g.seg[2] = seg(L.v, W.v, m->pf_y + qw + kvw, LDY);
      g.part = m->pf_part; g.part_floats = gemm_part_floats(m->pf_cap, d.hidden); g.aux = m->pf_aux; g.amax = m->pf_aux;
      if ((rc = gemm_launch(g, st))) return rc;
      AttnPrefill ap;
      ap.qg = m->pf_y; ap.ld_qg = LDY; ap.k = m->pf_y + qw; ap.v = m->pf_y + qw + kvw; ap.ld_kv = LDY;
      ap.qnw = L.q_norm; ap.knw = L.k_norm; ap.eps = d.eps; ap.rcos = m->rope_cos; ap.rsin = m->rope_sin;
      ap.rot = d.rot_dim; ap.kc = v.kc[l]; ap.vc = v.vc[l]; ap.tmax = v.tmax; ap.p0 = p0; ap.T = T; ap.nh = ah;
      ap.nkv = kvh; ap.qbuf = m->pf_q; ap.out = m->pf_a; ap.ld_out = ah * hd;
      ap.scale = (float)(1.0 / sqrt((double)hd));
      if ((rc = attn_prefill_launch(ap, st))) return rc;
      GemmCall o;
      o.x = m->pf_a; o.ldx = ah * hd; o.M = T; o.K = ah * hd; o.nseg = 1; o.accumulate = 1;
      o.seg[0] = seg(L.o, W.o, m->pf_x, H);
      o.defer_reduce = 1; o.ksplit_out = &pend;
      o.part = m->pf_part; o.part_floats = gemm_part_floats(m->pf_cap, d.hidden); o.aux = m->pf_aux;
      if ((rc = gemm_launch(o, st))) return rc;
    }
    if ((rc = rms_rows_launch(m->pf_x, H, T, H, L.post_norm, d.eps, m->pf_xn, H, st, m->pf_aux, m->pf_part, pend,
                              pstride, H, m->pf_act_max)))
      return rc;
    pend = 1;
    // gate | up (interleaved by column block) with the SwiGLU in the GEMM's epilogue: the rows
    // up * silu(gate) and their maxima (cleared by the RMSNorm above) come straight out of it
    GemmCall g;
    g.x = m->pf_xn; g.ldx = H; g.M = T; g.K = H; g.nseg = 1;
    g.seg[0] = GemmSeg{W.gu.q, W.gu.s, m->pf_y, 2 * F, Q35_KN_MB, LDY, W.gu.smax};
    g.part = m->pf_part; g.part_floats = gemm_part_floats(m->pf_cap, d.hidden); g.aux = m->pf_aux; g.amax = m->pf_aux;
    g.act = m->pf_a; g.ld_act = F; g.act_amax = m->pf_act_max;
    if ((rc = gemm_launch(g, st))) return rc;
    GemmCall dn;
    dn.x = m->pf_a; dn.ldx = F; dn.M = T; dn.K = F; dn.nseg = 1; dn.accumulate = 1;
    dn.seg[0] = seg(L.down, W.down, m->pf_x, H);
    dn.defer_reduce = l + 1 < d.n_layers ? 1 : 0;  // (the lm_head reads the last residual row)
    dn.ksplit_out = &pend;
    dn.part = m->pf_part; dn.part_floats = gemm_part_floats(m->pf_cap, d.hidden); dn.aux = m->pf_aux; dn.amax = m->pf_act_max;
      if ((rc = gemm_launch(dn, st))) return rc;
  }
  if ((rc = store_i32_launch(v.pos, p0 + T - 1, st))) return rc;
  NkCall n;
  n.q = m->embed.q; n.s = m->embed.s; n.N = d.vocab; n.K = H; n.M = 1;
  n.x = m->pf_x + (size_t)(T - 1) * H; n.ldx = H; n.y = m->logits; n.ldy = d.vocab; n.pro = PRO_RMS;
  n.pw = m->final_norm; n.eps = d.eps;
  n.argmax_out = v.token; n.pos_inc = v.pos; n.hist = v.hist;
  return nk_launch(n, m->ws, m->ws_bytes, st);
}

namespace {

// The n prompt ids already in m->prompt[host_pos..) through the prompt path, in passes.
int prefill(q35_model* m, int n, hipStream_t st) {
  int rc;
  if ((rc = ensure_prefill(m, st))) return rc;
  if ((int64_t)m->host_pos + n > m->tmax) return fail(Q35_E_SHAPE, "model_prefill: tmax too small");
  for (int done = 0; done < n;) {
    const int T = std::min(m->pf_cap, n - done);
    if ((rc = prefill_pass(m, model_view(m), m->prompt + m->host_pos, T, m->host_pos, st))) return rc;
    m->host_pos += T;
    done += T;
  }
  return Q35_OK;
}

// Reads the persistent kernel's sticky error word (synchronises the stream).
int check_persistent(q35_model* m, hipStream_t st) {
  if (m->step_rc != Q35_OK) return Q35_OK;
  if (m->step_failed) return fail(m->step_fail_code, m->step_fail_msg);
  Q35_HIP_TRY(hipMemcpyAsync(m->pinned + 8, m->step_args.err, sizeof(uint32_t), hipMemcpyDeviceToHost, st));
  Q35_HIP_TRY(hipStreamSynchronize(st));
  if (m->pinned[8] != 0) {
    m->step_failed = true;
    m->step_fail_msg = (m->pinned[8] & kStepErrRange) ? kStepRange : kStepFailed;
    m->step_fail_code = (m->pinned[8] & kStepErrRange) ? Q35_E_RANGE : Q35_E_HIP;
    return fail(m->step_fail_code, m->step_fail_msg);
  }
  return Q35_OK;
}

// Reads and clears the workspace error word of the stepwise launch modes (synchronises the
// stream): kWsErrRange, a fixed-point accumulator met a non-finite or out-of-range value;
// kWsErrPos, an attention position outside the cache.
int check_numeric(q35_model* m, hipStream_t st) {
  uint32_t* word = ws_counters(m->ws) + kWsErrWord;
  Q35_HIP_TRY(hipMemcpyAsync(m->pinned + 9, word, sizeof(uint32_t), hipMemcpyDeviceToHost, st));
  Q35_HIP_TRY(hipStreamSynchronize(st));
  const uint32_t v = (uint32_t)m->pinned[9];
  if (v == 0) return Q35_OK;
  m->pinned[9] = 0;
  Q35_HIP_TRY(hipMemcpyAsync(word, m->pinned + 9, sizeof(uint32_t), hipMemcpyHostToDevice, st));
  Q35_HIP_TRY(hipStreamSynchronize(st));
  if (v & kWsErrRange)
    return fail(Q35_E_RANGE, "decode step: a value for a fixed-point sum was not finite or |v| >= 2^31; it was "
                             "dropped and the model state is invalid until q35_model_reset");
  if (v & kWsErrPos) return fail(Q35_E_SHAPE, "decode step: an attention position was outside the cache");
  return fail(Q35_E_HIP, "decode step: unknown error bits " + std::to_string(v));
}

int step(q35_model* m, int use_graph, hipStream_t st) {
  if (m->host_pos >= m->tmax) return fail(Q35_E_SHAPE, "model_step: cache full (position == tmax)");
  if (use_graph == Q35_LAUNCH_PERSISTENT) return persistent(m, 1, st);
  if (use_graph) {
    int rc = capture(m, st);
    if (rc) return rc;
    Q35_HIP_TRY(hipGraphLaunch(m->exec, st));
  } else {
    int rc = launch_step(m, st);
    if (rc) return rc;
  }
  m->host_pos += 1;
  return Q35_OK;
}

}  // namespace
}  // namespace q35

namespace q35 {
namespace {

// The f32 values of one decoder tensor in the builder's layout (see TensorSpec).
using ValuesFn = std::function<int(const TensorSpec&, float*)>;

int build_model(const q35_dims* dp, uint64_t seed, int32_t tmax, const ValuesFn& values, q35_model** out) {
  if (!dp || !out) return fail(Q35_E_ARG, "model_create: null pointer");
  *out = nullptr;
  int rc = validate_dims(*dp);
  if (rc) return rc;
  if (tmax < 1) return fail(Q35_E_SHAPE, "model_create: tmax must be >= 1");
  q35_model* m = new q35_model();
  m->d = *dp; m->seed = seed; m->tmax = tmax;
  const q35_dims& d = m->d;
  auto bail = [&](int code) { destroy(m); return code; };
  if (hipStreamCreateWithFlags(&m->own_stream, hipStreamNonBlocking) != hipSuccess)
    return bail(fail(Q35_E_HIP, "hipStreamCreate failed"));

  // weights
  std::vector<float> host;
  std::vector<int8_t> hq;
  std::vector<float> hs;
  std::vector<int8_t> tq;
  std::vector<float> ts;
  for (const TensorSpec& t : model_specs(d)) {
    const size_t n = (size_t)t.rows * t.cols;
    host.resize(n);
    if ((rc = values(t, host.data()))) return bail(rc);
    if (t.kind == kF32) {
      float* p;
      if ((rc = dev_alloc_t(m, t.name, n, &p))) return bail(rc);
      if (hipMemcpy(p, host.data(), n * 4, hipMemcpyHostToDevice) != hipSuccess) return bail(fail(Q35_E_HIP, "upload " + t.name));
    } else {
      hq.resize(n);
      hs.resize(n / 64);
      quantize_q8f(host.data(), t.rows, t.cols, hq.data(), hs.data());
      size_t nq = n, ns = n / 64;
      if (t.kind == kQ8KN) {
        // projections are stored tile-major (Q35_KN_TILED) so that each split-K block of the
        // matvec streams one contiguous run of HBM
        nq = (size_t)q35_q8f_tiled_q_count((int32_t)t.rows, (int32_t)t.cols);
        ns = (size_t)q35_q8f_tiled_scale_count((int32_t)t.rows, (int32_t)t.cols);
        tq.resize(nq);
        ts.resize(ns);
        pack_kn_tiled(hq.data(), hs.data(), t.rows, t.cols, tq.data(), ts.data());
      }
      const int8_t* srcq = t.kind == kQ8KN ? tq.data() : hq.data();
      const float* srcs = t.kind == kQ8KN ? ts.data() : hs.data();
      int8_t* pq; float* ps;
      if ((rc = dev_alloc_t(m, t.name + ".q", nq, &pq))) return bail(rc);
      if ((rc = dev_alloc_t(m, t.name + ".scale", ns, &ps))) return bail(rc);
      if (hipMemcpy(pq, srcq, nq, hipMemcpyHostToDevice) != hipSuccess ||
          hipMemcpy(ps, srcs, ns * 4, hipMemcpyHostToDevice) != hipSuccess)
        return bail(fail(Q35_E_HIP, "upload " + t.name));
    }
  }
  std::vector<float>().swap(host);
  std::vector<int8_t>().swap(hq);
  std::vector<float>().swap(hs);
  std::vector<int8_t>().swap(tq);
  std::vector<float>().swap(ts);
  auto f32 = [&](const std::string& n) { return static_cast<const float*>(m->tensors.at(n).p); };
  auto q8 = [&](const std::string& n, int rows, int cols) {
    return q35_model::Q8{static_cast<const int8_t*>(m->tensors.at(n + ".q").p), f32(n + ".scale"), rows, cols};
  };
  const int H = d.hidden, F = d.ffn, nh = d.lin_heads, vdim = nh * d.lin_dv, key_dim = nh * d.lin_dk;
  const int conv_dim = 2 * key_dim + vdim, ah = d.attn_heads, kvh = d.kv_heads, hd = d.head_dim;
  m->embed = q8("embed_tokens", d.vocab, H);
  m->final_norm = f32("norm");
  m->layers.resize(d.n_layers);
  for (int l = 0; l < d.n_layers; ++l) {
    q35_model::Layer& L = m->layers[l];
    const std::string p = "layers." + std::to_string(l) + ".";
    L.full = is_full_layer(d, l);
    L.in_norm = f32(p + "input_layernorm");
    L.post_norm = f32(p + "post_attention_layernorm");
    if (!L.full) {
      const std::string a = p + "linear_attn.";
      L.qkv = q8(a + "in_proj_qkv", H, conv_dim);
      L.z = q8(a + "in_proj_z", H, vdim);
      L.out = q8(a + "out_proj", vdim, H);
      L.w_b = f32(a + "in_proj_b"); L.w_a = f32(a + "in_proj_a");
      L.a_log = f32(a + "a_log"); L.dt_bias = f32(a + "dt_bias");
      L.conv_w = f32(a + "conv1d"); L.norm_w = f32(a + "norm");
      if ((rc = dev_alloc_t(m, a + "conv_state", (size_t)conv_dim * (d.conv_k - 1), &L.conv_state))) return bail(rc);
      if ((rc = dev_alloc_t(m, a + "recurrent_state", (size_t)nh * d.lin_dk * d.lin_dv, &L.rec))) return bail(rc);
    } else {
      const std::string a = p + "self_attn.";
      L.q = q8(a + "q_proj", H, ah * hd * 2);
      L.k = q8(a + "k_proj", H, kvh * hd);
      L.v = q8(a + "v_proj", H, kvh * hd);
      L.o = q8(a + "o_proj", ah * hd, H);
      L.q_norm = f32(a + "q_norm"); L.k_norm = f32(a + "k_norm");
      if ((rc = dev_alloc_t(m, a + "k_cache", (size_t)kvh * tmax * hd, &L.kc))) return bail(rc);
      if ((rc = dev_alloc_t(m, a + "v_cache", (size_t)kvh * tmax * hd, &L.vc))) return bail(rc);
    }
    const std::string mp = p + "mlp.";
    L.gate = q8(mp + "gate_proj", H, F);
    L.up = q8(mp + "up_proj", H, F);
    L.down = q8(mp + "down_proj", F, H);
  }
  // rotary tables
  {
    std::vector<float> cs((size_t)tmax * d.rot_dim), sn((size_t)tmax * d.rot_dim);
    q35_rope_tables(&d, tmax, cs.data(), sn.data());
    if ((rc = dev_alloc_t(m, "rope_cos", cs.size(), &m->rope_cos))) return bail(rc);
    if ((rc = dev_alloc_t(m, "rope_sin", sn.size(), &m->rope_sin))) return bail(rc);
    if (hipMemcpy(m->rope_cos, cs.data(), cs.size() * 4, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(m->rope_sin, sn.data(), sn.size() * 4, hipMemcpyHostToDevice) != hipSuccess)
      return bail(fail(Q35_E_HIP, "upload rope tables"));
  }
  // activations, control scalars, workspace
  const int64_t proj_n = std::max<int64_t>(conv_dim + vdim, (int64_t)ah * hd * 2 + 2 * kvh * hd);
  m->acc_proj_n = proj_n;
  {  // acc_ba directly follows acc_proj so one side task clears both
    fx_t* both = nullptr;
    if ((rc = dev_alloc_t(m, "acc_proj", (size_t)(proj_n + 2 * nh), &both))) return bail(rc);
    m->acc_proj = both;
    m->acc_ba = both + proj_n;
  }
  if ((rc = dev_alloc_t(m, "h", H, &m->h)) || (rc = dev_alloc_t(m, "acc_gu", 2 * F, &m->acc_gu)) ||
      (rc = dev_alloc_t(m, "o_raw", vdim, &m->o_raw)) || (rc = dev_alloc_t(m, "attn", ah * hd, &m->attn)) ||
      (rc = dev_alloc_t(m, "logits", d.vocab, &m->logits)) || (rc = dev_alloc_t(m, "token", 1, &m->token)) ||
      (rc = dev_alloc_t(m, "pos", 1, &m->pos)) || (rc = dev_alloc_t(m, "prompt", tmax, &m->prompt)) ||
      (rc = dev_alloc_t(m, "plen", 1, &m->plen)) || (rc = dev_alloc_t(m, "hist", tmax, &m->hist)))
    return bail(rc);
  m->ws_bytes = model_ws_bytes(d, tmax);
  if ((rc = dev_alloc(m, "workspace", m->ws_bytes, &m->ws))) return bail(rc);
  if (hipHostMalloc(reinterpret_cast<void**>(&m->pinned), 64 * sizeof(int32_t), hipHostMallocDefault) != hipSuccess)
    return bail(fail(Q35_E_NOMEM, "hipHostMalloc failed"));
  if (hipHostMalloc(reinterpret_cast<void**>(&m->tok_stream), (size_t)tmax * sizeof(int32_t),
                    hipHostMallocMapped | hipHostMallocCoherent) != hipSuccess)
    return bail(fail(Q35_E_NOMEM, "hipHostMalloc (token stream) failed"));
  for (int q = 0; q < tmax; ++q) m->tok_stream[q] = -1;
  if (hipHostGetDevicePointer(reinterpret_cast<void**>(&m->tok_stream_dev), m->tok_stream, 0) != hipSuccess)
    return bail(fail(Q35_E_HIP, "hipHostGetDevicePointer (token stream) failed"));
  if (hipMemset(m->ws, 0, m->ws_bytes) != hipSuccess) return bail(fail(Q35_E_HIP, "workspace clear"));
  if ((rc = setup_persistent(m))) return bail(rc);
  if ((rc = q35_model_reset(m, nullptr))) return bail(rc);
  if (hipStreamSynchronize(m->own_stream) != hipSuccess) return bail(fail(Q35_E_HIP, "sync"));
  *out = m;
  return Q35_OK;
}

}  // namespace
}  // namespace q35

namespace q35 {
namespace {
// Greedy steps from position pe (the token slot holds the current token) until a stop id or
// max_new steps; see q35_model_generate_until.
int decode_until(q35_model* m, int32_t pe, int32_t max_new, const int32_t* stop_ids_host, int32_t n_stop,
                 int32_t* out_tokens_host, int32_t* n_out_host, int32_t use_graph, double* decode_seconds_host,
                 hipStream_t st);
}  // namespace
}  // namespace q35

using namespace q35;

extern "C" {

int q35_model_create_synthetic(const q35_dims* dp, uint64_t seed, int32_t tmax, q35_model** out) {
  return build_model(dp, seed, tmax, [seed](const TensorSpec& t, float* v) {
    synth_values(t, seed, v);
    return Q35_OK;
  }, out);
}

int q35_model_create_from_safetensors(const q35_dims* dp, const char* path, int32_t tmax, q35_model** out) {
  if (!dp || !path || !out) return fail(Q35_E_ARG, "model_create_from_safetensors: null pointer");
  int rc = Q35_OK;
  SafeTensorsPtr st = open_safetensors(path, &rc);
  if (rc) return rc;
  return build_model(dp, 0, tmax, [&st](const TensorSpec& t, float* v) { return safetensors_values(*st, t, v); }, out);
}

int q35_model_destroy(q35_model* m) {
  if (!m) return Q35_OK;
  (void)hipDeviceSynchronize();
  destroy(m);
  return Q35_OK;
}

int q35_model_reset(q35_model* m, void* stream) {
  if (!m) return fail(Q35_E_ARG, "model_reset: null model");
  hipStream_t st = pick(m, stream);
  for (auto& kv : m->tensors) {
    const std::string& n = kv.first;
    const bool state = n.find("conv_state") != std::string::npos || n.find("recurrent_state") != std::string::npos ||
                       n.find("k_cache") != std::string::npos || n.find("v_cache") != std::string::npos ||
                       n == "token" || n == "pos" || n == "plen" || n == "hist" || n == "prompt" ||
                       n == "h" || n == "acc_proj" || n == "acc_gu" || n == "step_h" || n == "step_acc" ||
                       n == "step_tokseq" || n == "step_argmax_partial" || n == "step_attn_partial_ml" ||
                       n == "step_attn_partial_o" || n == "step_error";
    if (state) Q35_HIP_TRY(hipMemsetAsync(kv.second.p, 0, kv.second.bytes, st));
  }
  Q35_HIP_TRY(hipMemsetAsync(ws_counters(m->ws) + kWsErrWord, 0, sizeof(uint32_t), st));
  m->host_pos = 0;
  m->step_failed = false;
  return Q35_OK;
}

int q35_model_set_token(q35_model* m, int32_t token, void* stream) {
  if (!m) return fail(Q35_E_ARG, "model_set_token: null model");
  if (token < 0 || token >= m->d.vocab) return fail(Q35_E_ARG, "model_set_token: token out of range");
  hipStream_t st = pick(m, stream);
  Q35_HIP_TRY(hipStreamSynchronize(st));
  m->pinned[0] = token;
  Q35_HIP_TRY(hipMemcpyAsync(m->token, m->pinned, sizeof(int32_t), hipMemcpyHostToDevice, st));
  Q35_HIP_TRY(hipStreamSynchronize(st));
  return Q35_OK;
}

int q35_model_step(q35_model* m, int32_t use_graph, void* stream) {
  if (!m) return fail(Q35_E_ARG, "model_step: null model");
  if (use_graph < Q35_LAUNCH_STREAM || use_graph > Q35_LAUNCH_PERSISTENT) return fail(Q35_E_ARG, "model_step: bad launch mode");
  return step(m, use_graph, pick(m, stream));
}

int q35_model_decode(q35_model* m, int32_t n_steps, int32_t mode, void* stream) {
  if (!m) return fail(Q35_E_ARG, "model_decode: null model");
  if (mode < Q35_LAUNCH_STREAM || mode > Q35_LAUNCH_PERSISTENT) return fail(Q35_E_ARG, "model_decode: bad launch mode");
  if (n_steps < 0) return fail(Q35_E_SHAPE, "model_decode: n_steps must be >= 0");
  if ((int64_t)m->host_pos + n_steps > m->tmax) return fail(Q35_E_SHAPE, "model_decode: tmax too small");
  hipStream_t st = pick(m, stream);
  if (mode == Q35_LAUNCH_PERSISTENT) return n_steps ? persistent(m, n_steps, st) : Q35_OK;
  for (int i = 0; i < n_steps; ++i) {
    const int rc = step(m, mode, st);
    if (rc) return rc;
  }
  return Q35_OK;
}

int q35_model_check(q35_model* m, void* stream) {
  if (!m) return fail(Q35_E_ARG, "model_check: null model");
  hipStream_t st = pick(m, stream);
  const int rc = check_persistent(m, st);
  return rc ? rc : check_numeric(m, st);
}

int q35_model_persistent_info(q35_model* m, int32_t* grid_out) {
  if (!m) return fail(Q35_E_ARG, "model_persistent_info: null model");
  if (grid_out) *grid_out = m->step_grid;
  if (m->step_rc != Q35_OK) return fail(m->step_rc, m->step_msg);
  return Q35_OK;
}

int q35_model_generate(q35_model* m, const int32_t* prompt_host, int32_t n_prompt, int32_t n_new,
                       int32_t* out_tokens_host, int32_t use_graph, int32_t readback_each,
                       double* decode_seconds_host, void* stream) {
  if (!m || !prompt_host || !out_tokens_host) return fail(Q35_E_ARG, "model_generate: null pointer");
  const bool gemm_prefill = (use_graph & Q35_PREFILL_GEMM) != 0;
  use_graph &= ~Q35_PREFILL_GEMM;
  if (use_graph < Q35_LAUNCH_STREAM || use_graph > Q35_LAUNCH_PERSISTENT) return fail(Q35_E_ARG, "model_generate: bad launch mode");
  if (n_prompt < 1 || n_new < 0) return fail(Q35_E_SHAPE, "model_generate: need n_prompt >= 1, n_new >= 0");
  const int32_t p0 = m->host_pos;
  if ((int64_t)p0 + n_prompt + n_new > m->tmax) return fail(Q35_E_SHAPE, "model_generate: tmax too small");
  for (int i = 0; i < n_prompt; ++i)
    if (prompt_host[i] < 0 || prompt_host[i] >= m->d.vocab) return fail(Q35_E_ARG, "model_generate: prompt id out of range");
  hipStream_t st = pick(m, stream);
  Q35_HIP_TRY(hipMemcpyAsync(m->prompt + p0, prompt_host, sizeof(int32_t) * n_prompt, hipMemcpyHostToDevice, st));
  Q35_HIP_TRY(hipStreamSynchronize(st));
  m->pinned[0] = p0 + n_prompt;
  Q35_HIP_TRY(hipMemcpyAsync(m->plen, m->pinned, sizeof(int32_t), hipMemcpyHostToDevice, st));
  Q35_HIP_TRY(hipStreamSynchronize(st));
  int rc;
  const bool pers = (use_graph == Q35_LAUNCH_PERSISTENT);
  if (use_graph == Q35_LAUNCH_GRAPH && (rc = capture(m, st))) return rc;
  if (gemm_prefill) {
    if ((rc = prefill(m, n_prompt, st))) return rc;
  } else if (pers) {
    if ((rc = persistent(m, n_prompt, st))) return rc;
  } else {
    for (int i = 0; i < n_prompt; ++i)
      if ((rc = step(m, use_graph, st))) return rc;
  }
  Q35_HIP_TRY(hipStreamSynchronize(st));
  const auto t0 = std::chrono::steady_clock::now();
  if (pers && !readback_each) {
    if ((rc = persistent(m, n_new, st))) return rc;
  } else {
    for (int i = 0; i < n_new; ++i) {
      if ((rc = step(m, use_graph, st))) return rc;
      if (readback_each) {  // main.rs:107: the token goes to the host every step
        Q35_HIP_TRY(hipMemcpyAsync(m->pinned, m->token, sizeof(int32_t), hipMemcpyDeviceToHost, st));
        Q35_HIP_TRY(hipStreamSynchronize(st));
      }
    }
  }
  Q35_HIP_TRY(hipStreamSynchronize(st));
  const auto t1 = std::chrono::steady_clock::now();
  if ((rc = pers ? check_persistent(m, st) : check_numeric(m, st))) return rc;
  if (decode_seconds_host) *decode_seconds_host = std::chrono::duration<double>(t1 - t0).count();
  Q35_HIP_TRY(hipMemcpy(out_tokens_host, m->hist + p0 + n_prompt - 1, sizeof(int32_t) * (n_new + 1), hipMemcpyDeviceToHost));
  return Q35_OK;
}

int q35_model_generate_until(q35_model* m, const int32_t* prompt_host, int32_t n_prompt, int32_t max_new,
                             const int32_t* stop_ids_host, int32_t n_stop, int32_t* out_tokens_host,
                             int32_t* n_out_host, int32_t use_graph, double* decode_seconds_host, void* stream) {
  if (!m || !prompt_host || !out_tokens_host || !n_out_host) return fail(Q35_E_ARG, "model_generate_until: null pointer");
  const bool gemm_prefill = (use_graph & Q35_PREFILL_GEMM) != 0;
  use_graph &= ~Q35_PREFILL_GEMM;
  if (n_stop < 0 || n_stop > Q35_MAX_STOP_IDS || (n_stop > 0 && !stop_ids_host))
    return fail(Q35_E_ARG, "model_generate_until: between 0 and 4 stop ids");
  if (use_graph < Q35_LAUNCH_STREAM || use_graph > Q35_LAUNCH_PERSISTENT) return fail(Q35_E_ARG, "model_generate_until: bad launch mode");
  if (n_prompt < 1 || max_new < 0) return fail(Q35_E_SHAPE, "model_generate_until: need n_prompt >= 1, max_new >= 0");
  const int32_t p0 = m->host_pos;
  if ((int64_t)p0 + n_prompt + max_new > m->tmax) return fail(Q35_E_SHAPE, "model_generate_until: tmax too small");
  for (int i = 0; i < n_prompt; ++i)
    if (prompt_host[i] < 0 || prompt_host[i] >= m->d.vocab) return fail(Q35_E_ARG, "model_generate_until: prompt id out of range");
  hipStream_t st = pick(m, stream);
  Q35_HIP_TRY(hipMemcpyAsync(m->prompt + p0, prompt_host, sizeof(int32_t) * n_prompt, hipMemcpyHostToDevice, st));
  Q35_HIP_TRY(hipStreamSynchronize(st));
  const int32_t pe = p0 + n_prompt;  // first generated position
  m->pinned[0] = pe;
  Q35_HIP_TRY(hipMemcpyAsync(m->plen, m->pinned, sizeof(int32_t), hipMemcpyHostToDevice, st));
  Q35_HIP_TRY(hipStreamSynchronize(st));
  int rc;
  const bool pers = (use_graph == Q35_LAUNCH_PERSISTENT);
  if (use_graph == Q35_LAUNCH_GRAPH && (rc = capture(m, st))) return rc;
  if (gemm_prefill) {
    if ((rc = prefill(m, n_prompt, st))) return rc;
  } else if (pers) {
    if ((rc = persistent(m, n_prompt, st))) return rc;
  } else {
    for (int i = 0; i < n_prompt; ++i)
      if ((rc = step(m, use_graph, st))) return rc;
  }
  return decode_until(m, pe, max_new, stop_ids_host, n_stop, out_tokens_host, n_out_host, use_graph,
                      decode_seconds_host, st);
}

int q35_model_decode_until(q35_model* m, int32_t max_new, const int32_t* stop_ids_host, int32_t n_stop,
                           int32_t* out_tokens_host, int32_t* n_out_host, int32_t use_graph,
                           double* decode_seconds_host, void* stream) {
  if (!m || !out_tokens_host || !n_out_host) return fail(Q35_E_ARG, "model_decode_until: null pointer");
  if (n_stop < 0 || n_stop > Q35_MAX_STOP_IDS || (n_stop > 0 && !stop_ids_host))
    return fail(Q35_E_ARG, "model_decode_until: between 0 and 4 stop ids");
  if (use_graph < Q35_LAUNCH_STREAM || use_graph > Q35_LAUNCH_PERSISTENT) return fail(Q35_E_ARG, "model_decode_until: bad launch mode");
  if (max_new < 0) return fail(Q35_E_SHAPE, "model_decode_until: max_new must be >= 0");
  if (m->host_pos < 1) return fail(Q35_E_SHAPE, "model_decode_until: nothing decoded yet (feed a prompt first)");
  if ((int64_t)m->host_pos + max_new > m->tmax) return fail(Q35_E_SHAPE, "model_decode_until: tmax too small");
  hipStream_t st = pick(m, stream);
  Q35_HIP_TRY(hipStreamSynchronize(st));
  m->pinned[0] = m->host_pos;  // generated steps from here on: the token slot feeds them
  Q35_HIP_TRY(hipMemcpyAsync(m->plen, m->pinned, sizeof(int32_t), hipMemcpyHostToDevice, st));
  Q35_HIP_TRY(hipStreamSynchronize(st));
  return decode_until(m, m->host_pos, max_new, stop_ids_host, n_stop, out_tokens_host, n_out_host, use_graph,
                      decode_seconds_host, st);
}

}  // extern "C"

namespace q35 {
namespace {

int decode_until(q35_model* m, int32_t pe, int32_t max_new, const int32_t* stop_ids_host, int32_t n_stop,
                 int32_t* out_tokens_host, int32_t* n_out_host, int32_t use_graph, double* decode_seconds_host,
                 hipStream_t st) {
  int rc;
  const bool pers = (use_graph == Q35_LAUNCH_PERSISTENT);
  if (use_graph == Q35_LAUNCH_GRAPH && (rc = capture(m, st))) return rc;
  Q35_HIP_TRY(hipStreamSynchronize(st));
  const auto t0 = std::chrono::steady_clock::now();
  int32_t produced = 0;
  if (pers) {
    // one launch; the kernel ends at the first generated step whose input token is a stop id
    if (max_new > 0 && (rc = persistent(m, max_new, st, stop_ids_host, n_stop))) return rc;
    Q35_HIP_TRY(hipMemcpyAsync(m->pinned, m->pos, sizeof(int32_t), hipMemcpyDeviceToHost, st));
    Q35_HIP_TRY(hipStreamSynchronize(st));
    if ((rc = check_persistent(m, st))) return rc;
    const int32_t dpos = m->pinned[0];
    if (dpos < pe || dpos > pe + max_new) return fail(Q35_E_HIP, "model_generate_until: device position out of range");
    produced = dpos - pe;
    m->host_pos = dpos;
  } else {
    // main.rs:105-110: read the token, stop on a stop id, else forward it
    for (; produced < max_new; ++produced) {
      Q35_HIP_TRY(hipMemcpyAsync(m->pinned, m->token, sizeof(int32_t), hipMemcpyDeviceToHost, st));
      Q35_HIP_TRY(hipStreamSynchronize(st));
      bool stop = false;
      for (int j = 0; j < n_stop; ++j) stop |= m->pinned[0] == stop_ids_host[j];
      if (stop) break;
      if ((rc = step(m, use_graph, st))) return rc;
    }
    Q35_HIP_TRY(hipStreamSynchronize(st));
  }
  const auto t1 = std::chrono::steady_clock::now();
  if (!pers && (rc = check_numeric(m, st))) return rc;
  if (decode_seconds_host) *decode_seconds_host = std::chrono::duration<double>(t1 - t0).count();
  Q35_HIP_TRY(hipMemcpy(out_tokens_host, m->hist + pe - 1, sizeof(int32_t) * (produced + 1), hipMemcpyDeviceToHost));
  *n_out_host = produced;
  return Q35_OK;
}

}  // namespace
}  // namespace q35

extern "C" {

int q35_model_prefill(q35_model* m, const int32_t* prompt_host, int32_t n_prompt, void* stream) {
  if (!m || !prompt_host) return fail(Q35_E_ARG, "model_prefill: null pointer");
  if (n_prompt < 1) return fail(Q35_E_SHAPE, "model_prefill: need n_prompt >= 1");
  const int32_t p0 = m->host_pos;
  if ((int64_t)p0 + n_prompt > m->tmax) return fail(Q35_E_SHAPE, "model_prefill: tmax too small");
  for (int i = 0; i < n_prompt; ++i)
    if (prompt_host[i] < 0 || prompt_host[i] >= m->d.vocab) return fail(Q35_E_ARG, "model_prefill: prompt id out of range");
  hipStream_t st = pick(m, stream);
  Q35_HIP_TRY(hipStreamSynchronize(st));
  Q35_HIP_TRY(hipMemcpyAsync(m->prompt + p0, prompt_host, sizeof(int32_t) * n_prompt, hipMemcpyHostToDevice, st));
  Q35_HIP_TRY(hipStreamSynchronize(st));
  m->pinned[0] = p0 + n_prompt;
  Q35_HIP_TRY(hipMemcpyAsync(m->plen, m->pinned, sizeof(int32_t), hipMemcpyHostToDevice, st));
  Q35_HIP_TRY(hipStreamSynchronize(st));
  return prefill(m, n_prompt, st);
}

int q35_model_decode_stream(q35_model* m, int32_t max_steps, const int32_t* stop_ids_host, int32_t n_stop, void* stream) {
  if (!m) return fail(Q35_E_ARG, "model_decode_stream: null model");
  if (n_stop < 0 || n_stop > Q35_MAX_STOP_IDS || (n_stop > 0 && !stop_ids_host))
    return fail(Q35_E_ARG, "model_decode_stream: between 0 and 4 stop ids");
  if (max_steps < 0) return fail(Q35_E_SHAPE, "model_decode_stream: max_steps must be >= 0");
  if ((int64_t)m->host_pos + max_steps > m->tmax) return fail(Q35_E_SHAPE, "model_decode_stream: tmax too small");
  if (n_stop > 0 && m->host_pos < 1) return fail(Q35_E_SHAPE, "model_decode_stream: nothing decoded yet (feed a prompt first)");
  hipStream_t st = pick(m, stream);
  m->stream_p0 = m->host_pos;
  m->stream_max = max_steps;
  if (max_steps == 0) return Q35_OK;
  if (n_stop > 0) {  // generated steps from here on: a stop id among their input tokens ends the launch
    Q35_HIP_TRY(hipStreamSynchronize(st));
    m->pinned[0] = m->host_pos;
    Q35_HIP_TRY(hipMemcpyAsync(m->plen, m->pinned, sizeof(int32_t), hipMemcpyHostToDevice, st));
    Q35_HIP_TRY(hipStreamSynchronize(st));
  }
  // the slots this launch writes start at -1 (host stores, before the launch is enqueued; an
  // earlier launch still running writes only slots below host_pos)
  volatile int32_t* slot = m->tok_stream;
  for (int32_t q = m->host_pos; q < m->host_pos + max_steps; ++q) slot[q] = -1;
  std::atomic_thread_fence(std::memory_order_seq_cst);
  return persistent(m, max_steps, st, stop_ids_host, n_stop, true);
}

int q35_model_stream_end(q35_model* m, int32_t* n_steps_out, void* stream) {
  if (!m) return fail(Q35_E_ARG, "model_stream_end: null model");
  hipStream_t st = pick(m, stream);
  int rc;
  if (m->stream_max > 0) {
    Q35_HIP_TRY(hipMemcpyAsync(m->pinned, m->pos, sizeof(int32_t), hipMemcpyDeviceToHost, st));
    Q35_HIP_TRY(hipStreamSynchronize(st));
    if ((rc = check_persistent(m, st))) return rc;
    const int32_t dpos = m->pinned[0];
    if (dpos < m->stream_p0 || dpos > m->stream_p0 + m->stream_max)
      return fail(Q35_E_HIP, "model_stream_end: device position out of range");
    m->host_pos = dpos;  // (a launch that met a stop id ran fewer steps than it was given)
  } else {
    Q35_HIP_TRY(hipStreamSynchronize(st));
  }
  if (n_steps_out) *n_steps_out = m->host_pos - m->stream_p0;
  m->stream_max = 0;
  return Q35_OK;
}

const int32_t* q35_model_token_stream(q35_model* m) { return m ? m->tok_stream : nullptr; }

int q35_model_position(q35_model* m, int32_t* pos_out) {
  if (!m || !pos_out) return fail(Q35_E_ARG, "model_position: null pointer");
  *pos_out = m->host_pos;
  return Q35_OK;
}

int q35_model_tensor(q35_model* m, const char* name, void** dptr, size_t* bytes) {
  if (!m || !name || !dptr) return fail(Q35_E_ARG, "model_tensor: null pointer");
  auto it = m->tensors.find(name);
  if (it == m->tensors.end()) return fail(Q35_E_ARG, std::string("model_tensor: unknown tensor ") + name);
  *dptr = it->second.p;
  if (bytes) *bytes = it->second.bytes;
  return Q35_OK;
}

}  // extern "C"
