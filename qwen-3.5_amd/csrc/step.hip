// Persistent decode step: the whole TextForCausalLM forward at seq_len 1 (model.rs:27-84,
// 113-129) plus the greedy argmax (main.rs:131), for `ntok` consecutive tokens, in ONE launch.
//
// Why: a decode step streams ~2 GB of Q8F weights through ~100 dependent stages.  As separate
// kernels every stage boundary costs a launch gap plus a ramp-up/drain with HBM idle; here the
// grid is one co-resident block per CU (cooperative launch) that runs every stage.  Each block
// issues the weight loads of its next stage as soon as it has published its part of the current
// one, so the weight stream of stage s+1 overlaps the tail of stage s.
//
// Stages per token (each consumes the outputs of the one before):
//   linear-attention layer: qkvz  [RMSNorm(h) or embedding -> in_proj_qkv|in_proj_z; in_proj_b|a]
//                           out   [conv1d + SiLU, l2norm, gated delta rule step, gated
//                                  RMSNorm(o, z) -> out_proj -> +h]
//   full-attention layer:   qkv   [RMSNorm(h) or embedding -> q|gate, k, v]
//                           attn  [q/k RMSNorm, RoPE, KV append, split-T softmax partials]
//                           o     [merge attention partials * sigmoid(gate) -> o_proj -> +h]
//   MLP:                    gu    [RMSNorm(h) -> gate|up]
//                           down  [SwiGLU -> down_proj -> +h]
//   head:                   lm    [final RMSNorm -> tied lm_head -> logits, block argmax]
// The next token's first stage reduces the block argmaxes (or takes the prompt id).
//
// Matvec stages use the split-K decomposition of the standalone KN kernel on the tile-major
// layout: an item is (256-column tile, kch rows); 512 threads = 16 column groups x 32 row
// groups, every lane holds up to 16 rows (16-byte loads) of its item in registers; partial
// sums go through LDS and then 64-bit fixed-point atomics (fx_add) into the output.  Every
// value exchanged between blocks inside the launch is written with agent-scope atomics or
// sc1 stores and read with sc1 loads (no stale per-CU / per-XCD cache lines).
//
// Synchronisation: there is no grid barrier.  Every value one block hands to another carries its
// own completion state, and the consumer spins on the data itself:
//  * split-K accumulators (residual stream, projection outputs) are counted fixed point: each
//    contribution adds value * 2^32 + 2^56, so the top byte counts contributions (modulo 256) and
//    a word is complete when it holds the number of contributions its stage makes (every item
//    of a stage adds once to each column of its tile, so that number is the stage's chunk count);
//  * values that are stored rather than added (attention partials, argmax partials) carry a tag
//    unique to the token and layer that wrote them.
// A consumer issues its next stage's weight loads, then its inputs; when an input is not yet
// complete, the wave polls one incomplete word (one load per poll) and then re-reads.  That is
// one memory round trip from the last producer's add to the consumer's data, where an arrive
// (after the adds' acknowledgements), a barrier poll and a separate input read took three.
// Ordering of the plain stores that are not tagged (KV rows, DeltaNet states, the clearing of
// the next token's accumulators) follows from the data: none is read within the token that
// wrote it, a block waits for all its stores to complete before it publishes its argmax partial
// of the token, and every reader in a later token first observes all partials (or data made by
// blocks that did).  No counted word is ever added to
// after its readers' count is reached: accumulators are not re-used within a token (one set per
// layer), and the residual stream has a copy per residual stage, which receives the previous
// copy once (the stage's first-chunk items add it with their contributions) and that stage's
// contributions (a reader that falls behind would otherwise find its words already past its
// count; the carry costs no extra atomic).  So a count never
// exceeds 1 + 120 and never wraps.  The lm stage of token t clears the set of token t + 1 (token
// parity); every block reads all argmax partials of token t before it starts token t + 1, so the
// clearing is complete before any block adds into that set.
// Every wait is bounded: on time-out a block sets the sticky error word and returns; other
// blocks poll the word while they wait and return too, so the grid always drains; a later
// launch that finds the word set returns at entry.  The launch is cooperative only so that all
// blocks are co-resident (a block that waits needs its producers running).
#include "q35_internal.h"

#include <algorithm>
#include <climits>

namespace q35 {

namespace {

constexpr int kT = kStepThreads;  // 512
constexpr int kNW = kT / 64;      // waves per block
constexpr int kTile = 256;
constexpr int kRG = kT / 16;      // matvec row groups (16 lanes cover a 256-byte tile row)
constexpr int kU = 13;            // rows per lane per item (the register budget)
constexpr int kKch = kRG * kU;    // rows per item, at most 416
constexpr int kRmsRegs = 8;       // RMSNorm prologue: K <= 8 * 512
constexpr uint32_t kSpin = 1u << 21;  // polls before a wait gives up (seconds)
constexpr int kHd = 256;          // attention head dim
constexpr int kMaxRep = 4;        // query heads per kv head
constexpr int kMaxChunk = 256;    // cached tokens per attention item (x 128 chunks: 32768 tokens)
constexpr int kMaxChunkLong = 2048;  // the long-context build of the kernel: 262144 tokens
constexpr int kMinChunk = 8;
constexpr int kMaxNmax = 256;     // attention chunks per kv head
constexpr int kMaxTouch = 8;      // norm groups / heads one matvec item's rows can span
constexpr int kDk = 128;          // DeltaNet key head dim
constexpr int kDv = 128;          // DeltaNet value head dim
constexpr int kGdnG = kStepThreads / kDv;  // DeltaNet state row groups (4)
constexpr int kGdnR = kDk / kGdnG;         // DeltaNet state rows per thread (32)
constexpr int kSmem = 12288;      // floats of LDS shared by all stages (48 KB)
constexpr int kMergeB = 16;       // attention-merge partials loaded per batch
constexpr int kArgIdxBits = 18;   // argmax partial: index bits (vocabulary < 2^18)
constexpr uint32_t kArgNone = (1u << kArgIdxBits) - 1;

// LDS carve-up (float offsets)
constexpr int kXs = 0;                  // matvec x chunk [kKch]
constexpr int kRed = kXs + kKch;        // matvec wave partials [kNW][kTile]; prologue scratch [kRG][kTile]
static_assert(kRed + kRG * kTile <= kSmem, "LDS");
static_assert(512 + 2 * kT + kDv <= kRG * kTile, "DeltaNet scratch fits in kRed");
static_assert(kKch <= kT, "one x element per thread in the gated / attention prologues");
static_assert(kMaxTouch * kMaxNmax + kT + kMaxTouch <= kRG * kTile, "attention merge scratch fits in kRed");
// LDS of the attention items of a build whose items hold up to mc cached tokens: q, k, v rows,
// RoPE scratch, scores [kMaxRep][mc], the waves' outputs, m and l; the stage LDS of that build
constexpr int attn_smem(int mc) { return (2 * kMaxRep + 3) * kHd + kMaxRep * mc + kNW * kMaxRep * kHd + 2 * kMaxRep; }
constexpr int smem_for(int mc) { return attn_smem(mc) <= kSmem ? kSmem : (attn_smem(mc) + 255) / 256 * 256; }
static_assert(attn_smem(kMaxChunk) <= kSmem, "attention item scratch fits in the stage LDS");

// threadIdx.x / blockIdx.x read through an empty asm: every use is then loop-variant, so each
// stage recomputes its per-thread address arithmetic instead of the compiler hoisting it out of
// the token / layer loops and keeping it live (spilled to scratch) across the whole kernel.
Q35_DEV int tix() {
  int t = threadIdx.x;
  asm volatile("" : "+v"(t));
  return t;
}
Q35_DEV int bix() {
  int b = blockIdx.x;
  asm volatile("" : "+s"(b));
  return b;
}

struct Shared {
  float* smem;
  float* shs;  // [kNW] block sums
  float* shv;  // [kNW] argmax values
  int* shi;    // [kNW] argmax indices
  int* fail;   // set by any wave whose wait failed (time-out or error word); read after a barrier
};

// ------------------------------------------------------------------ block reductions
// lead_sync = false: the caller guarantees a workgroup barrier between the previous block_sum's
// reads of shs and this call.
Q35_DEV float block_sum(float v, float* shs, bool lead_sync = true) {
  v = wave_sum(v);
  const int lane = tix() & 63, wid = tix() >> 6;
  if (lead_sync) __syncthreads();
  if (lane == 0) shs[wid] = v;
  __syncthreads();
  static_assert(kNW == 8, "two 16-byte reads");
  const float4 a = *reinterpret_cast<const float4*>(shs), b = *reinterpret_cast<const float4*>(shs + 4);
  return ((((((a.x + a.y) + a.z) + a.w) + b.x) + b.y) + b.z) + b.w;
}

Q35_DEV void block_argmax(float& v, int& i, float* shv, int* shi, const ArgOrder& o) {
  wave_argmax(v, i, o);
  const int lane = tix() & 63, wid = tix() >> 6;
  __syncthreads();
  if (lane == 0) { shv[wid] = v; shi[wid] = i; }
  __syncthreads();
  v = shv[0];
  i = shi[0];
#pragma unroll
  for (int w = 1; w < kNW; ++w)
    if (argmax_better(shv[w], shi[w], v, i, o)) { v = shv[w]; i = shi[w]; }
}

Q35_DEV float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

Q35_DEV uint64_t ld_agent64(const uint64_t* p) {
  return __hip_atomic_load((Q35_GLOBAL uint64_t*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
Q35_DEV void st_agent64(uint64_t* p, uint64_t v) {
  __hip_atomic_store((Q35_GLOBAL uint64_t*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ------------------------------------------------------------------ counted words and tags
// A counted accumulator word: two's complement value * 2^32 plus (contributions mod 256) * 2^56.
// With |value| < 2^23 the word minus e * 2^56 lies in (-2^55, 2^55) exactly when it holds e
// contributions, and it is then the value itself.
Q35_DEV uint64_t cnt_of(uint32_t e) { return (uint64_t)e << 56; }
Q35_DEV bool fxc_ok(fx_t w, uint32_t e) { return ((uint64_t)w - cnt_of(e) + (1ull << 55)) < (1ull << 56); }
Q35_DEV float fxc_val(fx_t w, uint32_t e) { return from_fx((fx_t)((uint64_t)w - cnt_of(e))); }

Q35_DEV void raise_err(const StepArgs& a, uint32_t bit) {
  __hip_atomic_fetch_or((Q35_GLOBAL uint32_t*)a.err, bit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// One contribution v to a counted word (fire-and-forget agent-scope atomic).  A value that is not
// finite or whose magnitude reaches 2^22 (the total must stay below 2^23) is not added: it sets
// the range bit of the error word, which the host reports after the launch.  `base` (a fixed-point
// value, exact) is added with it.
Q35_DEV void fxc_add(const StepArgs& a, fx_t* p, float v, fx_t base = 0) {
  if (!fxc_addable(v)) {
    raise_err(a, kStepErrRange);
    v = 0.f;
  }
  __hip_atomic_fetch_add((Q35_GLOBAL unsigned long long*)p, (unsigned long long)to_fx(v) + (uint64_t)base + (1ull << 56),
                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Tagged f32 (attention partials): (tag << 32) | bits
Q35_DEV uint64_t tagged(float v, uint32_t tag) { return ((uint64_t)tag << 32) | __float_as_uint(v); }
Q35_DEV bool tag_ok(uint64_t w, uint32_t tag) { return (uint32_t)(w >> 32) == tag; }
Q35_DEV float tag_val(uint64_t w) { return __uint_as_float((uint32_t)w); }
// Tag of the attention partials of token ti, layer l (never 0, the value of a cleared buffer,
// for the first tokens after a reset)
Q35_DEV uint32_t att_tag(const StepArgs& a, uint32_t ti, int l) { return ti * (uint32_t)a.n_layers + (uint32_t)l + 1u; }
// Argmax partial of token ti: tag (14 bits) | index (18 bits) | f32 value
Q35_DEV uint32_t arg_tag(uint32_t ti) { return (ti + 1u) & 0x3fffu; }
Q35_DEV uint64_t arg_pack(float v, int i, uint32_t ti) {
  const uint32_t ix = (i == INT_MAX) ? kArgNone : (uint32_t)i;
  return ((uint64_t)arg_tag(ti) << 50) | ((uint64_t)ix << 32) | __float_as_uint(v);
}
Q35_DEV bool arg_ok(uint64_t w, uint32_t ti) { return (uint32_t)(w >> 50) == arg_tag(ti); }
Q35_DEV void arg_unpack(uint64_t w, float& v, int& i) {
  const uint32_t ix = (uint32_t)(w >> 32) & kArgNone;
  v = __uint_as_float((uint32_t)w);
  i = (ix == kArgNone) ? INT_MAX : (int)ix;
}

Q35_DEV const void* readlane_ptr(const void* p, int lane) {
  const uint64_t u = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)u, lane), hi = __builtin_amdgcn_readlane((uint32_t)(u >> 32), lane);
  return reinterpret_cast<const void*>(((uint64_t)hi << 32) | lo);
}

// Polls one word (the same address in every lane, so one load per poll) until ready(word).
// Returns false once the error word is set or after kSpin polls (then it sets the time-out bit).
template <class Ready>
Q35_DEV bool wait_on(const StepArgs& a, const uint64_t* p, Ready ready) {
  for (uint32_t n = 1;; ++n) {
    if (ready(ld_agent64(p))) return true;
    if ((n & 31) == 0) {
      if (ld_agent(a.err) != 0u) return false;
      if (n >= kSpin) {
        raise_err(a, kStepErrTimeout);
        return false;
      }
    }
    __builtin_amdgcn_s_sleep(1);
  }
}

// Completes a thread's N input words w (loaded once already): test(j, w[j]) says whether word j
// is complete, load_all(w) reloads every word (addresses recomputed, so nothing extra stays live
// in registers), addr(j) is the address of word j (j wave-uniform).  While some lane of the wave
// has an incomplete word, the wave polls one such word (a lane's last), then reloads.  Wave-level
// (no workgroup barrier); returns false on error / time-out.
template <int N, class W, class LoadAll, class Addr, class Test>
Q35_DEV bool gather(const StepArgs& a, W (&w)[N], LoadAll load_all, Addr addr, Test test) {
  while (true) {
    // the last incomplete word is polled: inputs listed in producer order (chunks, then their
    // statistics) complete roughly in that order, so it is the one most likely to complete last
    // and fewer poll-and-reload rounds follow (0.7% faster than the first)
    int jf = N;
#pragma unroll
    for (int j = 0; j < N; ++j)
      if (!test(j, (uint64_t)w[j])) jf = j;
    const uint64_t bad = __ballot(jf < N);
    if (bad == 0) return true;
    const int sh = (bix() * 13 + (tix() >> 6) * 5) & 63;
    const uint64_t rot = sh ? ((bad >> sh) | (bad << (64 - sh))) : bad;
    const int lf = (__ffsll((unsigned long long)rot) - 1 + sh) & 63;
    const int jw = __builtin_amdgcn_readlane(jf, lf);
    const uint64_t* pw = static_cast<const uint64_t*>(readlane_ptr(addr(jw), lf));
    if (!wait_on(a, pw, [&](uint64_t x) { return test(jw, x); })) return false;
    load_all(w);
  }
}

// The layer table is never written by the kernel: read through the constant address space, its
// uniform fields are scalar loads (scalar cache) rather than vector loads that would queue behind
// the weight stream and force vmcnt waits.
typedef const __attribute__((address_space(4))) StepLayer CLayer;
Q35_DEV CLayer& layer_at(const StepArgs& a, int l) { return *(CLayer*)(a.layers + l); }

// Per token and layer: where this token's counted accumulators are and what a complete word holds.
struct Tok {
  fx_t* h;       // the residual stream as the last residual stage left it (parity set)
  fx_t* hn;      // the copy the next residual stage adds into (parity set)
  fx_t* acc;     // this layer's accumulators (parity set)
  uint32_t hc;   // contributions a complete word of h holds
  uint32_t ti;   // tokens run since the last reset, this one included (minus 1)
  int l;         // layer
};

// ------------------------------------------------------------------ matvec stages
struct Mv {
  const int8_t *w0, *w1, *w2;
  const float *s0, *s1, *s2;
  fx_t *a0, *a1, *a2;
  int n0, n1, n2;
  int t1, t2, t3;  // first tile of segments 1 and 2, total tiles
  int K, kch, nchunk;
  int spm;  // ~15 when the accumulator is the residual stream (index k at k + (k & ~15)), else 0
};

Q35_DEV int tiles_of(int n) { return (n + kTile - 1) / kTile; }

Q35_DEV Mv make_mv(const StepArgs& a, CLayer& L, const Tok& t, int kind) {
  Mv d{};
  const StepMv pl = a.mv[kind];
  d.kch = pl.kch;
  d.nchunk = pl.nchunk;
  fx_t* proj = t.acc;
  switch (kind) {
    case SMV_QKVZ:
      d.K = a.H;
      d.w0 = L.qkv_q; d.s0 = L.qkv_s; d.a0 = proj; d.n0 = a.conv_dim;
      d.w1 = L.z_q; d.s1 = L.z_s; d.a1 = proj + a.conv_dim; d.n1 = a.vdim;
      d.t1 = tiles_of(d.n0); d.t2 = d.t1 + tiles_of(d.n1); d.t3 = d.t2;
      break;
    case SMV_OUT:
      d.K = a.vdim;
      d.w0 = L.out_q; d.s0 = L.out_s; d.a0 = t.hn; d.n0 = a.H; d.spm = ~15;
      d.t1 = d.t2 = d.t3 = tiles_of(d.n0);
      break;
    case SMV_QKV: {
      const int ldqg = a.ah * a.hd * 2, nkv = a.kvh * a.hd;
      d.K = a.H;
      d.w0 = L.q_q; d.s0 = L.q_s; d.a0 = proj; d.n0 = ldqg;
      d.w1 = L.k_q; d.s1 = L.k_s; d.a1 = proj + ldqg; d.n1 = nkv;
      d.w2 = L.v_q; d.s2 = L.v_s; d.a2 = proj + ldqg + nkv; d.n2 = nkv;
      d.t1 = tiles_of(d.n0); d.t2 = d.t1 + tiles_of(d.n1); d.t3 = d.t2 + tiles_of(d.n2);
    } break;
    case SMV_O:
      d.K = a.ah * a.hd;
      d.w0 = L.o_q; d.s0 = L.o_s; d.a0 = t.hn; d.n0 = a.H; d.spm = ~15;
      d.t1 = d.t2 = d.t3 = tiles_of(d.n0);
      break;
    case SMV_GU:
      d.K = a.H;
      d.w0 = L.gate_q; d.s0 = L.gate_s; d.a0 = t.acc + a.acc_gu_off; d.n0 = a.F;
      d.w1 = L.up_q; d.s1 = L.up_s; d.a1 = t.acc + a.acc_gu_off + a.F; d.n1 = a.F;
      d.t1 = tiles_of(d.n0); d.t2 = d.t1 + tiles_of(d.n1); d.t3 = d.t2;
      break;
    default:  // SMV_DOWN
      d.K = a.F;
      d.w0 = L.down_q; d.s0 = L.down_s; d.a0 = t.hn; d.n0 = a.H; d.spm = ~15;
      d.t1 = d.t2 = d.t3 = tiles_of(d.n0);
      break;
  }
  return d;
}

struct MvItem {
  const int8_t* w;
  const float* s;
  fx_t* acc;
  int N, tile, tl, k0, klen, spm;
};

Q35_DEV MvItem mv_item(const Mv& d, int item) {
  MvItem it;
  const int tile = item / d.nchunk, ch = item - tile * d.nchunk;
  it.tile = tile;
  if (tile < d.t1) { it.w = d.w0; it.s = d.s0; it.acc = d.a0; it.N = d.n0; it.tl = tile; }
  else if (tile < d.t2) { it.w = d.w1; it.s = d.s1; it.acc = d.a1; it.N = d.n1; it.tl = tile - d.t1; }
  else { it.w = d.w2; it.s = d.s2; it.acc = d.a2; it.N = d.n2; it.tl = tile - d.t2; }
  it.k0 = ch * d.kch;
  it.klen = min(d.kch, d.K - it.k0);
  it.spm = d.spm;
  return it;
}

// rows of one item held per lane: U <= kU (the out stage's items have at most dv = 128 rows)
template <int U>
struct MvPf {
  uint4 w[U];
  float s[U];
};
constexpr int kUOut = kDv / kRG;

// Lane (cg, rr) loads 16 columns [cg*16, cg*16+16) of rows rr, rr+32, ... of the item.
// Loads are unconditional and branch-free so that all of them are in flight at once: a row past
// the item is clamped to its last row (mv_compute zeroes its contribution), and the columns past
// N of the last tile are the zero padding of the tiled layout.  32-bit offsets from the matrix
// base (every tiled matrix is < 4 GB) keep one VGPR per address.
template <int U>
Q35_DEV void mv_load(const MvItem& it, int K, MvPf<U>& pf) {
  const int cg = tix() & 15, rr = tix() >> 4;
  const uint32_t row0 = (uint32_t)it.tl * (uint32_t)K + (uint32_t)it.k0;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    if (kRG * u >= it.klen) break;  // uniform
    const uint32_t row = row0 + (uint32_t)min(rr + kRG * u, it.klen - 1);
    pf.w[u] = ldg16_nt(it.w + (row * (uint32_t)kTile + (uint32_t)(cg * 16)));
    pf.s[u] = ldg_nt(it.s + (row * (uint32_t)(kTile / 64) + (uint32_t)(cg >> 2)));
  }
}

// y[tile cols] += scale * sum over the item's rows of x[k] * dequant(W[k][cols]); x chunk in xs.  aux_dst
// (optional): one more sum, of which each wave holds its part in aux, reduced with the columns.
// The column sums are multiplied by `scale` (a deferred RMSNorm scale, else 1); thread n < kTile
// adds `base` (fixed point) to its column's contribution.
template <int U>
Q35_DEV void mv_compute(const StepArgs& a, const MvItem& it, const MvPf<U>& pf, const float* xs, float* red,
                        float scale, fx_t base, float aux = 0.f, fx_t* aux_dst = nullptr) {
  const int tid = tix(), cg = tid & 15, rr = tid >> 4;
  float acc[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) acc[j] = 0.f;
  // every row's x is read (clamped index) before the first is used: one LDS round trip, not one
  // per row behind a branch
  float xr[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    if (kRG * u >= it.klen) break;
    xr[u] = xs[min(rr + kRG * u, it.klen - 1)];
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    if (kRG * u >= it.klen) break;
    const float c = (rr + kRG * u < it.klen) ? xr[u] * pf.s[u] : 0.f;
    float f[16];
    unpack16(pf.w[u], f);
#pragma unroll
    for (int j = 0; j < 16; ++j) acc[j] += f[j] * c;
  }
  // The wave's 4 row groups (its 16-lane rows) are summed in registers with the gfx950 lane
  // swaps: first between the 32-lane halves (acc[j] with acc[j + 8]), then between neighbouring
  // rows; afterwards lane (row q, cg) holds columns cg*16 + 4q .. +3 of the wave's partial.
  float s8[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const auto x = __builtin_amdgcn_permlane32_swap(__float_as_uint(acc[j]), __float_as_uint(acc[j + 8]), false, false);
    s8[j] = __uint_as_float(x[0]) + __uint_as_float(x[1]);
  }
  float t4[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const auto x = __builtin_amdgcn_permlane16_swap(__float_as_uint(s8[j]), __float_as_uint(s8[j + 4]), false, false);
    t4[j] = __uint_as_float(x[0]) + __uint_as_float(x[1]);
  }
  *reinterpret_cast<float4*>(&red[(rr >> 2) * kTile + cg * 16 + 4 * (rr & 3)]) = make_float4(t4[0], t4[1], t4[2], t4[3]);
  if (aux_dst && (tid & 63) == 0) red[kNW * kTile + (tid >> 6)] = aux;
  __syncthreads();
  if (aux_dst && tid == 0) {
    float s = 0.f;
#pragma unroll
    for (int w = 0; w < kNW; ++w) s += red[kNW * kTile + w];
    fxc_add(a, aux_dst, s * scale);
  }
  if (tid < kTile) {
    // all kNW wave partials read before any is summed: one LDS round trip
    float pr[kNW];
#pragma unroll
    for (int i = 0; i < kNW; ++i) pr[i] = red[i * kTile + tid];
    __builtin_amdgcn_sched_barrier(0);  // keep the reads ahead of the sums (not interleaved)
    float v = 0.f;
#pragma unroll
    for (int i = 0; i < kNW; ++i) v += pr[i];
    const int n = it.tl * kTile + tid;
    if (n < it.N) fxc_add(a, &it.acc[n + (n & it.spm)], v * scale, base);
  }
  __syncthreads();
}

// xs[i] = x[k0+i] * rsqrt(mean(x^2) + eps) * (1 + w[k0+i]); thread t holds x[t + 512 j],
// j < KR (K <= 512 KR).  All loads (x and the thread's norm weights) are issued before any value
// is used, and all KR of each (indices clamped, masked afterwards): a compile-time number of
// loads, so the compiler's waits on them are exact.  The prologue costs one round trip when its
// input is complete: `src.load(k)` returns the raw element, `src.complete` waits for incomplete
// ones (counted inputs), `src.conv` turns it into f32.  `post` (more weight loads of the caller)
// is issued behind the prologue's loads and before their first use; scheduling barriers keep the
// compiler from moving either group across it.  Returns false when a wait failed.
// DEFER: xs gets x * (1 + w) only, and each wave leaves its part of the sum of squares in shs; the
// caller applies rsqrt(mean + eps) to the matvec's column sums (the scale is the same for every
// row: W^T (x r (1 + w)) = r W^T (x (1 + w))), which takes the block sum off the path to the
// multiply-adds.
template <int KR, bool DEFER, class Raw, class Src, class Post>
Q35_DEV bool pro_rms(const StepArgs& a, const Src& src, Raw (&raw)[KR], int K, const float* w, int k0, int klen, float* xs,
                     float* shs, Post post) {
  const int tid = tix();
  float wn[KR];
#pragma unroll
  for (int j = 0; j < KR; ++j) {
    const int k = tid + kT * j;
    raw[j] = src.load(min(k, K - 1));
    wn[j] = ldg(w + min(max(k, k0), k0 + klen - 1));
  }
  __builtin_amdgcn_sched_barrier(0);
  post();
  __builtin_amdgcn_sched_barrier(0);
  const bool ok = src.template complete<KR>(a, raw, K, 0, K);
  float v[KR];
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < KR; ++j) {
    v[j] = (tid + kT * j < K) ? src.conv(raw[j]) : 0.f;
    ss += v[j] * v[j];
  }
  if constexpr (DEFER) {
    ss = wave_sum(ss);
    if ((tid & 63) == 0) shs[tid >> 6] = ss;
#pragma unroll
    for (int j = 0; j < KR; ++j) {
      const int k = tid + kT * j;
      if (k >= k0 && k < k0 + klen) xs[k - k0] = v[j] * (1.0f + wn[j]);
    }
    return ok;
  }
  // every caller reaches here right after a workgroup barrier (the stage's start, or the
  // previous item's reduction), so the block sum needs no leading one
  ss = block_sum(ss, shs, false);
  const float r = rsqrt_f(ss * rcp_f((float)K) + a.eps);
#pragma unroll
  for (int j = 0; j < KR; ++j) {
    const int k = tid + kT * j;
    if (k >= k0 && k < k0 + klen) xs[k - k0] = (v[j] * r) * (1.0f + wn[j]);
  }
  return ok;
}

// the residual stream h (counted fixed point, e contributions) as pro_rms input
struct HSrc {
  const fx_t* h;
  uint32_t e;
  Q35_DEV const fx_t* at(int k) const { return h + (k + (k & ~15)); }
  Q35_DEV fx_t load(int k) const { return ld_agent(at(k)); }
  Q35_DEV float conv(fx_t x) const { return fxc_val(x, e); }
  // completes the thread's elements k in [lo, hi) (the others may stay incomplete)
  template <int KR>
  Q35_DEV bool complete(const StepArgs& a, fx_t (&raw)[KR], int K, int lo, int hi) const {
    return gather<KR>(
        a, raw,
        [&](fx_t (&r)[KR]) {
#pragma unroll
          for (int j = 0; j < KR; ++j) r[j] = load(min(tix() + kT * j, K - 1));
        },
        [&](int j) { return (const void*)at(min(tix() + kT * j, K - 1)); },
        [&](int j, uint64_t w) {
          const int k = min(tix() + kT * j, K - 1);
          return k < lo || k >= hi || fxc_ok((fx_t)w, e);
        });
  }
};
// a row of the Q8F embedding table as pro_rms input: (byte, block scale) pairs
struct EmbRaw {
  int8_t q;
  float s;
};
struct EmbSrc {
  const int8_t* q;
  const float* s;
  Q35_DEV EmbRaw load(int k) const { return EmbRaw{ldg(q + k), ldg(s + (k >> 6))}; }
  Q35_DEV float conv(EmbRaw x) const { return (float)x.q * x.s; }
  template <int KR>
  Q35_DEV bool complete(const StepArgs&, EmbRaw (&)[KR], int, int, int) const { return true; }
};

// The argmax of token ti from the per-block partials (the reference's order), once all carry
// that token's tag.  Returns false when a wait failed.
Q35_DEV bool reduce_argmax(const StepArgs& a, uint32_t ti, const Shared& sh, int& tok) {
  float v = -INFINITY;
  int ix = INT_MAX;
  const uint64_t* ap = a.argp + (size_t)(ti & 1u) * gridDim.x + min(tix(), (int)gridDim.x - 1);
  uint64_t w[1] = {ld_agent64(ap)};
  const bool ok = gather<1>(
      a, w, [&](uint64_t (&x)[1]) { x[0] = ld_agent64(ap); }, [&](int) { return (const void*)ap; },
      [&](int, uint64_t x) { return arg_ok(x, ti); });
  if (tix() < (int)gridDim.x) arg_unpack(w[0], v, ix);
  block_argmax(v, ix, sh.shv, sh.shi, a.ord);
  tok = (ix == INT_MAX) ? 0 : ix;
  return ok;
}

// The argmax after position q into hist[q], and in the streamed build (STREAM) into the host
// token stream tok_host[q] as well: a plain system-scope store; each slot is written once per
// launch and the host waits for it to leave the -1 it set before the launch.  A build of its own:
// a runtime branch on the stream pointer cost the plain kernel 0.5% (code layout), and an
// unconditional store (to hist when not streaming) 1%: stores and loads share the wave's memory
// counter here, so block 0's next waits sat behind the slow system-scope store.
template <bool STREAM>
Q35_DEV void record_token(const StepArgs& a, int q, int tok) {
  st_agent(&a.hist[q], tok);
  if constexpr (STREAM)
    __hip_atomic_store((Q35_GLOBAL int32_t*)(a.tok_host + q), tok, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// Token of step i at position p: the prompt id while p < plen, else the argmax of the previous
// step, or *token for the launch's first step.  Block 0 records the previous step's argmax in
// hist.  Returns false when a wait failed.
template <bool STREAM>
Q35_DEV bool select_token(const StepArgs& a, const Tok& t, int i, int p, const Shared& sh, int& tok) {
  bool ok = true;
  if (i == 0) {
    tok = ld_agent(a.token);
  } else {
    ok = reduce_argmax(a, t.ti - 1, sh, tok);
    if (bix() == 0 && tix() == 0) record_token<STREAM>(a, p - 1, tok);
  }
  if (p < ldg(a.plen)) tok = ldg(a.prompt + p);
  return ok;
}

// A generated step (position past the prompt) whose input token is a stop id is not run.  Every
// block reduces the same partials, so every block takes the same decision.
Q35_DEV bool is_stop(const StepArgs& a, int p, int tok) {
  if (a.n_stop <= 0 || p < ldg(a.plen)) return false;
  bool s = false;
#pragma unroll
  for (int j = 0; j < 4; ++j) s |= (j < a.n_stop) && tok == a.stop_ids[j];
  return s;
}

enum { kStageFail = 0, kStageOk = 1, kStageStop = 2 };

// ------------------------------------------------------------------ Gated DeltaNet step
// The out stage's prologue.  An out item covers rows [k0, k0 + klen) of the core output o, and
// klen divides dv, so they lie in one value head h.  The gated RMSNorm needs all dv outputs of
// h, so every block with an item in h runs the whole recurrent step of h (a dk x dv state) and
// keeps the rows it needs; the block holding tile 0 and the first rows of h writes the new
// recurrent state and the shifted conv state.  Both states have two copies per layer: step i of
// a launch reads copy i & 1 and writes the other, so that write never races the other blocks'
// reads of the old state (their loads are issued before their inputs are complete and may still
// be queued behind weight loads).
// text_modules.rs:134-162 (causal conv + state shift), :184-187 (l2norm), :365-443 (gated delta
// rule), RMSNormGated: x = w[k % dv] * (o * rsqrt(mean_h(o^2) + eps)) * silu(z).
//
// dk = dv = 128 (every Qwen3.5 text model).  Thread t holds column j = t % 128 of state rows
// 32 ig .. 32 ig + 31, ig = t / 128: every load and store instruction of a wave covers 256
// contiguous bytes of one row.  Thread t < 384 also owns conv channel t of the head (q | k | v).
struct GdnPf {
  float s[kGdnR];   // old state rows
  float cs[3];      // conv state of the thread's channel
  float cw[4];      // conv weights of the thread's channel
  float nw;         // gated-norm weight of the thread's o row
  float dtb, alog;
};

struct GdnBuf {
  const float *S, *cst;  // read this step
  float *S_w, *cst_w;    // written this step
};
Q35_DEV GdnBuf gdn_buf(CLayer& L, int i) {
  if (i & 1) return GdnBuf{L.rec_alt, L.conv_alt, L.rec, L.conv_state};
  return GdnBuf{L.rec, L.conv_state, L.rec_alt, L.conv_alt};
}

// conv channel of the head's q | k | v element t (t < 2dk + dv)
Q35_DEV int gdn_channel(const StepArgs& a, int h, int t) {
  if (t < kDk) return h * kDk + t;
  if (t < 2 * kDk) return a.key_dim + h * kDk + (t - kDk);
  return 2 * a.key_dim + h * kDv + (t - 2 * kDk);
}

// Everything of the step that does not depend on the qkvz stage: issued before its inputs.
Q35_DEV void gdn_load(const StepArgs& a, CLayer& L, const MvItem& it, int i, GdnPf& g) {
  const int tid = tix(), j = tid % kDv, ig = tid / kDv;
  const int h = it.k0 / kDv;
  const GdnBuf b = gdn_buf(L, i);
  // uniform head base + 32-bit lane offsets: one VGPR per address
  const float* S = b.S + (size_t)h * kDk * kDv;
  const uint32_t off = (uint32_t)(ig * kGdnR * kDv + j);
#pragma unroll
  for (int r = 0; r < kGdnR; ++r) g.s[r] = ld_agent(S + (off + (uint32_t)(r * kDv)));
  const int c = gdn_channel(a, h, min(tid, 2 * kDk + kDv - 1));
#pragma unroll
  for (int e = 0; e < 3; ++e) g.cs[e] = ld_agent(&b.cst[(size_t)c * 3 + e]);
#pragma unroll
  for (int e = 0; e < 4; ++e) g.cw[e] = ldg(L.conv_w + (size_t)c * 4 + e);
  g.nw = ldg(L.norm_w + (it.k0 + min(tid, it.klen - 1)) % kDv);
  g.dtb = ldg(L.dt_bias + h);
  g.alog = ldg(L.a_log + h);
}

Q35_DEV bool pro_gdn(const StepArgs& a, CLayer& L, const Tok& t, const MvItem& it, int i, GdnPf& g, float* xs,
                     float* scratch) {
  const int tid = tix(), lane = tid & 63;
  const int j = tid % kDv, ig = tid / kDv;
  const int h = it.k0 / kDv, nch = 2 * kDk + kDv;
  float* qkv = scratch;          // [2dk + dv] conv outputs q | k | v of head h
  float* part0 = scratch + 512;  // [kT] per-row-group column partials
  float* part1 = part0 + kT;     // [kT]
  float* ov = part1 + kT;        // [dv] outputs of head h
  // qkvz-stage outputs: the thread's conv input, its z element and the two gate projections
  const uint32_t e = (uint32_t)a.mv[SMV_QKVZ].nchunk;
  const int c = gdn_channel(a, h, min(tid, nch - 1));
  auto ad = [&](int q) -> const fx_t* {
    const int tq = tix();
    if (q == 0) return &t.acc[gdn_channel(a, h, min(tq, nch - 1))];
    if (q == 1) return &t.acc[a.conv_dim + it.k0 + min(tq, it.klen - 1)];
    return &t.acc[a.acc_ba_off + (size_t)(q == 2 ? h : a.nh + h) * kStepBaStride];
  };
  auto load_all = [&](fx_t (&r)[4]) {
#pragma unroll
    for (int q = 0; q < 4; ++q) r[q] = ld_agent(ad(q));
  };
  fx_t in[4];
  load_all(in);
  const bool done = gather<4>(a, in, load_all, [&](int q) { return (const void*)ad(q); },
                              [&](int, uint64_t w) { return fxc_ok((fx_t)w, e); });
  const float x = fxc_val(in[0], e), zv = fxc_val(in[1], e), bs = fxc_val(in[2], e), as = fxc_val(in[3], e);
  if (tid < nch) qkv[tid] = silu_f(((g.cw[0] * g.cs[0] + g.cw[1] * g.cs[1]) + g.cw[2] * g.cs[2]) + g.cw[3] * x);
  const bool writer = it.tl == 0 && (it.k0 % kDv) == 0;  // uniform
  const GdnBuf b = gdn_buf(L, i);
  // gates: beta = sigmoid(b); g = -exp(A_log) * softplus(a + dt_bias) (kernels.rs:228-244)
  const float beta = sigmoid_f(bs);
  const float xg = as + g.dtb;
  const float pre = logf(expf(xg) + 1.0f);
  const float decay = expf(-expf(g.alog) * (pre > 20.0f ? xg : pre));
  __syncthreads();
  // l2 norms of q and k (dk = 128): every wave sums all the squares itself, so no second barrier
  const float q0 = qkv[lane], q1 = qkv[lane + 64], k0 = qkv[kDk + lane], k1 = qkv[kDk + lane + 64];
  const float rq = rsqrt_f(wave_sum(q0 * q0 + q1 * q1) + 1e-6f);
  const float rk = rsqrt_f(wave_sum(k0 * k0 + k1 * k1) + 1e-6f);
  const float kq = wave_sum(q0 * k0 + q1 * k1);  // k_raw . q_raw
  // With k = rk k_raw, q = rq qscale q_raw and S the old state:
  //   S' = decay S,  m = S'^T k = decay rk u,  delta = beta (v - m),  S'' = S' + k delta^T,
  //   o = S''^T q = rq qscale (decay w + rk kq delta),  u = S^T k_raw,  w = S^T q_raw,
  // so one pass over the state gives u and w, and only the writer forms S'' (to store it).
  const float* kr = qkv + kDk + ig * kGdnR;
  const float* qr = qkv + ig * kGdnR;
  float u = 0.f, w = 0.f;
#pragma unroll
  for (int r = 0; r < kGdnR; ++r) {
    u += g.s[r] * kr[r];
    w += g.s[r] * qr[r];
  }
  part0[tid] = u;
  part1[tid] = w;
  __syncthreads();
  auto colsum = [&](const float* part, int jj) {  // sum over the row groups of column jj
    float s = 0.f;
#pragma unroll
    for (int gg = 0; gg < kGdnG; ++gg) s += part[gg * kDv + jj];
    return s;
  };
  // the thread's column j: delta and output (the ig = 0 threads publish the dv outputs)
  const float dl = (qkv[2 * kDk + j] - (decay * rk) * colsum(part0, j)) * beta;
  const float oj = (rq * a.qscale) * (decay * colsum(part1, j) + (rk * kq) * dl);
  if (tid < kDv) ov[tid] = oj;
  __syncthreads();
  // gated RMSNorm over the dv outputs of h, whose sum of squares every wave forms itself
  const float oa = ov[lane], ob = ov[lane + 64];
  const float rg = rsqrt_f(wave_sum(oa * oa + ob * ob) / (float)kDv + a.eps);
  if (tid < it.klen) xs[tid] = (g.nw * (ov[it.k0 % kDv + tid] * rg)) * silu_f(zv);
  // Off the path to the out_proj multiply-adds: the writer's new state S'' (column j) and conv
  // state [c] <- [s1, s2, x], stored while the multiply-adds run.  Their completion is ordered
  // before the writer's next contributions (the gate|up stage's), not before this stage's.
  if (writer) {
    const float dlk = dl * rk;
    float* Sw = b.S_w + (size_t)h * kDk * kDv;
    const uint32_t off = (uint32_t)(ig * kGdnR * kDv + j);
#pragma unroll
    for (int r = 0; r < kGdnR; ++r) st_agent(Sw + (off + (uint32_t)(r * kDv)), decay * g.s[r] + kr[r] * dlk);
    if (tid < nch) {
      float* cw = b.cst_w + (size_t)c * 3;
      st_agent(&cw[0], g.cs[1]);
      st_agent(&cw[1], g.cs[2]);
      st_agent(&cw[2], x);
    }
  }
  return done;
}

Q35_DEV void attn_chunking(const StepArgs& a, int T, int& chunk, int& nact) {
  chunk = max(kMinChunk, (T + a.att_nmax - 1) / a.att_nmax);
  nact = (T + chunk - 1) / chunk;
}

// o_proj input: merge the split-T partials of each touched query head (flash-decoding merge,
// chunks in order) and apply the sigmoid output gate (text_modules.rs:936).  The partials carry
// the attention stage's tag; the gate is a counted projection output.
Q35_DEV bool pro_attn(const StepArgs& a, const Tok& t, int T, int k0, int klen, float* xs, float* scratch) {
  const int tid = tix(), lane = tid & 63, wid = tid >> 6;
  const int rep = a.ah / a.kvh;
  int chunk, nact;
  attn_chunking(a, T, chunk, nact);
  const uint32_t tag = att_tag(a, t.ti, t.l), eg = (uint32_t)a.mv[SMV_QKV].nchunk;
  float* wts = scratch;                         // [kMaxTouch][kMaxNmax] exp(m_c - M)
  float* pbuf = scratch + kMaxTouch * kMaxNmax; // [kT] per-part sums
  float* wl = pbuf + kT;                        // [kMaxTouch] L
  const int h0 = k0 / kHd, h1 = (k0 + klen - 1) / kHd;  // at most 3 heads (klen <= 512): waves 0..2
  // Thread (part, i): output element k0 + i, chunks part, part + parts, ...  The partial outputs
  // do not depend on the statistics, so the first batch is issued with them: one round trip.
  const int parts = klen <= 64 ? 8 : (klen <= 128 ? 4 : (klen <= 256 ? 2 : 1));
  const int span = kT / parts;
  const int i = tid % span, part = tid / span;
  const int kk = k0 + min(i, klen - 1), hk = kk / kHd;  // clamped; masked below
  const uint64_t* og = a.att_o + ((size_t)(hk / rep) * a.att_nmax * kMaxRep + hk % rep) * kHd + kk % kHd;  // + c*kMaxRep*kHd
  // the wave's head (wave w < h1 - h0 + 1 merges the statistics of head h0 + w)
  const int hh = min(h0 + wid, h1);
  constexpr int kQ = kMaxNmax / 64;
  constexpr int kIn = kMergeB + 1 + 2 * kQ;
  // input words: [0, kMergeB) first batch of partial outputs, kMergeB the gate (counted),
  // then the chunk statistics m, l of chunks lane + 64q (clamped; masked below)
  auto addr = [&](int q) -> const void* {
    const int tq = tix(), iq = tq % span, pq = tq / span, kq = k0 + min(iq, klen - 1), hq = kq / kHd;
    if (q < kMergeB)
      return a.att_o + ((size_t)(hq / rep) * a.att_nmax * kMaxRep + hq % rep) * kHd + kq % kHd +
             (size_t)min(pq + q * parts, nact - 1) * kMaxRep * kHd;
    if (q == kMergeB) {
      const int kg = k0 + min(tq, klen - 1);
      return t.acc + (size_t)(kg / kHd) * 2 * kHd + kHd + kg % kHd;
    }
    const int hw = min(h0 + (tq >> 6), h1);
    const int qq = (q - kMergeB - 1) % kQ, ml_l = (q - kMergeB - 1) / kQ;
    const int c = min((tq & 63) + 64 * qq, nact - 1);
    return a.att_ml + (size_t)(hw / rep) * a.att_nmax * 2 * kMaxRep + (size_t)c * 2 * kMaxRep + ml_l * kMaxRep + hw % rep;
  };
  auto load_all = [&](uint64_t (&r)[kIn]) {
#pragma unroll
    for (int q = 0; q < kIn; ++q) r[q] = ld_agent64(static_cast<const uint64_t*>(addr(q)));
  };
  uint64_t in[kIn];
  load_all(in);
  bool done = gather<kIn>(a, in, load_all, addr, [&](int q, uint64_t w) {
    return q == kMergeB ? fxc_ok((fx_t)w, eg) : tag_ok(w, tag);
  });
  if (wid <= h1 - h0) {
    float M = -INFINITY;
#pragma unroll
    for (int q = 0; q < kQ; ++q) M = fmaxf(M, (lane + 64 * q < nact) ? tag_val(in[kMergeB + 1 + q]) : -INFINITY);
    M = wave_max(M);
    float Ls = 0.f;
#pragma unroll
    for (int q = 0; q < kQ; ++q) {
      const int c = lane + 64 * q;
      const float w = expf(tag_val(in[kMergeB + 1 + q]) - M);
      if (c < nact) {
        wts[(hh - h0) * kMaxNmax + c] = w;
        Ls += tag_val(in[kMergeB + 1 + kQ + q]) * w;
      }
    }
    Ls = wave_sum(Ls);
    if (lane == 0) wl[hh - h0] = Ls;
  }
  __syncthreads();
  float o = 0.f;
  if (i < klen) {
    const float* w = wts + (hk - h0) * kMaxNmax;
    // every chunk weight is read (clamped) before the first is used: the reads inside the mask's
    // branches were waited for one by one
    float wc[kMergeB];
#pragma unroll
    for (int j = 0; j < kMergeB; ++j) wc[j] = w[min(part + j * parts, nact - 1)];
#pragma unroll
    for (int j = 0; j < kMergeB; ++j) o += (part + j * parts < nact) ? tag_val(in[j]) * wc[j] : 0.f;
  }
  // further batches (long contexts with more than kMergeB chunks per part)
  for (int c0 = part + kMergeB * parts; c0 < nact; c0 += kMergeB * parts) {  // uniform per wave
    uint64_t v[kMergeB];  // all of a batch in flight at once (clamped; masked below)
    auto vaddr = [&](int j) -> const void* { return og + (size_t)min(c0 + j * parts, nact - 1) * kMaxRep * kHd; };
    auto vload = [&](uint64_t (&r)[kMergeB]) {
#pragma unroll
      for (int j = 0; j < kMergeB; ++j) r[j] = ld_agent64(static_cast<const uint64_t*>(vaddr(j)));
    };
    vload(v);
    done &= gather<kMergeB>(a, v, vload, vaddr, [&](int, uint64_t w) { return tag_ok(w, tag); });
    if (i < klen) {
      const float* w = wts + (hk - h0) * kMaxNmax;
      float wv[kMergeB];
#pragma unroll
      for (int j = 0; j < kMergeB; ++j) wv[j] = w[min(c0 + j * parts, nact - 1)];
#pragma unroll
      for (int j = 0; j < kMergeB; ++j) o += (c0 + j * parts < nact) ? tag_val(v[j]) * wv[j] : 0.f;
    }
  }
  pbuf[part * span + i] = o;
  __syncthreads();
  if (tid < klen) {
    float s = 0.f;
    for (int q = 0; q < parts; ++q) s += pbuf[q * span + tid];
    const int hq = (k0 + tid) / kHd;
    xs[tid] = (s * rcp_f(wl[hq - h0])) * sigmoid_f(fxc_val((fx_t)in[kMergeB], eg));
  }
  return done;
}

// One matvec stage.  The in_proj_b / in_proj_a gate projection (f32, [H][nh] each,
// kernels.rs:174-247) rides on the qkvz stage: the item of tile t < 2*nh also forms the partial
// dot product of its rows with column t of [W_b | W_a].  U: rows per lane the stage's items need;
// KR: hidden-size elements per thread in the RMSNorm prologue (hidden <= 512 KR).
// Returns kStageOk, kStageFail (a wait failed) or, for the first stage of a step, kStageStop
// (the step's input token is a stop id; *stop_tok receives it, nothing of the step has run).
template <int U, int KR, bool STREAM = false>
Q35_DEV int mv_stage(const StepArgs& a, CLayer& L, const Tok& t, int kind, int pro, int i, int p, const Shared& sh,
                     int* stop_tok = nullptr) {
  const Mv d = make_mv(a, L, t, kind);
  const int nitems = d.t3 * d.nchunk;
  int item = bix();
  if (kind == SMV_GU) {
    // The out stage's state writers (out items with tile 0 and k0 % dv == 0, i.e. blocks b < nh cph
    // with b % cph == 0) finish last and so issue this stage's weights last: a permutation of
    // [0, grid) gives them the last slots, which are idle when the stage has fewer items than blocks.
    const int cph = kDv / a.mv[SMV_OUT].kch, nw = a.nh, g = (int)gridDim.x, b = bix();
    if (nw * cph <= g) {
      const bool w = b < nw * cph && b % cph == 0;
      item = w ? g - nw + b / cph : b - min((b + cph - 1) / cph, nw);
    }
  }
  MvPf<U> pf;
  MvItem it{};
  GdnPf gp;
  float auxw = 0.f;
  const int naux = 2 * a.nh;
  // A residual stage adds into a fresh copy of the stream (t.hn); its first-chunk items carry the
  // previous copy (t.h, complete: every block that reads this stage's inputs has seen it so) into
  // it, each with its columns' words, loaded with the weights and checked after the prologue.
  const bool carry = (kind == SMV_OUT || kind == SMV_O || kind == SMV_DOWN) && t.h != t.hn;
  auto carry_at = [&]() {
    const int n = min(it.tl * kTile + (tix() & (kTile - 1)), it.N - 1);
    return &t.h[n + (n & ~15)];
  };
  fx_t hp[1] = {0};
  if (item < nitems) {
    it = mv_item(d, item);
    mv_load(it, d.K, pf);
    if (pro == PRO_GDN) gdn_load(a, L, it, i, gp);
    if (carry && it.k0 == 0) hp[0] = ld_agent(carry_at());
  }
  int tok = 0;
  // Blocks with an item need the token for the embedding; with stop ids every block forms it,
  // so that every block sees a stop.
  if (pro == PRO_EMBED_RMS && (item < nitems || a.n_stop > 0)) {
    if (!select_token<STREAM>(a, t, i, p, sh, tok)) return kStageFail;
    if (is_stop(a, p, tok)) {
      if (stop_tok) *stop_tok = tok;
      return kStageStop;
    }
  }
  float* xs = sh.smem + kXs;
  float* red = sh.smem + kRed;
  for (bool first = true; item < nitems; item += gridDim.x, first = false) {
    if (!first) {
      it = mv_item(d, item);
      mv_load(it, d.K, pf);
      if (pro == PRO_GDN) gdn_load(a, L, it, i, gp);
      if (carry && it.k0 == 0) hp[0] = ld_agent(carry_at());
    }
    // the qkvz item's gate column (a 64-byte-strided gather) is issued behind the norm's inputs
    auto aux_load = [&]() {
      if (kind == SMV_QKVZ && it.tile < naux && first) {  // row clamped; masked where it is used
        const float* W = it.tile < a.nh ? L.w_b : L.w_a;
        auxw = ldg(W + ((size_t)(it.k0 + min(tix(), it.klen - 1)) * a.nh + (it.tile % a.nh)));
      }
    };
    bool ok = true;
    const HSrc hsrc{t.h, t.hc};
    fx_t hraw[KR];
    switch (pro) {
      case PRO_EMBED_RMS: {
        const int K = d.K, nbK = K >> 6;
        const EmbSrc src{a.emb_q + (size_t)tok * K, a.emb_s + (size_t)tok * nbK};
        EmbRaw eraw[KR];
        pro_rms<KR, true, EmbRaw>(a, src, eraw, K, L.in_norm, it.k0, it.klen, xs, sh.shs, aux_load);
        if (bix() == 0 && first)  // the residual stream starts as the embedding row (one contribution)
          for (int k = tix(); k < K; k += kT) fxc_add(a, &t.hn[k + (k & ~15)], src.conv(src.load(k)));
      } break;
      case PRO_RMS:
        ok = pro_rms<KR, true, fx_t>(a, hsrc, hraw, d.K, kind == SMV_GU ? L.post_norm : L.in_norm, it.k0, it.klen, xs,
                                     sh.shs, aux_load);
        break;
      case PRO_GDN:
        ok = pro_gdn(a, L, t, it, i, gp, xs, red);
        break;
      case PRO_SWIGLU: {  // klen <= 512 = threads: one element per thread
        const int k = it.k0 + min(tix(), it.klen - 1);
        const uint32_t e = (uint32_t)a.mv[SMV_GU].nchunk;
        const fx_t* gu = t.acc + a.acc_gu_off;
        auto ad = [&](int q) { return q == 0 ? &gu[a.F + k] : &gu[k]; };
        auto load_all = [&](fx_t (&r)[2]) {
          r[0] = ld_agent(ad(0));
          r[1] = ld_agent(ad(1));
        };
        fx_t in[2];
        load_all(in);
        ok = gather<2>(a, in, load_all, [&](int q) { return (const void*)ad(q); },
                       [&](int, uint64_t w) { return fxc_ok((fx_t)w, e); });
        if (tix() < it.klen) xs[tix()] = fxc_val(in[0], e) * silu_f(fxc_val(in[1], e));
      } break;
      default:  // PRO_ATTN: merged attention output
        ok = pro_attn(a, t, p + 1, it.k0, it.klen, xs, red);
        break;
    }
    if (ok && carry && it.k0 == 0)
      ok = gather<1>(
          a, hp, [&](fx_t (&r)[1]) { r[0] = ld_agent(carry_at()); }, [&](int) { return (const void*)carry_at(); },
          [&](int, uint64_t w) { return fxc_ok((fx_t)w, t.hc); });
    if (!ok) *sh.fail = 1;
    __syncthreads();
    if (*sh.fail) return kStageFail;
    // the RMSNorm scale deferred by the prologue (1 for the other prologues)
    float rn = 1.f;
    if (pro == PRO_RMS || pro == PRO_EMBED_RMS) {
      const float4 s0 = *reinterpret_cast<const float4*>(sh.shs), s1 = *reinterpret_cast<const float4*>(sh.shs + 4);
      const float ss = ((((((s0.x + s0.y) + s0.z) + s0.w) + s1.x) + s1.y) + s1.z) + s1.w;
      rn = rsqrt_f(ss * rcp_f((float)d.K) + a.eps);
    }
    // in_proj_b | in_proj_a column it.tile (there are at least as many qkvz tiles, 1.5 nh + 0.5 nh
    // rounded up, as the 2 nh columns): each wave's part of the dot product goes into the matvec
    // reduction
    float auxp = 0.f;
    fx_t* auxd = nullptr;
    if (kind == SMV_QKVZ && it.tile < naux) {
      float w = auxw;
      if (!first) {
        const float* W = it.tile < a.nh ? L.w_b : L.w_a;
        w = ldg(W + ((size_t)(it.k0 + min(tix(), it.klen - 1)) * a.nh + (it.tile % a.nh)));
      }
      auxp = wave_sum((tix() < it.klen) ? xs[tix()] * w : 0.f);
      auxd = t.acc + a.acc_ba_off + (size_t)it.tile * kStepBaStride;
    }
    const fx_t base = (carry && it.k0 == 0) ? (fx_t)((uint64_t)hp[0] - cnt_of(t.hc)) : 0;
    mv_compute(a, it, pf, xs, red, rn, base, auxp, auxd);
  }
  return kStageOk;
}

// ------------------------------------------------------------------ attention partials
// Item (kv head g, chunk c of `chunk` cached tokens) for the rep query heads of g
// (text_modules.rs:842-944): q/k RMSNorm (1+w), partial RoPE (:739-774), KV append at p
// (the item holding p), scores, chunk softmax statistics and P.V, stored tagged.
//
// Nothing the qkv stage writes is needed to fetch the first item's cached K / V rows t < p
// (written by earlier steps), the q / k norm weights and the thread's RoPE factors, so they are
// loaded before its inputs: the stage then has one memory round trip (its q, k, v inputs)
// instead of four.  Wave w holds rows t0 + w + 8j, j < kAttnPf; rows beyond are loaded in-stage.
constexpr int kAttnPf = 2;
template <int MC>
Q35_DEV bool attn_stage(const StepArgs& a, CLayer& L, const Tok& t, int p, const Shared& sh) {
  const int tid = tix(), lane = tid & 63, wid = tid >> 6;
  const int T = p + 1, rep = a.ah / a.kvh;
  int chunk, nact;
  attn_chunking(a, T, chunk, nact);
  if ((int)bix() >= a.kvh * nact) return true;  // no item
  float4 kp[kAttnPf], vp[kAttnPf];
  {
    const int it0 = bix();
    const int g = it0 / nact, t0 = (it0 % nact) * chunk;
    const float* Kc = L.kc + (size_t)g * a.tmax * kHd;
    const float* Vc = L.vc + (size_t)g * a.tmax * kHd;
#pragma unroll
    for (int j = 0; j < kAttnPf; ++j) {  // clamped to written rows; the row at p comes from LDS
      const int tt = max(0, min(t0 + wid + kNW * j, p - 1));
      kp[j] = make_float4(ld_agent(&Kc[(size_t)tt * kHd + 4 * lane]), ld_agent(&Kc[(size_t)tt * kHd + 4 * lane + 1]),
                          ld_agent(&Kc[(size_t)tt * kHd + 4 * lane + 2]), ld_agent(&Kc[(size_t)tt * kHd + 4 * lane + 3]));
      vp[j] = make_float4(ld_agent(&Vc[(size_t)tt * kHd + 4 * lane]), ld_agent(&Vc[(size_t)tt * kHd + 4 * lane + 1]),
                          ld_agent(&Vc[(size_t)tt * kHd + 4 * lane + 2]), ld_agent(&Vc[(size_t)tt * kHd + 4 * lane + 3]));
    }
  }
  const float4 qw = make_float4(ldg(L.q_norm + 4 * lane), ldg(L.q_norm + 4 * lane + 1), ldg(L.q_norm + 4 * lane + 2),
                                ldg(L.q_norm + 4 * lane + 3));
  const float4 kw = make_float4(ldg(L.k_norm + 4 * lane), ldg(L.k_norm + 4 * lane + 1), ldg(L.k_norm + 4 * lane + 2),
                                ldg(L.k_norm + 4 * lane + 3));
  const float csv = ldg(a.rope_cos + (size_t)p * a.rot + tid % a.rot);  // rot divides 512: the same
  const float snv = ldg(a.rope_sin + (size_t)p * a.rot + tid % a.rot);  // element in every round
  float* qn = sh.smem;               // [kMaxRep][kHd]
  float* kn = qn + kMaxRep * kHd;    // [kHd]
  float* vn = kn + kHd;              // [kHd]
  float* rtmp = vn + kHd;            // [kMaxRep + 1][kHd]
  float* sc = rtmp + (kMaxRep + 1) * kHd;  // [kMaxRep][MC]
  float* ored = sc + kMaxRep * MC;  // [kNW][kMaxRep][kHd]
  float* hm = ored + kNW * kMaxRep * kHd;  // [kMaxRep]
  float* hl = hm + kMaxRep;                // [kMaxRep]
  const int ldqg = a.ah * kHd * 2;
  const uint32_t e = (uint32_t)a.mv[SMV_QKV].nchunk, tag = att_tag(a, t.ti, t.l);
  for (int item = bix(), first = 1; item < a.kvh * nact; item += gridDim.x, first = 0) {
    const int g = item / nact, c = item % nact;
    const int t0 = c * chunk, len = min(chunk, T - t0);
    const bool has_new = (c == nact - 1);
    // wave w < rep: query head g*rep + w; w == rep: k of g; w == rep + 1: v of g (the item at p)
    const int w = wid;
    if (w < rep + (has_new ? 2 : 0)) {
      const int d = 4 * lane;
      const fx_t* src = (w < rep)    ? t.acc + (size_t)(g * rep + w) * 2 * kHd + d
                        : (w == rep) ? t.acc + ldqg + (size_t)g * kHd + d
                                     : t.acc + ldqg + (size_t)(a.kvh + g) * kHd + d;
      auto load_all = [&](fx_t (&r)[4]) {
#pragma unroll
        for (int q = 0; q < 4; ++q) r[q] = ld_agent(src + q);
      };
      fx_t in[4];
      load_all(in);
      const bool done = gather<4>(a, in, load_all, [&](int q) { return (const void*)(src + q); },
                                  [&](int, uint64_t x) { return fxc_ok((fx_t)x, e); });
      if (!done) *sh.fail = 1;
      const float4 v = make_float4(fxc_val(in[0], e), fxc_val(in[1], e), fxc_val(in[2], e), fxc_val(in[3], e));
      if (w < rep) {
        const float ss = wave_sum(v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w);
        const float r = rsqrt_f(ss / (float)kHd + a.eps);
        qn[w * kHd + d + 0] = (v.x * r) * (1.0f + qw.x);
        qn[w * kHd + d + 1] = (v.y * r) * (1.0f + qw.y);
        qn[w * kHd + d + 2] = (v.z * r) * (1.0f + qw.z);
        qn[w * kHd + d + 3] = (v.w * r) * (1.0f + qw.w);
      } else if (w == rep) {
        const float ss = wave_sum(v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w);
        const float r = rsqrt_f(ss / (float)kHd + a.eps);
        kn[d + 0] = (v.x * r) * (1.0f + kw.x);
        kn[d + 1] = (v.y * r) * (1.0f + kw.y);
        kn[d + 2] = (v.z * r) * (1.0f + kw.z);
        kn[d + 3] = (v.w * r) * (1.0f + kw.w);
      } else {
        *reinterpret_cast<float4*>(&vn[d]) = v;
      }
    }
    __syncthreads();
    if (*sh.fail) return false;
    // RoPE on dims [0, rot): x' = x*cos + rotate_half(x)*sin
    const int half = a.rot / 2;
    const int nrot = rep + (has_new ? 1 : 0);
    for (int e2 = tid; e2 < nrot * a.rot; e2 += kT) {
      const int hh = e2 / a.rot, ii = e2 % a.rot;
      const float* src = (hh < rep) ? qn + hh * kHd : kn;
      const float rh = (ii < half) ? -src[ii + half] : src[ii - half];
      rtmp[hh * kHd + ii] = src[ii] * csv + rh * snv;
    }
    __syncthreads();
    for (int e2 = tid; e2 < nrot * a.rot; e2 += kT) {
      const int hh = e2 / a.rot, ii = e2 % a.rot;
      if (hh < rep) qn[hh * kHd + ii] = rtmp[hh * kHd + ii];
      else kn[ii] = rtmp[hh * kHd + ii];
    }
    __syncthreads();
    float* Kc = L.kc + (size_t)g * a.tmax * kHd;
    float* Vc = L.vc + (size_t)g * a.tmax * kHd;
    if (has_new) {  // append post-RoPE k and raw v at row p
      if (tid < kHd) st_agent(&Kc[(size_t)p * kHd + tid], kn[tid]);
      else st_agent(&Vc[(size_t)p * kHd + tid - kHd], vn[tid - kHd]);
    }
    float q4[kMaxRep][4];
#pragma unroll
    for (int h = 0; h < kMaxRep; ++h)
#pragma unroll
      for (int e2 = 0; e2 < 4; ++e2) q4[h][e2] = (h < rep) ? qn[h * kHd + 4 * lane + e2] : 0.f;
    auto score = [&](int tt, float4 kv) {
#pragma unroll
      for (int h = 0; h < kMaxRep; ++h) {
        if (h >= rep) break;
        float dd = q4[h][0] * kv.x + q4[h][1] * kv.y + q4[h][2] * kv.z + q4[h][3] * kv.w;
        dd = wave_sum(dd);
        if (lane == 0) sc[h * MC + tt] = dd * a.ascale;
      }
    };
    auto ld4 = [&](const float* q) {
      return make_float4(ld_agent(q), ld_agent(q + 1), ld_agent(q + 2), ld_agent(q + 3));
    };
    const float4 kn4 = *reinterpret_cast<const float4*>(&kn[4 * lane]);
#pragma unroll
    for (int j = 0; j < kAttnPf; ++j) {  // rows held since before the inputs (first item)
      const int tt = wid + kNW * j;
      if (tt >= len) break;  // uniform
      const int tr = t0 + tt;
      const float4 kv = (tr == p) ? kn4 : (first ? kp[j] : ld4(&Kc[(size_t)tr * kHd + 4 * lane]));
      score(tt, kv);
    }
    for (int tt = wid + kNW * kAttnPf; tt < len; tt += kNW) {
      const int tr = t0 + tt;
      score(tt, (tr == p) ? kn4 : ld4(&Kc[(size_t)tr * kHd + 4 * lane]));
    }
    __syncthreads();
    for (int h = wid; h < rep; h += kNW) {
      float mx = -INFINITY;
      for (int tt = lane; tt < len; tt += 64) mx = fmaxf(mx, sc[h * MC + tt]);
      mx = wave_max(mx);
      float l = 0.f;
      for (int tt = lane; tt < len; tt += 64) {
        const float pe = expf(sc[h * MC + tt] - mx);
        sc[h * MC + tt] = pe;
        l += pe;
      }
      l = wave_sum(l);
      if (lane == 0) { hm[h] = mx; hl[h] = l; }
    }
    __syncthreads();
    float acc[kMaxRep][4];
#pragma unroll
    for (int h = 0; h < kMaxRep; ++h)
#pragma unroll
      for (int e2 = 0; e2 < 4; ++e2) acc[h][e2] = 0.f;
    auto pv = [&](int tt, float4 vv) {
#pragma unroll
      for (int h = 0; h < kMaxRep; ++h) {
        if (h >= rep) break;
        const float pe = sc[h * MC + tt];
        acc[h][0] += pe * vv.x; acc[h][1] += pe * vv.y; acc[h][2] += pe * vv.z; acc[h][3] += pe * vv.w;
      }
    };
    const float4 vn4 = *reinterpret_cast<const float4*>(&vn[4 * lane]);
#pragma unroll
    for (int j = 0; j < kAttnPf; ++j) {
      const int tt = wid + kNW * j;
      if (tt >= len) break;  // uniform
      const int tr = t0 + tt;
      pv(tt, (tr == p) ? vn4 : (first ? vp[j] : ld4(&Vc[(size_t)tr * kHd + 4 * lane])));
    }
    for (int tt = wid + kNW * kAttnPf; tt < len; tt += kNW) {
      const int tr = t0 + tt;
      pv(tt, (tr == p) ? vn4 : ld4(&Vc[(size_t)tr * kHd + 4 * lane]));
    }
#pragma unroll
    for (int h = 0; h < kMaxRep; ++h)
      *reinterpret_cast<float4*>(&ored[(wid * kMaxRep + h) * kHd + 4 * lane]) = make_float4(acc[h][0], acc[h][1], acc[h][2], acc[h][3]);
    __syncthreads();
    const size_t pc = (size_t)g * a.att_nmax + c;
    for (int e2 = tid; e2 < rep * kHd; e2 += kT) {
      const int h = e2 / kHd, d = e2 % kHd;
      float o = 0.f;
#pragma unroll
      for (int w2 = 0; w2 < kNW; ++w2) o += ored[(w2 * kMaxRep + h) * kHd + d];
      st_agent64(&a.att_o[(pc * kMaxRep + h) * kHd + d], tagged(o, tag));
    }
    if (tid < rep) {
      st_agent64(&a.att_ml[pc * 2 * kMaxRep + tid], tagged(hm[tid], tag));
      st_agent64(&a.att_ml[pc * 2 * kMaxRep + kMaxRep + tid], tagged(hl[tid], tag));
    }
    __syncthreads();
  }
  return true;
}

// ------------------------------------------------------------------ lm_head + argmax
// Tied embedding [V][H] as lm_head (kernels.rs:251-291): wave w owns R rows per block step,
// lane l reads the 16-byte chunks 16*(l + 64c), c < CPW, of each row; two steps of loads
// (2 x 8 per lane, 128 KB per block) are kept in flight.  Block argmax (reference order,
// ArgOrder) -> argp, tagged with the token.  Also clears the next token's accumulators.
template <int CPW>
Q35_DEV bool lm_stage(const StepArgs& a, const Tok& t, const Shared& sh) {
  constexpr int R = 8 / CPW;
  constexpr int RPB = kNW * R;
  const int tid = tix(), lane = tid & 63, wid = tid >> 6;
  const int K = a.H, nbK = K >> 6;
  const int nrb = (a.V + RPB - 1) / RPB;
  uint4 wa[R][CPW], wb[R][CPW];
  float sa[R][CPW], sb[R][CPW];
  auto load = [&](int rb, uint4 (&wv)[R][CPW], float (&sv)[R][CPW]) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int row = rb * RPB + wid * R + r;
#pragma unroll
      for (int c = 0; c < CPW; ++c) {
        // branch-free: clamped into the table; compute() drops rows past V and chunks past K
        const uint32_t rw = (uint32_t)min(row, a.V - 1), k = (uint32_t)min(16 * (lane + 64 * c), K - 16);
        wv[r][c] = ldg16_nt(a.emb_q + (rw * (uint32_t)K + k));
        sv[r][c] = ldg_nt(a.emb_s + (rw * (uint32_t)nbK + (k >> 6)));
      }
    }
  };
  float* xs = sh.smem;
  float best_v = -INFINITY;
  int best_i = INT_MAX;
  auto compute = [&](int rb, const uint4 (&wv)[R][CPW], const float (&sv)[R][CPW]) {
    float pr[R];
#pragma unroll
    for (int r = 0; r < R; ++r) pr[r] = 0.f;
#pragma unroll
    for (int c = 0; c < CPW; ++c) {
      const int k = 16 * (lane + 64 * c);
      if (k >= K) continue;
      float xv[16];
      const float4* xp = reinterpret_cast<const float4*>(&xs[k]);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float4 tq = xp[q];
        xv[4 * q] = tq.x; xv[4 * q + 1] = tq.y; xv[4 * q + 2] = tq.z; xv[4 * q + 3] = tq.w;
      }
#pragma unroll
      for (int r = 0; r < R; ++r) {
        float f[16];
        unpack16(wv[r][c], f);
        float dd = 0.f;
#pragma unroll
        for (int e = 0; e < 16; ++e) dd += f[e] * xv[e];
        pr[r] += dd * sv[r][c];
      }
    }
    const float v = fold_rows<R>(pr, lane);
    const int row = rb * RPB + wid * R + lane / (64 / R);
    if ((lane % (64 / R)) == 0 && row < a.V) {
      if (a.logits) stg(a.logits + row, v);
      if (argmax_better(v, row, best_v, best_i, a.ord)) { best_v = v; best_i = row; }
    }
  };
  const int rb0 = bix(), gs = gridDim.x;
  if (rb0 < nrb) load(rb0, wa, sa);
  // the second row block is issued behind the norm's inputs (rows clamped: always in the table)
  fx_t hraw[2 * CPW];
  const bool ok = pro_rms<2 * CPW, false, fx_t>(a, HSrc{t.h, t.hc}, hraw, K, a.final_norm, 0, K, xs, sh.shs,
                                         [&]() { load(rb0 + gs, wb, sb); });
  if (!ok) *sh.fail = 1;
  __syncthreads();
  if (*sh.fail) return false;
  {
    // clear the other parity set (the next token's residual stream and accumulators): the last
    // readers of it were the previous token's, and every block finished those before this token
    // (of the stream copies only the words in use: 16 of every 32)
    const int64_t nh = (int64_t)a.n_res * a.H, na = a.acc_par, n = nh + na;
    fx_t* hz = a.h + (size_t)((t.ti + 1) & 1) * 2 * nh;
    fx_t* az = a.acc + (size_t)((t.ti + 1) & 1) * na;
    const int64_t per = (n + gs - 1) / gs, lo = (int64_t)bix() * per, hi = min(n, lo + per);
    for (int64_t q = lo + tid; q < hi; q += kT) st_agent(q < nh ? &hz[q + (q & ~15)] : &az[q - nh], (fx_t)0);
  }
  for (int rb = rb0; rb < nrb; rb += 2 * gs) {
    if (rb != rb0 && rb + gs < nrb) load(rb + gs, wb, sb);
    compute(rb, wa, sa);
    if (rb + gs >= nrb) break;
    if (rb + 2 * gs < nrb) load(rb + 2 * gs, wa, sa);
    compute(rb + gs, wb, sb);
  }
  block_argmax(best_v, best_i, sh.shv, sh.shi, a.ord);
  // every store of the block in this token (the clearing, KV rows, DeltaNet and conv states)
  // completes before the partial that the next token's blocks wait for
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (tid == 0) st_agent64(&a.argp[(size_t)(t.ti & 1u) * gs + bix()], arg_pack(best_v, best_i, t.ti));
  return true;
}

// After an odd number of steps the newest recurrent and conv states are in the second copies:
// copy them back, so that every launch starts and ends with the state in rec / conv_state.
// Float4 elements over all layers, kB per thread in flight.
Q35_DEV void state_copy_back(const StepArgs& a) {
  constexpr int kB = 8;
  const int64_t gt = (int64_t)bix() * kT + tix(), gs = (int64_t)gridDim.x * kT;
  const int64_t nr = (int64_t)a.nh * kDk * a.dv / 4, nc = (int64_t)a.conv_dim * 3 / 4, per = nr + nc;
  const int64_t total = (int64_t)a.n_layers * per;
  for (int64_t e0 = gt; e0 < total; e0 += kB * gs) {
    float4 v[kB];
    float* dst[kB];
#pragma unroll
    for (int u = 0; u < kB; ++u) {
      const int64_t e = e0 + u * gs;
      dst[u] = nullptr;
      if (e < total) {
        const int l = (int)(e / per);
        const int64_t r = e - (int64_t)l * per;
        const StepLayer& L = a.layers[l];
        if (!L.full) {
          const float* src = r < nr ? L.rec_alt + 4 * r : L.conv_alt + 4 * (r - nr);
          dst[u] = r < nr ? L.rec + 4 * r : L.conv_state + 4 * (r - nr);
          v[u] = make_float4(ld_agent(src), ld_agent(src + 1), ld_agent(src + 2), ld_agent(src + 3));
        }
      }
    }
#pragma unroll
    for (int u = 0; u < kB; ++u) {
      if (dst[u] == nullptr) continue;
      st_agent(dst[u] + 0, v[u].x);
      st_agent(dst[u] + 1, v[u].y);
      st_agent(dst[u] + 2, v[u].z);
      st_agent(dst[u] + 3, v[u].w);
    }
  }
}

// ------------------------------------------------------------------ the kernel
template <int CPW, int MC, bool STREAM>
__global__ __launch_bounds__(kT) void step_kernel(const StepArgs a) {
  constexpr int KR = 2 * CPW;  // hidden <= 256 CPW = 512 KR
  __shared__ __align__(16) float smem[smem_for(MC)];
  __shared__ __align__(16) float shs[kNW];
  __shared__ float shv[kNW];
  __shared__ int shi[kNW];
  __shared__ int fail;
  const Shared sh{smem, shs, shv, shi, &fail};
  // a failed earlier launch left the model state invalid: do nothing until a reset
  if (ld_agent(a.err) != 0u) return;
  if (tix() == 0) fail = 0;
  __syncthreads();
  const int p0 = ldg(a.pos);
  const uint32_t ts0 = ld_agent(a.tokseq);
  int executed = a.ntok, stop_tok = 0;
  for (int i = 0; i < a.ntok && executed == a.ntok; ++i) {
    const int p = p0 + i;
    Tok t;
    t.ti = ts0 + (uint32_t)i;
    const int par = (int)(t.ti & 1u);
    t.hn = a.h + (size_t)par * a.n_res * 2 * a.H;  // the first copy: the embedding row + the first mixer
    t.h = t.hn;
    fx_t* acc0 = a.acc + (size_t)par * a.acc_par;
    t.hc = 0;
    // after a residual stage: its copy is the stream (a word holds the stage's chunk contributions,
    // the first chunk's carrying the previous copy, and in the first copy the embedding row)
    auto advance = [&](int kind, bool more) {
      t.hc = (t.h == t.hn ? 1u : 0u) + (uint32_t)a.mv[kind].nchunk;
      t.h = t.hn;
      if (more) t.hn += 2 * a.H;
    };
    for (int l = 0; l < a.n_layers; ++l) {
      CLayer& L = layer_at(a, l);
      t.l = l;
      t.acc = acc0 + (size_t)l * a.acc_stride;
      const int pro0 = (l == 0) ? PRO_EMBED_RMS : PRO_RMS;
      int r;
      if (!L.full) {
        r = mv_stage<kU, KR, STREAM>(a, L, t, SMV_QKVZ, pro0, i, p, sh, &stop_tok);
        if (r == kStageStop) { executed = i; break; }
        if (r == kStageFail) return;
        if (!mv_stage<kUOut, KR>(a, L, t, SMV_OUT, PRO_GDN, i, p, sh)) return;
        advance(SMV_OUT, true);
      } else {
        r = mv_stage<kU, KR, STREAM>(a, L, t, SMV_QKV, pro0, i, p, sh, &stop_tok);
        if (r == kStageStop) { executed = i; break; }
        if (r == kStageFail) return;
        if (!attn_stage<MC>(a, L, t, p, sh)) return;
        if (!mv_stage<kU, KR>(a, L, t, SMV_O, PRO_ATTN, i, p, sh)) return;
        advance(SMV_O, true);
      }
      if (!mv_stage<kU, KR>(a, L, t, SMV_GU, PRO_RMS, i, p, sh)) return;
      if (!mv_stage<kU, KR>(a, L, t, SMV_DOWN, PRO_SWIGLU, i, p, sh)) return;
      advance(SMV_DOWN, l + 1 < a.n_layers);  // the last copy is read by the lm stage
    }
    if (executed != a.ntok) break;
    if (!lm_stage<CPW>(a, t, sh)) return;
  }
  // Every block has read all argmax partials of the last executed step (or passed its lm stage),
  // so all state writes of the launch are complete and ordered before this point.
  if (executed & 1) state_copy_back(a);
  // tail: block 0 turns the last step's block argmaxes into the token
  if (bix() != 0) return;
  if (executed != a.ntok) {  // the stop id stays the next token; hist already holds it
    if (tix() == 0) {
      stg(a.token, (int32_t)stop_tok);
      stg(a.pos, (int32_t)(p0 + executed));
      st_agent((int32_t*)a.tokseq, (int32_t)(ts0 + (uint32_t)executed));
    }
    return;
  }
  int tok = 0;
  if (!reduce_argmax(a, ts0 + (uint32_t)a.ntok - 1u, sh, tok)) return;
  if (tix() == 0) {
    const int pl = p0 + a.ntok - 1;
    record_token<STREAM>(a, pl, tok);
    stg(a.token, (int32_t)tok);
    stg(a.pos, (int32_t)(pl + 1));
    st_agent((int32_t*)a.tokseq, (int32_t)(ts0 + (uint32_t)a.ntok));
  }
}

// The build for contexts of up to kMaxChunk tokens per attention item, or the long-context one
// (more LDS for the items' scores; kept apart because the larger allocation costs the common case
// ~0.5% in register allocation); each with and without the host token stream.
template <bool STREAM>
const void* kernel_for_t(int hidden, bool long_ctx) {
  if (long_ctx) {
    if (hidden <= 1024) return reinterpret_cast<const void*>(step_kernel<1, kMaxChunkLong, STREAM>);
    if (hidden <= 2048) return reinterpret_cast<const void*>(step_kernel<2, kMaxChunkLong, STREAM>);
    return reinterpret_cast<const void*>(step_kernel<4, kMaxChunkLong, STREAM>);
  }
  if (hidden <= 1024) return reinterpret_cast<const void*>(step_kernel<1, kMaxChunk, STREAM>);
  if (hidden <= 2048) return reinterpret_cast<const void*>(step_kernel<2, kMaxChunk, STREAM>);
  return reinterpret_cast<const void*>(step_kernel<4, kMaxChunk, STREAM>);
}
const void* kernel_for(int hidden, bool long_ctx, bool stream) {
  return stream ? kernel_for_t<true>(hidden, long_ctx) : kernel_for_t<false>(hidden, long_ctx);
}

}  // namespace

int step_grid(int hidden) {
  if (hidden < 64 || hidden > 4096) return 0;
  int dev = 0, ncu = 0, coop = 0, nb = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  if (hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  if (hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, dev) != hipSuccess || !coop) return 0;
  for (const bool lc : {false, true})
    for (const bool sm : {false, true})
      if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, kernel_for(hidden, lc, sm), kT, 0) != hipSuccess || nb < 1)
        return 0;
  return std::min(ncu, kT);  // one block per CU; the argmax reduction reads one partial per thread
}

int step_att_nmax(int grid, int kvh) { return std::max(1, std::min(kMaxNmax, grid / std::max(1, kvh))); }

int step_validate(const q35_dims& d, int tmax, int grid) {
  if (grid < 1) return fail(Q35_E_HIP, "persistent step: device cannot co-schedule the step kernel");
  if (d.hidden > 4096 || d.hidden > kRmsRegs * kT) return fail(Q35_E_SHAPE, "persistent step: hidden must be <= 4096");
  if (d.hidden % 64 != 0) return fail(Q35_E_SHAPE, "persistent step: hidden must be a multiple of 64");
  if (d.ffn > kRmsRegs * kT * 4) return fail(Q35_E_SHAPE, "persistent step: ffn too large");
  if (d.lin_dk != kDk || d.lin_dv != kDv || d.conv_k != 4)
    return fail(Q35_E_SHAPE, "persistent step: DeltaNet needs dk 128, dv 128, conv 4");
  if (d.head_dim != kHd || d.kv_heads < 1 || d.attn_heads % d.kv_heads != 0 || d.attn_heads / d.kv_heads > kMaxRep)
    return fail(Q35_E_SHAPE, "persistent step: attention needs head_dim 256 and <= 4 query heads per kv head");
  if (d.rot_dim < 2 || d.rot_dim > kHd || (d.rot_dim % 2) != 0 || (kT % d.rot_dim) != 0)
    return fail(Q35_E_SHAPE, "persistent step: rotary dims must be even, <= 256 and divide 512");
  if (d.vocab >= (int)kArgNone) return fail(Q35_E_SHAPE, "persistent step: vocabulary must be < 2^18 - 1");
  if ((long long)tmax > (long long)kMaxChunkLong * step_att_nmax(grid, d.kv_heads))
    return fail(Q35_E_SHAPE, "persistent step: tmax too large for the attention split");
  return Q35_OK;
}

// Items per stage: nchunk chunks of each tile, nchunk = floor(grid / tiles) (at least 1), chunk
// rows rounded up to 16 and at most 512 (more chunks, i.e. a second round, only beyond that).
// The out stage's chunk divides dv (its DeltaNet prologue serves one value head per item).
void step_plan(const q35_dims& d, int grid, StepMv* mv) {
  auto tiles = [](long long n) { return (int)((n + kTile - 1) / kTile); };
  const int nh = d.lin_heads, vdim = nh * d.lin_dv, key_dim = nh * d.lin_dk, conv_dim = 2 * key_dim + vdim;
  const int ah = d.attn_heads, kvh = d.kv_heads, hd = d.head_dim;
  struct S { int kind, tiles, K; } st[SMV_COUNT] = {
      {SMV_QKVZ, tiles(conv_dim) + tiles(vdim), d.hidden},
      {SMV_OUT, tiles(d.hidden), vdim},
      {SMV_QKV, tiles((long long)ah * hd * 2) + 2 * tiles((long long)kvh * hd), d.hidden},
      {SMV_O, tiles(d.hidden), ah * hd},
      {SMV_GU, 2 * tiles(d.ffn), d.hidden},
      {SMV_DOWN, tiles(d.hidden), d.ffn},
  };
  for (const S& s : st) {
    // at most 120 chunks: a residual word then gets < 128 contributions per stage, which keeps
    // every reader's window of possible counts below the counter's 256 (see the kernel)
    int nchunk = std::max(1, std::min(120, grid / s.tiles));
    int kch = (s.K + nchunk - 1) / nchunk;
    kch = (kch + 15) & ~15;
    if (kch > kKch) kch = kKch;
    if (s.kind == SMV_OUT) {
      int kc = d.lin_dv;
      while (kc > kch && kc % 32 == 0 && (s.K + kc / 2 - 1) / (kc / 2) <= 120) kc /= 2;
      kch = kc;
    }
    nchunk = (s.K + kch - 1) / kch;
    mv[s.kind] = StepMv{kch, nchunk};
  }
}

int step_launch(const StepArgs& a, int grid, hipStream_t st) {
  if (a.ntok < 1) return Q35_OK;
  if (!a.err || !a.tokseq || !a.argp || !a.hist) return fail(Q35_E_ARG, "persistent step: null error word, token counter or history");
  StepArgs args = a;
  void* params[] = {&args};
  const bool long_ctx = (long long)a.tmax > (long long)kMaxChunk * a.att_nmax;
  Q35_HIP_TRY(hipLaunchCooperativeKernel(kernel_for(a.H, long_ctx, a.tok_host != nullptr), dim3(grid), dim3(kT), params, 0, st));
  return Q35_OK;
}

}  // namespace q35
