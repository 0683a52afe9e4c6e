// Persistent decode step: the whole TextForCausalLM forward at seq_len 1 (model.rs:27-84,
// 113-129) plus the greedy argmax (main.rs:131), for `ntok` consecutive tokens, in ONE launch.
//
// Why: a decode step streams ~2 GB of Q8F weights through ~120 dependent stages.  As separate
// kernels every stage boundary costs a launch gap plus a ramp-up/drain with HBM idle; here the
// grid is one co-resident block per CU (cooperative launch) and stages are separated by a grid
// barrier.  Each block issues the weight loads of its next stage *between* arriving at the
// barrier and polling it, so the weight stream of stage s+1 overlaps the barrier latency and
// the tail of stage s.
//
// Stages per token (each ends with a grid barrier):
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
// Barrier: blocks arrive on one of 32 group counters (blockIdx % 32) with a non-returning
// atomic after their stores have completed; the waiting wave reads all group counters with one
// load per lane.  Counters only grow (they are zeroed by a model reset, never by a launch); the
// launch is told how many barriers earlier launches passed (bar_base), so the target of its
// n-th barrier is (blocks in group) * (bar_base + n), compared in wrapping uint32 arithmetic.
// Every wait is bounded: on time-out the block sets the sticky error word and returns, and the
// other blocks see the word and return too, so the grid always drains; a later launch that
// finds the word set returns at entry.
#include "q35_internal.h"

#include <algorithm>
#include <climits>

namespace q35 {

namespace {

constexpr int kT = kStepThreads;  // 512
constexpr int kNW = kT / 64;      // waves per block
constexpr int kTile = 256;
constexpr int kRG = kT / 16;      // matvec row groups (16 lanes cover a 256-byte tile row)
constexpr int kU = 16;            // rows per lane per item
constexpr int kKch = kRG * kU;    // rows per item, at most 512
constexpr int kRmsRegs = 8;       // RMSNorm prologue: K <= 8 * 512
constexpr int kGroups = 32;       // barrier counters
constexpr int kCtrStride = 64;    // uint32 words between counters (own 256-byte line each)
constexpr uint32_t kSpin = 1u << 20;
constexpr int kHd = 256;          // attention head dim
constexpr int kMaxRep = 4;        // query heads per kv head
constexpr int kMaxChunk = 256;    // cached tokens per attention item
constexpr int kMinChunk = 8;
constexpr int kMaxNmax = 256;     // attention chunks per kv head
constexpr int kMaxTouch = 8;      // norm groups / heads one matvec item's rows can span
constexpr int kDk = 128;          // DeltaNet key head dim
constexpr int kDv = 128;          // DeltaNet value head dim
constexpr int kGdnG = kStepThreads / kDv;  // DeltaNet state row groups (4)
constexpr int kGdnR = kDk / kGdnG;         // DeltaNet state rows per thread (32)
constexpr int kSmem = 12288;      // floats of LDS shared by all stages (48 KB)
constexpr int kMergeB = 16;       // attention-merge partials loaded per batch

// LDS carve-up (float offsets)
constexpr int kXs = 0;                  // matvec x chunk [kKch]
constexpr int kRed = kXs + kKch;        // matvec wave partials [kNW][kTile]; prologue scratch [kRG][kTile]
static_assert(kRed + kRG * kTile <= kSmem, "LDS");
static_assert(512 + 2 * kT + kDv <= kRG * kTile, "DeltaNet scratch fits in kRed");
static_assert(kKch <= kT, "one x element per thread in the gated / attention prologues");
static_assert(kMaxTouch * kMaxNmax + kT + kMaxTouch <= kRG * kTile, "attention merge scratch fits in kRed");

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
  int* ok;
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

Q35_DEV float4 ld4_agent(const float* p) {
  return make_float4(ld_agent(p), ld_agent(p + 1), ld_agent(p + 2), ld_agent(p + 3));
}
Q35_DEV float4 ld4_fx(const fx_t* p) {
  const fx_t a = ld_agent(p), b = ld_agent(p + 1), c = ld_agent(p + 2), d = ld_agent(p + 3);
  return make_float4(from_fx(a), from_fx(b), from_fx(c), from_fx(d));
}

// ------------------------------------------------------------------ grid barrier
struct Bar {
  uint32_t* ctr;
  uint32_t* err;
  uint32_t epoch;  // barriers passed so far by this block, counted from the counters' last reset
};

// Publishes this block's completion of the current stage: all of its memory operations are
// complete (s_waitcnt 0 in every wave, then the workgroup barrier) before the counter add.
Q35_DEV void bar_arrive(Bar& b) {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (tix() == 0)
    __hip_atomic_fetch_add((Q35_GLOBAL uint32_t*)&b.ctr[(bix() % kGroups) * kCtrStride], 1u, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
  b.epoch += 1;
}

// Waits until every block has arrived `epoch` times.  Wave 0 polls: lane g < 32 reads group
// counter g.  Returns false (in every thread of the block) on time-out or when another block
// has raised the error word.
Q35_DEV bool bar_wait(const Bar& b, int* sh_ok) {
  if (tix() < 64) {
    const int g = tix();
    const uint32_t nb = gridDim.x;
    const uint32_t per = g < kGroups ? (nb + kGroups - 1 - (uint32_t)g) / kGroups : 0u;
    const uint32_t target = per * b.epoch;  // wraps; compared as a signed difference below
    uint32_t spin = 0;
    bool ok = true;
    while (true) {
      const uint32_t v = g < kGroups ? ld_agent(&b.ctr[g * kCtrStride]) : target;
      const uint32_t e = ld_agent(b.err);
      if (__all((int32_t)(v - target) >= 0)) break;
      if (e != 0u || ++spin > kSpin) { ok = false; break; }
      __builtin_amdgcn_s_sleep(2);
    }
    if (tix() == 0) {
      if (!ok) __hip_atomic_fetch_or((Q35_GLOBAL uint32_t*)b.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      *sh_ok = ok ? 1 : 0;
    }
  }
  __syncthreads();
  return *sh_ok != 0;
}

// The layer table is never written by the kernel: read through the constant address space, its
// uniform fields are scalar loads (scalar cache) rather than vector loads that would queue behind
// the weight stream and force vmcnt waits.
typedef const __attribute__((address_space(4))) StepLayer CLayer;
Q35_DEV CLayer& layer_at(const StepArgs& a, int l) { return *(CLayer*)(a.layers + l); }

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

Q35_DEV Mv make_mv(const StepArgs& a, CLayer& L, int kind) {
  Mv d{};
  const StepMv pl = a.mv[kind];
  d.kch = pl.kch;
  d.nchunk = pl.nchunk;
  switch (kind) {
    case SMV_QKVZ:
      d.K = a.H;
      d.w0 = L.qkv_q; d.s0 = L.qkv_s; d.a0 = a.acc_proj; d.n0 = a.conv_dim;
      d.w1 = L.z_q; d.s1 = L.z_s; d.a1 = a.acc_proj + a.conv_dim; d.n1 = a.vdim;
      d.t1 = tiles_of(d.n0); d.t2 = d.t1 + tiles_of(d.n1); d.t3 = d.t2;
      break;
    case SMV_OUT:
      d.K = a.vdim;
      d.w0 = L.out_q; d.s0 = L.out_s; d.a0 = a.h; d.n0 = a.H; d.spm = ~15;
      d.t1 = d.t2 = d.t3 = tiles_of(d.n0);
      break;
    case SMV_QKV: {
      const int ldqg = a.ah * a.hd * 2, nkv = a.kvh * a.hd;
      d.K = a.H;
      d.w0 = L.q_q; d.s0 = L.q_s; d.a0 = a.acc_proj; d.n0 = ldqg;
      d.w1 = L.k_q; d.s1 = L.k_s; d.a1 = a.acc_proj + ldqg; d.n1 = nkv;
      d.w2 = L.v_q; d.s2 = L.v_s; d.a2 = a.acc_proj + ldqg + nkv; d.n2 = nkv;
      d.t1 = tiles_of(d.n0); d.t2 = d.t1 + tiles_of(d.n1); d.t3 = d.t2 + tiles_of(d.n2);
    } break;
    case SMV_O:
      d.K = a.ah * a.hd;
      d.w0 = L.o_q; d.s0 = L.o_s; d.a0 = a.h; d.n0 = a.H; d.spm = ~15;
      d.t1 = d.t2 = d.t3 = tiles_of(d.n0);
      break;
    case SMV_GU:
      d.K = a.H;
      d.w0 = L.gate_q; d.s0 = L.gate_s; d.a0 = a.acc_gu; d.n0 = a.F;
      d.w1 = L.up_q; d.s1 = L.up_s; d.a1 = a.acc_gu + a.F; d.n1 = a.F;
      d.t1 = tiles_of(d.n0); d.t2 = d.t1 + tiles_of(d.n1); d.t3 = d.t2;
      break;
    default:  // SMV_DOWN
      d.K = a.F;
      d.w0 = L.down_q; d.s0 = L.down_s; d.a0 = a.h; d.n0 = a.H; d.spm = ~15;
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

// y[tile cols] += sum over the item's rows of x[k] * dequant(W[k][cols]); x chunk in xs.  aux_dst
// (optional): one more sum, of which each wave holds its part in aux, reduced with the columns.
template <int U>
Q35_DEV void mv_compute(const MvItem& it, const MvPf<U>& pf, const float* xs, float* red, float aux = 0.f,
                        fx_t* aux_dst = nullptr) {
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
    fx_add(aux_dst, s);
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
    if (n < it.N) fx_add(&it.acc[n + (n & it.spm)], v);
  }
  __syncthreads();
}

// xs[i] = x[k0+i] * rsqrt(mean(x^2) + eps) * (1 + w[k0+i]); thread t holds x[t + 512 j],
// j < KR (K <= 512 KR).  All loads (x and the thread's norm weights) are issued before any value
// is used, and all KR of each (indices clamped, masked afterwards): a compile-time number of
// loads, so the compiler's waits on them are exact.  The prologue costs one round trip:
// `load(k)` returns the raw element, `conv` turns it into f32.  `post` (more weight loads of the
// caller) is issued behind the prologue's loads and before their first use; scheduling barriers
// keep the compiler from moving either group across it.
template <int KR, class Raw, class Load, class Conv, class Post>
Q35_DEV void pro_rms(Load load, Conv conv, int K, const float* w, float eps, int k0, int klen, float* xs,
                     float* shs, Post post) {
  const int tid = tix();
  Raw raw[KR];
  float wn[KR];
#pragma unroll
  for (int j = 0; j < KR; ++j) {
    const int k = tid + kT * j;
    raw[j] = load(min(k, K - 1));
    wn[j] = ldg(w + min(max(k, k0), k0 + klen - 1));
  }
  __builtin_amdgcn_sched_barrier(0);
  post();
  __builtin_amdgcn_sched_barrier(0);
  float v[KR];
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < KR; ++j) {
    v[j] = (tid + kT * j < K) ? conv(raw[j]) : 0.f;
    ss += v[j] * v[j];
  }
  // every caller reaches here right after a workgroup barrier (the stage's grid-barrier wait, or
  // the previous item's reduction), so the block sum needs no leading one
  ss = block_sum(ss, shs, false);
  const float r = rsqrt_f(ss * rcp_f((float)K) + eps);
#pragma unroll
  for (int j = 0; j < KR; ++j) {
    const int k = tid + kT * j;
    if (k >= k0 && k < k0 + klen) xs[k - k0] = (v[j] * r) * (1.0f + wn[j]);
  }
}

// the residual stream h (fixed point) as pro_rms input
struct HLoad {
  const fx_t* h;
  Q35_DEV fx_t operator()(int k) const { return ld_agent(h + (k + (k & ~15))); }
};
struct HConv {
  Q35_DEV float operator()(fx_t x) const { return from_fx(x); }
};
// a row of the Q8F embedding table as pro_rms input: (byte, block scale) pairs
struct EmbRaw {
  int8_t q;
  float s;
};
struct EmbLoad {
  const int8_t* q;
  const float* s;
  Q35_DEV EmbRaw operator()(int k) const { return EmbRaw{ldg(q + k), ldg(s + (k >> 6))}; }
};
struct EmbConv {
  Q35_DEV float operator()(EmbRaw x) const { return (float)x.q * x.s; }
};

// Token of step i at position p: the prompt id while p < plen, else the argmax of the previous
// step (reduced here from the per-block partials), or *token for the launch's first step.
// Block 0 records the previous step's argmax in hist.
Q35_DEV int select_token(const StepArgs& a, int i, int p, const Shared& sh) {
  int tok;
  if (i == 0) {
    tok = ld_agent(a.token);
  } else {
    float v = -INFINITY;
    int ix = INT_MAX;
    if (tix() < (int)gridDim.x) { v = ld_agent(&a.arg_v[tix()]); ix = ld_agent(&a.arg_i[tix()]); }
    block_argmax(v, ix, sh.shv, sh.shi, a.ord);
    tok = (ix == INT_MAX) ? 0 : ix;
    if (bix() == 0 && tix() == 0) st_agent(&a.hist[p - 1], tok);
  }
  if (p < ldg(a.plen)) tok = ldg(a.prompt + p);
  return tok;
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
// reads of the old state (their loads are issued before the barrier and may still be queued
// behind weight loads after it).
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

// Everything of the step that does not depend on the qkvz stage: issued before its barrier.
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

Q35_DEV void pro_gdn(const StepArgs& a, CLayer& L, const MvItem& it, int i, GdnPf& g, float* xs,
                     float* scratch) {
  const int tid = tix(), lane = tid & 63;
  const int j = tid % kDv, ig = tid / kDv;
  const int h = it.k0 / kDv, nch = 2 * kDk + kDv;
  float* qkv = scratch;          // [2dk + dv] conv outputs q | k | v of head h
  float* part0 = scratch + 512;  // [kT] per-row-group column partials
  float* part1 = part0 + kT;     // [kT]
  float* ov = part1 + kT;        // [dv] outputs of head h
  // qkvz-stage outputs: the thread's conv input, its z element and the two gate projections
  const int c = gdn_channel(a, h, min(tid, nch - 1));
  const fx_t xr = ld_agent(&a.acc_proj[c]);
  const fx_t zr = ld_agent(&a.acc_proj[a.conv_dim + it.k0 + min(tid, it.klen - 1)]);
  const float bs = from_fx(ld_agent(&a.acc_ba[(size_t)h * kStepBaStride]));
  const float as = from_fx(ld_agent(&a.acc_ba[(size_t)(a.nh + h) * kStepBaStride]));
  const float x = from_fx(xr);
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
  if (tid < it.klen) xs[tid] = (g.nw * (ov[it.k0 % kDv + tid] * rg)) * silu_f(from_fx(zr));
  // Off the path to the out_proj multiply-adds: the writer's new state S'' (column j) and conv
  // state [c] <- [s1, s2, x], stored while the multiply-adds run.
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
}

Q35_DEV void attn_chunking(const StepArgs& a, int T, int& chunk, int& nact) {
  chunk = max(kMinChunk, (T + a.att_nmax - 1) / a.att_nmax);
  nact = (T + chunk - 1) / chunk;
}

// o_proj input: merge the split-T partials of each touched query head (flash-decoding merge,
// chunks in order) and apply the sigmoid output gate (text_modules.rs:936).
Q35_DEV void pro_attn(const StepArgs& a, int T, int k0, int klen, float* xs, float* scratch) {
  const int tid = tix(), lane = tid & 63, wid = tid >> 6;
  const int rep = a.ah / a.kvh;
  int chunk, nact;
  attn_chunking(a, T, chunk, nact);
  float* wts = scratch;                         // [kMaxTouch][kMaxNmax] exp(m_c - M)
  float* pbuf = scratch + kMaxTouch * kMaxNmax; // [kT] per-part sums
  float* wl = pbuf + kT;                        // [kMaxTouch] L
  const int h0 = k0 / kHd, h1 = (k0 + klen - 1) / kHd;
  // Thread (part, i): output element k0 + i, chunks part, part + parts, ...  The partial outputs
  // do not depend on the statistics, so the first batch is issued with them: one round trip.
  const int parts = klen <= 64 ? 8 : (klen <= 128 ? 4 : (klen <= 256 ? 2 : 1));
  const int span = kT / parts;
  const int i = tid % span, part = tid / span;
  const int kk = k0 + min(i, klen - 1), hk = kk / kHd;  // clamped; masked below
  const float* og = a.att_o + ((size_t)(hk / rep) * a.att_nmax * kMaxRep + hk % rep) * kHd + kk % kHd;  // + c*kMaxRep*kHd
  float v0[kMergeB];
#pragma unroll
  for (int j = 0; j < kMergeB; ++j) v0[j] = ld_agent(&og[(size_t)min(part + j * parts, nact - 1) * kMaxRep * kHd]);
  // the thread's output gate (klen <= 512 = threads), loaded with the chunk statistics
  const int kg = k0 + min(tid, klen - 1);
  const fx_t graw = ld_agent(&a.acc_proj[(size_t)(kg / kHd) * 2 * kHd + kHd + kg % kHd]);
  for (int hh = h0 + wid; hh <= h1; hh += kNW) {
    const int g = hh / rep, hr = hh % rep;
    const float* ml = a.att_ml + (size_t)g * a.att_nmax * 2 * kMaxRep;
    float mv[kMaxNmax / 64], lv[kMaxNmax / 64];  // chunk c = lane + 64q (clamped; masked below)
#pragma unroll
    for (int q = 0; q < kMaxNmax / 64; ++q) {
      const int c = min(lane + 64 * q, nact - 1);
      mv[q] = ld_agent(&ml[c * 2 * kMaxRep + hr]);
      lv[q] = ld_agent(&ml[c * 2 * kMaxRep + kMaxRep + hr]);
    }
    float M = -INFINITY;
#pragma unroll
    for (int q = 0; q < kMaxNmax / 64; ++q) M = fmaxf(M, (lane + 64 * q < nact) ? mv[q] : -INFINITY);
    M = wave_max(M);
    float Ls = 0.f;
#pragma unroll
    for (int q = 0; q < kMaxNmax / 64; ++q) {
      const int c = lane + 64 * q;
      const float w = expf(mv[q] - M);
      if (c < nact) {
        wts[(hh - h0) * kMaxNmax + c] = w;
        Ls += lv[q] * w;
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
    for (int j = 0; j < kMergeB; ++j) o += (part + j * parts < nact) ? v0[j] * wc[j] : 0.f;
    for (int c0 = part + kMergeB * parts; c0 < nact; c0 += kMergeB * parts) {
      float v[kMergeB];  // all of a batch in flight at once (clamped; masked below)
#pragma unroll
      for (int j = 0; j < kMergeB; ++j) v[j] = ld_agent(&og[(size_t)min(c0 + j * parts, nact - 1) * kMaxRep * kHd]);
      float wv[kMergeB];
#pragma unroll
      for (int j = 0; j < kMergeB; ++j) wv[j] = w[min(c0 + j * parts, nact - 1)];
#pragma unroll
      for (int j = 0; j < kMergeB; ++j) o += (c0 + j * parts < nact) ? v[j] * wv[j] : 0.f;
    }
  }
  pbuf[part * span + i] = o;
  __syncthreads();
  if (tid < klen) {
    float s = 0.f;
    for (int q = 0; q < parts; ++q) s += pbuf[q * span + tid];
    const int hh = (k0 + tid) / kHd;
    xs[tid] = (s * rcp_f(wl[hh - h0])) * sigmoid_f(from_fx(graw));
  }
}

// Block bix()'s contiguous share of p[0, n) set to zero, one element per thread.
Q35_DEV void zero_share(fx_t* p, int n) {
  const int nb = (int)gridDim.x, per = (n + nb - 1) / nb, lo = bix() * per, hi = min(n, lo + per);
  for (int i = lo + tix(); i < hi; i += kT) st_agent(&p[i], (fx_t)0);
}

// Side tasks of a stage (their inputs are final after its barrier, their outputs are not read
// before the next one), spread evenly over the grid and issued behind the prologue's loads: a
// block's loads would otherwise wait for its stores' acknowledgements (vmcnt counts both, in
// order), and the few blocks holding all the stores arrived last.
Q35_DEV void side_tasks(const StepArgs& a, int kind) {
  if (kind == SMV_QKVZ || kind == SMV_QKV) {  // gate|up accumulator: last read by the previous down stage
    zero_share(a.acc_gu, 2 * a.F);
  } else if (kind == SMV_GU) {  // projection + gate accumulators: last read by the out / o stage
    zero_share(a.acc_proj, (int)a.acc_zero_n);
    if (bix() == gridDim.x - 1 && tix() < 2 * a.nh) st_agent(&a.acc_ba[tix() * kStepBaStride], (fx_t)0);
  }
}

// One matvec stage.  The in_proj_b / in_proj_a gate projection (f32, [H][nh] each,
// kernels.rs:174-247) rides on the qkvz stage: the item of tile t < 2*nh also forms the partial
// dot product of its rows with column t of [W_b | W_a].  U: rows per lane the stage's items need;
// KR: hidden-size elements per thread in the RMSNorm prologue (hidden <= 512 KR).
// Returns kStageOk, kStageFail (barrier time-out) or, for the first stage of a step, kStageStop
// (the step's input token is a stop id; *stop_tok receives it, nothing of the step has run).
template <int U, int KR>
Q35_DEV int mv_stage(const StepArgs& a, CLayer& L, int kind, int pro, int i, int p, Bar& bar,
                     const Shared& sh, int* stop_tok = nullptr) {
  const Mv d = make_mv(a, L, kind);
  const int nitems = d.t3 * d.nchunk;
  int item = bix();
  if (kind == SMV_GU) {
    // The out stage's state writers (out items with tile 0 and k0 % dv == 0, i.e. blocks b < nh cph
    // with b % cph == 0) arrive last and so issue this stage's weights last: a permutation of
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
  if (item < nitems) {
    it = mv_item(d, item);
    mv_load(it, d.K, pf);
    if (pro == PRO_GDN) gdn_load(a, L, it, i, gp);
  }
  if (!bar_wait(bar, sh.ok)) return kStageFail;
  int tok = 0;
  // Blocks with an item need the token for the embedding; with stop ids every block forms it,
  // so that every block sees a stop (without them the idle blocks go straight to their side
  // tasks, whose stores would otherwise wait behind the token's reduction).
  if (pro == PRO_EMBED_RMS && (item < nitems || a.n_stop > 0)) {
    tok = select_token(a, i, p, sh);
    if (is_stop(a, p, tok)) {
      if (stop_tok) *stop_tok = tok;
      return kStageStop;
    }
  }
  if (item >= nitems) side_tasks(a, kind);  // blocks with an item run them in the prologue
  float* xs = sh.smem + kXs;
  float* red = sh.smem + kRed;
  for (bool first = true; item < nitems; item += gridDim.x, first = false) {
    if (!first) {
      it = mv_item(d, item);
      mv_load(it, d.K, pf);
      if (pro == PRO_GDN) gdn_load(a, L, it, i, gp);
    }
    // the qkvz item's gate column (a 64-byte-strided gather) is issued behind the norm's inputs,
    // not ahead of the barrier poll
    auto aux_load = [&]() {
      if (kind == SMV_QKVZ && it.tile < naux && first) {  // row clamped; masked where it is used
        const float* W = it.tile < a.nh ? L.w_b : L.w_a;
        auxw = ldg(W + ((size_t)(it.k0 + min(tix(), it.klen - 1)) * a.nh + (it.tile % a.nh)));
      }
      if (first) side_tasks(a, kind);
    };
    switch (pro) {
      case PRO_EMBED_RMS: {
        const int K = d.K, nbK = K >> 6;
        const EmbLoad src{a.emb_q + (size_t)tok * K, a.emb_s + (size_t)tok * nbK};
        pro_rms<KR, EmbRaw>(src, EmbConv{}, K, L.in_norm, a.eps, it.k0, it.klen, xs, sh.shs, aux_load);
        if (bix() == 0 && first)  // the residual stream starts as the embedding row
          for (int k = tix(); k < K; k += kT) st_agent(&a.h[k + (k & ~15)], to_fx(EmbConv{}(src(k))));
      } break;
      case PRO_RMS:
        pro_rms<KR, fx_t>(HLoad{a.h}, HConv{}, d.K, kind == SMV_GU ? L.post_norm : L.in_norm, a.eps, it.k0, it.klen,
                          xs, sh.shs, aux_load);
        break;
      case PRO_GDN:
        pro_gdn(a, L, it, i, gp, xs, red);
        break;
      case PRO_SWIGLU: {  // klen <= 512 = threads: one element per thread
        const int k = it.k0 + min(tix(), it.klen - 1);
        const fx_t up = ld_agent(&a.acc_gu[a.F + k]), gate = ld_agent(&a.acc_gu[k]);
        if (tix() < it.klen) xs[tix()] = from_fx(up) * silu_f(from_fx(gate));
      } break;
      default:  // PRO_ATTN: merged attention output
        pro_attn(a, p + 1, it.k0, it.klen, xs, red);
        break;
    }
    __syncthreads();
    // in_proj_b | in_proj_a column it.tile: each wave's part of the dot product goes into the
    // matvec reduction (further columns, when there are more than tiles, reduce on their own)
    float auxp = 0.f;
    fx_t* auxd = nullptr;
    if (kind == SMV_QKVZ) {
      for (int o = it.tile; o < naux; o += d.t3) {
        float w = auxw;
        if (o != it.tile || !first) {
          const float* W = o < a.nh ? L.w_b : L.w_a;
          w = ldg(W + ((size_t)(it.k0 + min(tix(), it.klen - 1)) * a.nh + (o % a.nh)));
        }
        const float v = (tix() < it.klen) ? xs[tix()] * w : 0.f;
        if (o == it.tile) {
          auxp = wave_sum(v);
          auxd = &a.acc_ba[(size_t)o * kStepBaStride];
        } else {
          const float s = block_sum(v, sh.shs);
          if (tix() == 0) fx_add(&a.acc_ba[(size_t)o * kStepBaStride], s);
        }
      }
    }
    mv_compute(it, pf, xs, red, auxp, auxd);
  }
  bar_arrive(bar);
  return kStageOk;
}

// ------------------------------------------------------------------ attention partials
// Item (kv head g, chunk c of `chunk` cached tokens) for the rep query heads of g
// (text_modules.rs:842-944): q/k RMSNorm (1+w), partial RoPE (:739-774), KV append at p
// (the item holding p), scores, chunk softmax statistics and P.V.
//
// Nothing the qkv stage writes is needed to fetch the first item's cached K / V rows t < p
// (written by earlier steps), the q / k norm weights and the thread's RoPE factors, so they are
// loaded before the barrier: after it the stage has one memory round trip (its q, k, v inputs)
// instead of four.  Wave w holds rows t0 + w + 8j, j < kAttnPf; rows beyond are loaded in-stage.
constexpr int kAttnPf = 2;
Q35_DEV bool attn_stage(const StepArgs& a, CLayer& L, int p, Bar& bar, const Shared& sh) {
  const int tid = tix(), lane = tid & 63, wid = tid >> 6;
  const int T = p + 1, rep = a.ah / a.kvh;
  int chunk, nact;
  attn_chunking(a, T, chunk, nact);
  float4 kp[kAttnPf], vp[kAttnPf];
  {
    const int it0 = min((int)bix(), a.kvh * nact - 1);
    const int g = it0 / nact, t0 = (it0 % nact) * chunk;
    const float* Kc = L.kc + (size_t)g * a.tmax * kHd;
    const float* Vc = L.vc + (size_t)g * a.tmax * kHd;
#pragma unroll
    for (int j = 0; j < kAttnPf; ++j) {  // clamped to written rows; the row at p comes from LDS
      const int t = max(0, min(t0 + wid + kNW * j, p - 1));
      kp[j] = ld4_agent(&Kc[(size_t)t * kHd + 4 * lane]);
      vp[j] = ld4_agent(&Vc[(size_t)t * kHd + 4 * lane]);
    }
  }
  const float4 qw = make_float4(ldg(L.q_norm + 4 * lane), ldg(L.q_norm + 4 * lane + 1), ldg(L.q_norm + 4 * lane + 2),
                                ldg(L.q_norm + 4 * lane + 3));
  const float4 kw = make_float4(ldg(L.k_norm + 4 * lane), ldg(L.k_norm + 4 * lane + 1), ldg(L.k_norm + 4 * lane + 2),
                                ldg(L.k_norm + 4 * lane + 3));
  const float csv = ldg(a.rope_cos + (size_t)p * a.rot + tid % a.rot);  // rot divides 512: the same
  const float snv = ldg(a.rope_sin + (size_t)p * a.rot + tid % a.rot);  // element in every round
  if (!bar_wait(bar, sh.ok)) return false;
  float* qn = sh.smem;               // [kMaxRep][kHd]
  float* kn = qn + kMaxRep * kHd;    // [kHd]
  float* vn = kn + kHd;              // [kHd]
  float* rtmp = vn + kHd;            // [kMaxRep + 1][kHd]
  float* sc = rtmp + (kMaxRep + 1) * kHd;  // [kMaxRep][kMaxChunk]
  float* ored = sc + kMaxRep * kMaxChunk;  // [kNW][kMaxRep][kHd]
  float* hm = ored + kNW * kMaxRep * kHd;  // [kMaxRep]
  float* hl = hm + kMaxRep;                // [kMaxRep]
  const int ldqg = a.ah * kHd * 2;
  for (int item = bix(), first = 1; item < a.kvh * nact; item += gridDim.x, first = 0) {
    const int g = item / nact, c = item % nact;
    const int t0 = c * chunk, len = min(chunk, T - t0);
    const bool has_new = (c == nact - 1);
    for (int w = wid; w < rep + (has_new ? 2 : 0); w += kNW) {
      const int d = 4 * lane;
      if (w < rep) {
        const float4 v = ld4_fx(&a.acc_proj[(size_t)(g * rep + w) * 2 * kHd + d]);
        const float ss = wave_sum(v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w);
        const float r = rsqrt_f(ss / (float)kHd + a.eps);
        qn[w * kHd + d + 0] = (v.x * r) * (1.0f + qw.x);
        qn[w * kHd + d + 1] = (v.y * r) * (1.0f + qw.y);
        qn[w * kHd + d + 2] = (v.z * r) * (1.0f + qw.z);
        qn[w * kHd + d + 3] = (v.w * r) * (1.0f + qw.w);
      } else if (w == rep) {
        const float4 v = ld4_fx(&a.acc_proj[ldqg + (size_t)g * kHd + d]);
        const float ss = wave_sum(v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w);
        const float r = rsqrt_f(ss / (float)kHd + a.eps);
        kn[d + 0] = (v.x * r) * (1.0f + kw.x);
        kn[d + 1] = (v.y * r) * (1.0f + kw.y);
        kn[d + 2] = (v.z * r) * (1.0f + kw.z);
        kn[d + 3] = (v.w * r) * (1.0f + kw.w);
      } else {
        const float4 v = ld4_fx(&a.acc_proj[ldqg + (size_t)(a.kvh + g) * kHd + d]);
        *reinterpret_cast<float4*>(&vn[d]) = v;
      }
    }
    __syncthreads();
    // RoPE on dims [0, rot): x' = x*cos + rotate_half(x)*sin
    const int half = a.rot / 2;
    const int nrot = rep + (has_new ? 1 : 0);
    for (int e = tid; e < nrot * a.rot; e += kT) {
      const int hh = e / a.rot, ii = e % a.rot;
      const float* src = (hh < rep) ? qn + hh * kHd : kn;
      const float rh = (ii < half) ? -src[ii + half] : src[ii - half];
      rtmp[hh * kHd + ii] = src[ii] * csv + rh * snv;
    }
    __syncthreads();
    for (int e = tid; e < nrot * a.rot; e += kT) {
      const int hh = e / a.rot, ii = e % a.rot;
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
      for (int e = 0; e < 4; ++e) q4[h][e] = (h < rep) ? qn[h * kHd + 4 * lane + e] : 0.f;
    auto score = [&](int tt, float4 kv) {
#pragma unroll
      for (int h = 0; h < kMaxRep; ++h) {
        if (h >= rep) break;
        float dd = q4[h][0] * kv.x + q4[h][1] * kv.y + q4[h][2] * kv.z + q4[h][3] * kv.w;
        dd = wave_sum(dd);
        if (lane == 0) sc[h * kMaxChunk + tt] = dd * a.ascale;
      }
    };
    const float4 kn4 = *reinterpret_cast<const float4*>(&kn[4 * lane]);
#pragma unroll
    for (int j = 0; j < kAttnPf; ++j) {  // rows held since before the barrier (first item)
      const int tt = wid + kNW * j;
      if (tt >= len) break;  // uniform
      const int t = t0 + tt;
      const float4 kv = (t == p) ? kn4 : (first ? kp[j] : ld4_agent(&Kc[(size_t)t * kHd + 4 * lane]));
      score(tt, kv);
    }
    for (int tt = wid + kNW * kAttnPf; tt < len; tt += kNW) {
      const int t = t0 + tt;
      score(tt, (t == p) ? kn4 : ld4_agent(&Kc[(size_t)t * kHd + 4 * lane]));
    }
    __syncthreads();
    for (int h = wid; h < rep; h += kNW) {
      float mx = -INFINITY;
      for (int tt = lane; tt < len; tt += 64) mx = fmaxf(mx, sc[h * kMaxChunk + tt]);
      mx = wave_max(mx);
      float l = 0.f;
      for (int tt = lane; tt < len; tt += 64) {
        const float pe = expf(sc[h * kMaxChunk + tt] - mx);
        sc[h * kMaxChunk + tt] = pe;
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
      for (int e = 0; e < 4; ++e) acc[h][e] = 0.f;
    auto pv = [&](int tt, float4 vv) {
#pragma unroll
      for (int h = 0; h < kMaxRep; ++h) {
        if (h >= rep) break;
        const float pe = sc[h * kMaxChunk + tt];
        acc[h][0] += pe * vv.x; acc[h][1] += pe * vv.y; acc[h][2] += pe * vv.z; acc[h][3] += pe * vv.w;
      }
    };
    const float4 vn4 = *reinterpret_cast<const float4*>(&vn[4 * lane]);
#pragma unroll
    for (int j = 0; j < kAttnPf; ++j) {
      const int tt = wid + kNW * j;
      if (tt >= len) break;  // uniform
      const int t = t0 + tt;
      pv(tt, (t == p) ? vn4 : (first ? vp[j] : ld4_agent(&Vc[(size_t)t * kHd + 4 * lane])));
    }
    for (int tt = wid + kNW * kAttnPf; tt < len; tt += kNW) {
      const int t = t0 + tt;
      pv(tt, (t == p) ? vn4 : ld4_agent(&Vc[(size_t)t * kHd + 4 * lane]));
    }
#pragma unroll
    for (int h = 0; h < kMaxRep; ++h)
      *reinterpret_cast<float4*>(&ored[(wid * kMaxRep + h) * kHd + 4 * lane]) = make_float4(acc[h][0], acc[h][1], acc[h][2], acc[h][3]);
    __syncthreads();
    const size_t pc = (size_t)g * a.att_nmax + c;
    for (int e = tid; e < rep * kHd; e += kT) {
      const int h = e / kHd, d = e % kHd;
      float o = 0.f;
#pragma unroll
      for (int w = 0; w < kNW; ++w) o += ored[(w * kMaxRep + h) * kHd + d];
      st_agent(&a.att_o[(pc * kMaxRep + h) * kHd + d], o);
    }
    if (tid < rep) {
      st_agent(&a.att_ml[pc * 2 * kMaxRep + tid], hm[tid]);
      st_agent(&a.att_ml[pc * 2 * kMaxRep + kMaxRep + tid], hl[tid]);
    }
    __syncthreads();
  }
  bar_arrive(bar);
  return true;
}

// ------------------------------------------------------------------ lm_head + argmax
// Tied embedding [V][H] as lm_head (kernels.rs:251-291): wave w owns R rows per block step,
// lane l reads the 16-byte chunks 16*(l + 64c), c < CPW, of each row; two steps of loads
// (2 x 8 per lane, 128 KB per block) are kept in flight.  Block argmax (reference order,
// ArgOrder) -> arg_v / arg_i.
template <int CPW>
Q35_DEV bool lm_stage(const StepArgs& a, Bar& bar, const Shared& sh) {
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
        const float4 t = xp[q];
        xv[4 * q] = t.x; xv[4 * q + 1] = t.y; xv[4 * q + 2] = t.z; xv[4 * q + 3] = t.w;
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
  if (!bar_wait(bar, sh.ok)) return false;
  // the second row block is issued behind the norm's inputs (rows clamped: always in the table)
  pro_rms<2 * CPW, fx_t>(HLoad{a.h}, HConv{}, K, a.final_norm, a.eps, 0, K, xs, sh.shs,
                         [&]() { load(rb0 + gs, wb, sb); });
  __syncthreads();
  for (int rb = rb0; rb < nrb; rb += 2 * gs) {
    if (rb != rb0 && rb + gs < nrb) load(rb + gs, wb, sb);
    compute(rb, wa, sa);
    if (rb + gs >= nrb) break;
    if (rb + 2 * gs < nrb) load(rb + 2 * gs, wa, sa);
    compute(rb + gs, wb, sb);
  }
  block_argmax(best_v, best_i, sh.shv, sh.shi, a.ord);
  if (tid == 0) { st_agent(&a.arg_v[bix()], best_v); st_agent(&a.arg_i[bix()], best_i); }
  bar_arrive(bar);
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
          v[u] = ld4_agent(src);
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
template <int CPW>
__global__ __launch_bounds__(kT) void step_kernel(const StepArgs a) {
  constexpr int KR = 2 * CPW;  // hidden <= 256 CPW = 512 KR
  __shared__ __align__(16) float smem[kSmem];
  __shared__ __align__(16) float shs[kNW];
  __shared__ float shv[kNW];
  __shared__ int shi[kNW];
  __shared__ int ok;
  const Shared sh{smem, shs, shv, shi, &ok};
  Bar bar{a.bar, a.err, a.bar_base};
  // a failed earlier launch left the model state invalid: do nothing until a reset
  if (ld_agent(a.err) != 0u) return;
  const int p0 = ldg(a.pos);
  int executed = a.ntok, stop_tok = 0;
  for (int i = 0; i < a.ntok && executed == a.ntok; ++i) {
    const int p = p0 + i;
    for (int l = 0; l < a.n_layers; ++l) {
      CLayer& L = layer_at(a, l);
      const int pro0 = (l == 0) ? PRO_EMBED_RMS : PRO_RMS;
      int r;
      if (!L.full) {
        r = mv_stage<kU, KR>(a, L, SMV_QKVZ, pro0, i, p, bar, sh, &stop_tok);
        if (r == kStageStop) { executed = i; break; }
        if (r == kStageFail) return;
        if (!mv_stage<kUOut, KR>(a, L, SMV_OUT, PRO_GDN, i, p, bar, sh)) return;
      } else {
        r = mv_stage<kU, KR>(a, L, SMV_QKV, pro0, i, p, bar, sh, &stop_tok);
        if (r == kStageStop) { executed = i; break; }
        if (r == kStageFail) return;
        if (!attn_stage(a, L, p, bar, sh)) return;
        if (!mv_stage<kU, KR>(a, L, SMV_O, PRO_ATTN, i, p, bar, sh)) return;
      }
      if (!mv_stage<kU, KR>(a, L, SMV_GU, PRO_RMS, i, p, bar, sh)) return;
      if (!mv_stage<kU, KR>(a, L, SMV_DOWN, PRO_SWIGLU, i, p, bar, sh)) return;
    }
    if (executed != a.ntok) break;
    if (!lm_stage<CPW>(a, bar, sh)) return;
  }
  if (executed != a.ntok) {
    // Stopped before step `executed` ran (every block decided alike): arrive once for all the
    // barriers the remaining steps would have passed, so the counters end where a full launch
    // leaves them (the host counts barriers per launch).
    const uint32_t final_epoch = a.bar_base + (uint32_t)a.ntok * (uint32_t)a.bar_per_token;
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tix() == 0)
      __hip_atomic_fetch_add((Q35_GLOBAL uint32_t*)&bar.ctr[(bix() % kGroups) * kCtrStride], final_epoch - bar.epoch,
                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    bar.epoch = final_epoch;
  }
  // Every block has passed the last executed step's lm-stage barrier (a stop is decided after
  // it), so all state writes are complete.
  if (executed & 1) state_copy_back(a);
  // tail: block 0 turns the last step's block argmaxes into the token
  if (bix() != 0) return;
  if (!bar_wait(bar, sh.ok)) return;
  if (executed != a.ntok) {  // the stop id stays the next token; hist already holds it
    if (tix() == 0) {
      stg(a.token, (int32_t)stop_tok);
      stg(a.pos, (int32_t)(p0 + executed));
    }
    return;
  }
  float v = -INFINITY;
  int ix = INT_MAX;
  if (tix() < (int)gridDim.x) { v = ld_agent(&a.arg_v[tix()]); ix = ld_agent(&a.arg_i[tix()]); }
  block_argmax(v, ix, sh.shv, sh.shi, a.ord);
  if (tix() == 0) {
    const int tok = (ix == INT_MAX) ? 0 : ix;
    const int pl = p0 + a.ntok - 1;
    stg(a.hist + pl, (int32_t)tok);
    stg(a.token, (int32_t)tok);
    stg(a.pos, (int32_t)(pl + 1));
  }
}

const void* kernel_for(int hidden) {
  if (hidden <= 1024) return reinterpret_cast<const void*>(step_kernel<1>);
  if (hidden <= 2048) return reinterpret_cast<const void*>(step_kernel<2>);
  return reinterpret_cast<const void*>(step_kernel<4>);
}

}  // namespace

int step_grid(int hidden) {
  if (hidden < 64 || hidden > 4096) return 0;
  int dev = 0, ncu = 0, coop = 0, nb = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  if (hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  if (hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, dev) != hipSuccess || !coop) return 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, kernel_for(hidden), kT, 0) != hipSuccess || nb < 1) return 0;
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
  if ((long long)tmax > (long long)kMaxChunk * step_att_nmax(grid, d.kv_heads))
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
    int nchunk = std::max(1, grid / s.tiles);
    int kch = (s.K + nchunk - 1) / nchunk;
    kch = (kch + 15) & ~15;
    if (kch > kKch) kch = kKch;
    if (s.kind == SMV_OUT) {
      int kc = d.lin_dv;
      while (kc > kch && kc % 32 == 0) kc /= 2;
      kch = kc;
    }
    nchunk = (s.K + kch - 1) / kch;
    mv[s.kind] = StepMv{kch, nchunk};
  }
}

int step_barriers_per_token(const q35_dims& d) {
  int n = 1;  // lm_head
  for (int l = 0; l < d.n_layers; ++l) n += ((l + 1) % d.full_interval == 0) ? 5 : 4;
  return n;
}

int step_launch(const StepArgs& a, int grid, hipStream_t st) {
  if (a.ntok < 1) return Q35_OK;
  if (!a.bar || !a.err) return fail(Q35_E_ARG, "persistent step: null barrier or error word");
  StepArgs args = a;
  void* params[] = {&args};
  Q35_HIP_TRY(hipLaunchCooperativeKernel(kernel_for(a.H), dim3(grid), dim3(kT), params, 0, st));
  return Q35_OK;
}

}  // namespace q35
