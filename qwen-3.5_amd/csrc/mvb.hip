// Batched decode projections on the matrix cores: Y[m][n] = sum_k X~[m][k] * dequant(W)[k][n] for
// up to 32 decode rows m at once (the B sequences of a batched step), so that every weight matrix
// is streamed once per step for all rows.  This is the reference's Linear on a QFloat weight
// (text_modules.rs:500-508, :578-595, :638-647, :880-890, :1003-1005; kernels.rs:53-92 for the
// Q8F block scales) with f32-equivalent arithmetic on the f16 matrix cores
// (v_mfma_f32_16x16x32_f16, f32 accumulation):
//   * the int8 weights are exact in f16;
//   * the scale of a weight's 64-column block multiplies the input instead, y = x~ * s (f32, the
//     scale varies along k only), and y is carried as two f16 values hi + lo (hi = f16(y * 2^e),
//     lo = f16(y * 2^e - hi)), about 22 significant bits, with 2^e a power of two per row chosen
//     so that the row's largest |y| lands in [2^13, 2^14);
//   * q * hi and q * lo are exact in the f32 accumulator; the result is scaled back by 2^-e.
//
// Weight layout (MB, built once from the tile-major projection layout): per 64-column block cb and
// 32-row step ks, 2 KB in which lane l = 16 g + c of a wave finds, as two 16-byte loads, the bytes
// u = q + 128 of q[32 ks + 8 g + j][64 cb + 16 nt + c] (j = 0..7) for each of the 4 column tiles
// nt: exactly its A operands (row c of tile nt, k slot g) of one MFMA, with the k order permuted
// inside the step (the sum is unchanged).  The batched decode reads a copy in stream order
// (mb_stream_launch): lane l's two 16-byte loads at 16 l and 1024 + 16 l instead of 32 l and
// 32 l + 16, so each load instruction reads 1 KB contiguous rather than half of each of 16 lines
// (the prompt GEMMs, which re-read every weight from L2, run faster on the MB order).  u converts to f16 as the bit pattern 0x6400 | u
// (= 1024 + u) minus 1152.  Scales are stored per column block, scale[cb][K].
//
// Block = 4 waves = one column block (64 outputs) x the block's K range (at most 1024 / MT rows).
// The block first stages its Mp x K-range input rows: transformed by the prologue (RMSNorm, gated
// RMSNorm or SwiGLU of the producer's output), multiplied by the column block's scales and split
// into the hi / lo planes in LDS, with one global round trip.  Then the waves stream their
// weights with no further synchronisation: wave p takes the 32-row step p of every 128-row round,
// its weights loaded 4 rounds ahead.  The 4 waves' accumulators are summed through LDS in a fixed
// order.  A block with the whole K writes its outputs directly; with split-K the blocks of a
// column block add their partials to counted fixed-point words with returning atomics, and the
// split that completes a word writes that output (exact sums, so deterministic).  Residual
// projections add into the f32 residual rows and accumulate each row's sum of squares for the
// next RMSNorm (fixed point, so the sum is order-independent).
//
// The lm_head (mbn_kernel) reads a copy of the tied [V][D] table in its load order (built once,
// mb_lm_table_launch): lane l = 16 g + c takes 16 consecutive bytes of vocab row c of a tile
// (k = 16 g .. 16 g + 15 of a 64-wide scale block), its A operands for two MFMAs, and the copy
// puts the 64 lanes' bytes of one load instruction side by side, so each instruction reads 1 KB
// contiguous (from the table itself it would touch 16 rows, 64 bytes each).  The block scale
// depends on the output row there, so each 64-k block is accumulated separately and added with
// the rows' scales (read from a transposed copy of the scale table).  Its input rows arrive
// already normalised and split (rms_rows_split_kernel).
#include "q35_internal.h"

#include <algorithm>
#include <climits>

namespace q35 {
namespace {

constexpr int kT = 256;            // threads per block (4 waves)
constexpr int kRound = 128;        // K rows per round (4 waves x one 32-row step)
constexpr int kDepth = 4;          // rounds of weights in flight per wave (mbk)
constexpr int kNDepth = 2;         // rounds in flight per wave (mbn)
constexpr int kNKmax = 2048;       // lm_head: largest hidden size (the whole x rows sit in LDS)
constexpr int kNLd = kNKmax + 8;   // lm_head: padded LDS row of one plane (halves)
constexpr int kAuxLd = kRound + 4; // f32 staging row of the gate side blocks (one 128-row chunk)
constexpr int kDirectKR = 1024;    // rows of K per block on the RMS direct path
// a counted split-K hand-off (mb_launch) costs one atomic per output and split: it is taken up
// to kCountedMax of them, or up to kCountedMaxSplit with 5 or more splits (whose partials would
// take longer to read back), measured on the decode projection shapes at 1-32 rows
constexpr size_t kCountedMax = 150000, kCountedMaxSplit = 300000;

typedef float f4 __attribute__((ext_vector_type(4)));
typedef q35_h2 h2;
typedef q35_h8 h8;

struct MbkSeg {
  const int8_t* q;  // MB layout
  const float* s;   // [N/64][K]
  float* y;
  const float* f;   // [N/64] split factors of the RMS direct path
  int32_t N, ldy, cb0;  // cb0: first column block of the segment in the launch
};
struct MbkArgs {
  MbkSeg seg[kMbMaxSeg];
  int32_t nseg, K, M, ncb, nsplit, kr;
  const float* x; int32_t ldx;
  int32_t pro; const float* pw; float eps; const fx_t* ss;
  const float* z; int32_t ldz, group, swiglu_off;
  int32_t add; fx_t* ss_out;
  int64_t dstride;   // > 0 with nsplit == 2: split s writes its partial to y + s * dstride (no hand-off)
  int64_t xsstride;  // consumer of such partials (XS = 2): the second copy's offset
  const float* aux_wb; const float* aux_wa; int32_t aux_nh; fx_t* aux_acc; int32_t aux_ldo, naux;
  float* part; uint32_t* ctr;  // split-K partials [ncb][nsplit][Mp][64] and arrival counters
  uint64_t* words;             // or counted fixed-point words [ncb][M][64], zero between launches
  int32_t counted;
  uint32_t* err;
};

Q35_DEV f4 ld4(const float* p) { return *(const Q35_GLOBAL f4*)p; }
Q35_DEV f4 lds4(const float* p) { return *(const f4*)p; }

// A block's input rows live in LDS for its whole K range: at most 1024 / MT rows of SR staged
// rows (SR = Mp = 16 MT, or 8 when a launch has at most 8: the matrix cores still take 16 rows, the
// reads of rows past SR repeat row SR - 1, whose outputs are never stored), as an f32 staging area
// (aux blocks) or as the hi / lo f16 planes, each row padded so that the 16 rows a B-operand read
// touches start in different banks.  Staging 8 rows puts 32 threads on each (half the loads and
// arithmetic per thread) and halves the planes.
template <int MT, int SR = 16 * MT>
struct XBuf {
  static constexpr int Mp = 16 * MT;
  static_assert(SR == Mp || (MT == 1 && SR == 8), "staged rows");
  static constexpr int KR = 1024 / MT;         // rows of K per block
  static constexpr int LDH = KR + 8;           // halves per row of one f16 plane
  static constexpr int NCH = KR / kRound;      // 128-row chunks
  static constexpr int TPR = kT / SR;          // staging threads per x row: 32, 16 or 8
  static constexpr int VPT = kRound / TPR;     // values per thread per chunk: 4, 8 or 16
  static constexpr int AUX = SR * kAuxLd * 4;  // f32 staging of one chunk (gate side blocks)
  static constexpr int RED = 4 * 16 * MT * 64 * 4;  // the 4 waves' accumulators
  static constexpr int PLANES = 2 * SR * LDH * 2;
  static constexpr int BYTES = PLANES > AUX ? (PLANES > RED ? PLANES : RED) : (AUX > RED ? AUX : RED);
  static constexpr int DBYTES = AUX > RED ? AUX : RED;  // direct path: no planes
};

// Stage x~ for rows [k0, k0 + klen) (klen a multiple of 128, <= KR): every load the range needs
// (x, the second operand, the norm weights, the row statistic) is issued first, so staging costs
// one round trip.  Thread t covers row t / TPR of every chunk, columns (t % TPR) * VPT .. + VPT;
// the rows of the chunk past M repeat row M - 1 (their outputs are never stored).
//   SPLIT = false (klen = 128): x~ is written as f32 rows (xs, [SR][kAuxLd]).
//   SPLIT = true: y = x~ * scale of the column block, split into hi / lo planes (xs: hi
//   [SR][LDH] then lo), with the row's inverse power of two in invf[row].
// `issue` runs right after the staging loads are issued: the caller's weight prefetch goes
// behind them, so the staging arithmetic waits only for its own loads (loads return in order).
// XS = 2: the input rows are two split-K partials of the producer, xsstride floats apart (summed
// here in split order, as the producer's own hand-off would have).
template <int MT, bool SPLIT, int XS = 1, int SR = 16 * MT, typename Issue>
Q35_DEV void stage_x(const MbkArgs& a, int k0, int klen, char* xbuf, float* scs, const float* scl, float* pws,
                     float* invf, Issue&& issue) {
  using X = XBuf<MT, SR>;
  const int t = threadIdx.x, mr = t / X::TPR, m = min(mr, a.M - 1), c0 = (t % X::TPR) * X::VPT;
  const int nch = klen / kRound;
  const bool rms = a.pro == MB_PRO_RMS, gated = a.pro == MB_PRO_GATED, two = gated || a.pro == MB_PRO_SWIGLU;
  const float* xr = a.x + (size_t)m * a.ldx + k0 + c0;
  const float* ur = gated ? a.z + (size_t)m * a.ldz + k0 + c0 : xr + a.swiglu_off;
  float v[X::NCH][X::VPT], u[X::NCH][X::VPT];
  float wg[X::VPT];  // gated norm weights (the same VPT for every chunk)
  // the block's scales and (RMS) norm weights go to LDS once (SPLIT), one 16-byte piece a thread
  f4 sc = f4{0.f, 0.f, 0.f, 0.f}, pw4 = f4{0.f, 0.f, 0.f, 0.f};
  if (SPLIT && 4 * t < klen) {
    sc = ld4(scl + k0 + 4 * t);
    if (rms) pw4 = ld4(a.pw + k0 + 4 * t);
  }
  const fx_t ssv = ldg(a.ss + m);  // (a valid dummy address without RMS: no branch, so the wait
                                   // for it lands after the x loads below are issued)
  if (gated) {
#pragma unroll
    for (int i = 0; i < X::VPT; i += 4) {
      const f4 q = ld4(a.pw + ((c0 + i) & (a.group - 1)));
      wg[i] = q[0]; wg[i + 1] = q[1]; wg[i + 2] = q[2]; wg[i + 3] = q[3];
    }
  }
#pragma unroll
  for (int ci = 0; ci < X::NCH; ++ci) {
    const int cc = min(ci, nch - 1) * kRound;  // (chunks past the range reload the last one)
#pragma unroll
    for (int i = 0; i < X::VPT; i += 4) {
      f4 q = ld4(xr + cc + i);
      if constexpr (XS == 2) q = q + ld4(xr + a.xsstride + cc + i);
      v[ci][i] = q[0]; v[ci][i + 1] = q[1]; v[ci][i + 2] = q[2]; v[ci][i + 3] = q[3];
      if (two || (rms && !SPLIT)) {
        f4 w = ld4(rms ? a.pw + k0 + cc + c0 + i : ur + cc + i);
        if constexpr (XS == 2) w = w + ld4(ur + a.xsstride + cc + i);  // (SwiGLU only)
        u[ci][i] = w[0]; u[ci][i + 1] = w[1]; u[ci][i + 2] = w[2]; u[ci][i + 3] = w[3];
      }
    }
  }
  issue();
  asm volatile("" ::: "memory");
  if (SPLIT && 4 * t < klen) {
    *(f4*)(scs + 4 * t) = sc;
    if (rms) *(f4*)(pws + 4 * t) = pw4;
  }
  // y = x * rsqrt(mean(x^2) + eps) * (1 + w)  (text_modules.rs:800-808); the row's sum of
  // squares comes from the projection that produced x; with SPLIT, (1 + w) is applied below
  const float r = rsqrt_f(from_fx(ssv) * rcp_f((float)a.K) + a.eps);
  const int tpg = gated ? a.group / X::VPT : 1;  // gated: threads per group (power of two <= TPR)
#pragma unroll
  for (int ci = 0; ci < X::NCH; ++ci) {
    if (rms) {
#pragma unroll
      for (int i = 0; i < X::VPT; ++i) v[ci][i] = SPLIT ? v[ci][i] * r : (v[ci][i] * r) * (1.0f + u[ci][i]);
    } else if (gated) {
      // RMSNormGated (text_modules.rs:91-100): per group of `group` values of the row,
      // w * (x * rsqrt(mean(x^2) + eps)) * silu(z); the group's threads are consecutive lanes
      float ss = 0.f;
#pragma unroll
      for (int i = 0; i < X::VPT; ++i) ss += v[ci][i] * v[ci][i];
      for (int o = 1; o < tpg; o <<= 1) ss += __shfl_xor(ss, o);
      const float rg = rsqrt_f(ss * rcp_f((float)a.group) + a.eps);
#pragma unroll
      for (int i = 0; i < X::VPT; ++i) v[ci][i] = (wg[i] * (v[ci][i] * rg)) * silu_f(u[ci][i]);
    } else if (two) {
      // MLP (text_modules.rs:1000-1011): up * silu(gate)
#pragma unroll
      for (int i = 0; i < X::VPT; ++i) v[ci][i] = u[ci][i] * silu_f(v[ci][i]);
    }
  }
  if (!SPLIT) {
    float* xs = reinterpret_cast<float*>(xbuf);
#pragma unroll
    for (int ci = 0; ci < X::NCH; ++ci)
      if (ci < nch) {
        float* dst = xs + mr * kAuxLd + ci * kRound + c0;
#pragma unroll
        for (int i = 0; i < X::VPT; i += 4) *(f4*)(dst + i) = f4{v[ci][i], v[ci][i + 1], v[ci][i + 2], v[ci][i + 3]};
      }
    return;
  }
  __syncthreads();  // scales in LDS
  float amax = 0.f;
#pragma unroll
  for (int ci = 0; ci < X::NCH; ++ci) {
#pragma unroll
    for (int i = 0; i < X::VPT; i += 4) {
      const int kk = min(ci, nch - 1) * kRound + c0 + i;
      const f4 s4 = lds4(scs + kk);
      const f4 w4 = rms ? lds4(pws + kk) : f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (rms) v[ci][i + j] = v[ci][i + j] * (1.0f + w4[j]);
        v[ci][i + j] *= s4[j];
        amax = fmaxf(amax, fabsf(v[ci][i + j]));
      }
    }
  }
  for (int o = 1; o < X::TPR; o <<= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
  float f, inv;
  split_scale(amax, f, inv);
  if ((t % X::TPR) == 0) invf[mr] = inv;
  _Float16* hp = reinterpret_cast<_Float16*>(xbuf) + mr * X::LDH + c0;
  _Float16* lp = hp + SR * X::LDH;
#pragma unroll
  for (int ci = 0; ci < X::NCH; ++ci)
    if (ci < nch) {
      if constexpr (X::VPT % 8 == 0) {
#pragma unroll
        for (int i = 0; i < X::VPT; i += 8) {
          uint32_t hi[4], lo[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) split2(v[ci][i + 2 * j] * f, v[ci][i + 2 * j + 1] * f, hi[j], lo[j]);
          *(q35_u32x4*)(hp + ci * kRound + i) = q35_u32x4{hi[0], hi[1], hi[2], hi[3]};
          *(q35_u32x4*)(lp + ci * kRound + i) = q35_u32x4{lo[0], lo[1], lo[2], lo[3]};
        }
      } else {  // 4 values per thread: one 8-byte store per plane
        uint32_t hi[2], lo[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) split2(v[ci][2 * j] * f, v[ci][2 * j + 1] * f, hi[j], lo[j]);
        typedef uint32_t u2 __attribute__((ext_vector_type(2)));
        *(u2*)(hp + ci * kRound) = u2{hi[0], hi[1]};
        *(u2*)(lp + ci * kRound) = u2{lo[0], lo[1]};
      }
    }
}

// Segment of column block cb (constant-index field selection).
Q35_DEV MbkSeg seg_of(const MbkArgs& a, int cb) {
  MbkSeg sg = a.seg[0];
#pragma unroll
  for (int i = 1; i < kMbMaxSeg; ++i)
    if (i < a.nseg && cb >= a.seg[i].cb0) sg = a.seg[i];
  return sg;
}

// Gate projection side blocks (in_proj_b | in_proj_a, f32 [K][nh] each, kernels.rs:174-247):
// block ab sums rows [128 ab, 128 ab + 128) of x~ . W for every row m and adds the raw sums to
// aux_acc (fixed point); the DeltaNet step applies the gates' activations.
template <int MT, int SR>
Q35_DEV void mbk_aux(const MbkArgs& a, int ab, char* xbuf, float* red) {
  const int t = threadIdx.x, kc = ab * kRound;
  stage_x<MT, false, 1, SR>(a, kc, kRound, xbuf, nullptr, nullptr, nullptr, nullptr, [] {});
  __syncthreads();
  const float* xs = reinterpret_cast<const float*>(xbuf);
  const int nh = a.aux_nh, no = 2 * nh;  // no <= 32
  const int o = t & 31, rg = t >> 5;     // 8 row groups of 16
  float w[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int k = kc + rg * 16 + i;
    const int oc = min(o < nh ? o : o - nh, nh - 1);
    const float* W = o < nh ? a.aux_wb : a.aux_wa;
    w[i] = (o < no) ? ldg(W + (size_t)k * nh + oc) : 0.f;
  }
  for (int m = 0; m < a.M; ++m) {
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc += xs[m * kAuxLd + rg * 16 + i] * w[i];
    red[rg * 32 + o] = acc;
    __syncthreads();
    if (t < no) {
      float v = 0.f;
#pragma unroll
      for (int g = 0; g < 8; ++g) v += red[g * 32 + t];
      fx_add_chk(&a.aux_acc[(size_t)m * a.aux_ldo + t], v, a.err);
    }
    __syncthreads();
  }
}

// DIRECT (RMSNorm prologue only): no staging.  Each lane forms its own B operands round by round
// from x, the norm weights and the scales it loads with the round's weights, y = ((x * r) * (1 +
// w)) * s, split with the column block's factor f = 2^e (a power of two fixed per column block:
// |x * r| <= sqrt(K) for an RMS-normalised row, so sqrt(K) * max|1 + w| * max|s| bounds every |y|
// of the block and f puts that bound in [2^13, 2^14)).  The bound is loose for most rows, which
// costs nothing: hi / lo keep about 22 bits of each y down to 2^-17 of the bound.
// SO: the weights are in stream order (lane l's bytes at 16 l and 1024 + 16 l of each 2 KB record;
// else the MB order's 32 l and 32 l + 16).  A compile-time choice, so both loads keep immediate
// offsets from one address.
template <int MT, bool DIRECT, int XS = 1, int SR = 16 * MT, bool SO = false>
__global__ __launch_bounds__(kT, 2) void mbk_kernel(const MbkArgs a) {
  using X = XBuf<MT, SR>;
  constexpr int Mp = X::Mp;
  constexpr int NCH = DIRECT ? kDirectKR / kRound : X::NCH;  // rounds per block at most
  // staged x~ (f32 or hi / lo planes); then the reduction
  __shared__ __align__(16) char xbuf[DIRECT ? X::DBYTES : X::BYTES];
  __shared__ __align__(16) float scs[DIRECT ? 4 : X::KR];
  __shared__ __align__(16) float pws[DIRECT ? 4 : X::KR];
  __shared__ __align__(16) float aux_red[256];
  __shared__ float invf[Mp];
  __shared__ fx_t sq[4][Mp];
  __shared__ int last_flag;

  const int nmain = a.ncb * a.nsplit;
  if ((int)blockIdx.x >= nmain) {
    mbk_aux<MT, SR>(a, (int)blockIdx.x - nmain, xbuf, aux_red);
    return;
  }
  const int tid = threadIdx.x, lane = tid & 63, p = tid >> 6, g = lane >> 4, c = lane & 15;
  const int cb = (int)blockIdx.x / a.nsplit, split = (int)blockIdx.x - cb * a.nsplit;
  const MbkSeg sg = seg_of(a, cb);
  const int lcb = cb - sg.cb0;
  const int k0 = split * a.kr, klen = min(a.kr, a.K - k0);
  const int nround = klen / kRound;
  const int nks = a.K >> 5;
  // wave p's 32-row step in round r: 4 r + p, relative to k0
  const int8_t* wq = sg.q + ((size_t)lcb * nks + (k0 >> 5) + p) * 2048 + lane * (SO ? 16 : 32);

  // Rounds past the block's range load 32 bytes per lane of its (cached) scale row instead (inside
  // the row: K >= 128), so every round issues the same loads and the compiler's waits count them
  // exactly.
  const float* scl = sg.s + (size_t)lcb * a.K;
  const int8_t* dummy = reinterpret_cast<const int8_t*>(scl + min(lane * 8, a.K - 8));
  q35_u32x4 wr[kDepth][2];
  // direct path: the round's scales, norm weights and x rows (8 consecutive k of the lane's slot)
  f4 sr[DIRECT ? kDepth : 1][2], pr[DIRECT ? kDepth : 1][2], xr[DIRECT ? kDepth : 1][MT][2];
  const float* xrow[MT];
  float rrow[MT];
  const int kl0 = k0 + 32 * p + 8 * g;  // the lane's first k (round 0)
  auto load_round = [&](int r, int d) {
    const bool in = r < nround;
    const int8_t* src = in ? wq + (size_t)r * 4 * 2048 : dummy;
    wr[d][0] = ldg16v_nt(src);
    wr[d][1] = ldg16v_nt(src + (in ? (SO ? 1024 : 16) : 16));
    if constexpr (DIRECT) {  // rounds past the range reload the last one (cached)
      const int kk = kl0 + min(r, nround - 1) * kRound;
      sr[d][0] = ld4(scl + kk);
      sr[d][1] = ld4(scl + kk + 4);
      pr[d][0] = ld4(a.pw + kk);
      pr[d][1] = ld4(a.pw + kk + 4);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        xr[d][mt][0] = ld4(xrow[mt] + kk);
        xr[d][mt][1] = ld4(xrow[mt] + kk + 4);
      }
    }
  };
  float fcb = 1.f;
  if constexpr (DIRECT) {
    fx_t ssv[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int m = min(16 * mt + c, a.M - 1);  // rows past M repeat row M - 1 (never stored)
      xrow[mt] = a.x + (size_t)m * a.ldx;
      ssv[mt] = ldg(a.ss + m);
    }
    fcb = ldg(sg.f + lcb);
    static_for<kDepth>([&](auto d) { load_round(d, d); });
    // y = x * rsqrt(mean(x^2) + eps) * (1 + w)  (text_modules.rs:800-808); the row's sum of
    // squares comes from the projection that produced x
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) rrow[mt] = rsqrt_f(from_fx(ssv[mt]) * rcp_f((float)a.K) + a.eps);
  } else {
    stage_x<MT, true, XS, SR>(a, k0, klen, xbuf, scs, scl, pws, invf,
                          [&] { static_for<kDepth>([&](auto d) { load_round(d, d); }); });
    __syncthreads();
  }

  const _Float16* xh = reinterpret_cast<const _Float16*>(xbuf);
  const _Float16* xl = xh + SR * X::LDH;
  f4 acc[4][MT];
#pragma unroll
  for (int nt = 0; nt < 4; ++nt)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[nt][mt] = f4{0.f, 0.f, 0.f, 0.f};

  // every round unrolled (at most NCH of them), so the compiler's waits for the weight loads
  // count exactly the rounds still in flight
  static_for<NCH>([&](auto rc) {
    constexpr int r = rc, d = r % kDepth;
    if (r < nround) {
      const int kl = r * kRound + 32 * p + 8 * g;
      h8 bh[MT], bl[MT];
      if constexpr (DIRECT) {
        float sf[8], wp[8];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          sf[j] = sr[d][0][j] * fcb;  // exact: fcb is a power of two
          sf[4 + j] = sr[d][1][j] * fcb;
          wp[j] = 1.0f + pr[d][0][j];
          wp[4 + j] = 1.0f + pr[d][1][j];
        }
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          float y[8];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            y[j] = ((xr[d][mt][0][j] * rrow[mt]) * wp[j]) * sf[j];
            y[4 + j] = ((xr[d][mt][1][j] * rrow[mt]) * wp[4 + j]) * sf[4 + j];
          }
          uint32_t hi[4], lo[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) split2(y[2 * j], y[2 * j + 1], hi[j], lo[j]);
          bh[mt] = __builtin_bit_cast(h8, q35_u32x4{hi[0], hi[1], hi[2], hi[3]});
          bl[mt] = __builtin_bit_cast(h8, q35_u32x4{lo[0], lo[1], lo[2], lo[3]});
        }
      } else {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const int row = min(16 * mt + c, SR - 1);  // (rows past SR: outputs never stored)
          bh[mt] = *(const h8*)(xh + row * X::LDH + kl);
          bl[mt] = *(const h8*)(xl + row * X::LDH + kl);
        }
      }
      const q35_u32x4 w0 = wr[d][0], w1 = wr[d][1];
      const h8 aw[4] = {a8_from(w0[0], w0[1]), a8_from(w0[2], w0[3]), a8_from(w1[0], w1[1]), a8_from(w1[2], w1[3])};
#pragma unroll
      for (int nt = 0; nt < 4; ++nt)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          acc[nt][mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(aw[nt], bh[mt], acc[nt][mt], 0, 0, 0);
#pragma unroll
      for (int nt = 0; nt < 4; ++nt)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          acc[nt][mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(aw[nt], bl[mt], acc[nt][mt], 0, 0, 0);
      if (r + kDepth < NCH) {
        load_round(r + kDepth, d);
        asm volatile("" ::: "memory");  // keep the prefetch here (not sunk to its use)
      }
    }
  });

  // lane holds columns n = 16 p + 4 g + i (i = 0..3) of row m = 16 mt + c after the reduction;
  // residual projections read those outputs' old values now (rows clamped), so the round trip
  // overlaps the reduction and the split-K hand-off
  const int ncol0 = 64 * lcb + 16 * p + 4 * g;
  f4 yold[MT];
  if (a.add) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) yold[mt] = ld4(sg.y + (size_t)min(16 * mt + c, a.M - 1) * sg.ldy + ncol0);
  }

  // Sum the 4 waves' partial sums: wave p writes its accumulators, then finalises column tile
  // nt = p (16 columns x Mp rows) from all four in wave order; the row's 2^-e undoes the split's
  // scaling.
  float* red = reinterpret_cast<float*>(xbuf);
  __syncthreads();
#pragma unroll
  for (int nt = 0; nt < 4; ++nt)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
      *(f4*)&red[((p * 4 + nt) * MT + mt) * 256 + lane * 4] = acc[nt][mt];
  __syncthreads();
  f4 out[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    f4 v = *(const f4*)&red[((0 * 4 + p) * MT + mt) * 256 + lane * 4];
#pragma unroll
    for (int q = 1; q < 4; ++q) v += *(const f4*)&red[((q * 4 + p) * MT + mt) * 256 + lane * 4];
    // the split's 2^e undone: per row (staged) or per column block (direct; 2^-e exactly)
    out[mt] = v * (DIRECT ? __int_as_float((254 << 23) - __float_as_int(fcb)) : invf[16 * mt + c]);
  }
  if (a.dstride > 0) {  // two splits, each writes its partial (scaled) for the consumer to sum
    float* yb = sg.y + (size_t)split * a.dstride;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int m = 16 * mt + c;
      if (m < a.M) *(f4*)(yb + (size_t)m * sg.ldy + ncol0) = out[mt];
    }
    return;
  }
  // fin: this lane writes element (mt, i) (row < M; with split-K, only the split that completes
  // the element's sum)
  bool fin[MT][4];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int i = 0; i < 4; ++i) fin[mt][i] = 16 * mt + c < a.M;
  if (a.nsplit > 1 && !a.counted) {
    float* pp = a.part + ((size_t)cb * a.nsplit + split) * Mp * 64;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i) st_agent(pp + (16 * mt + c) * 64 + 16 * p + 4 * g + i, out[mt][i]);
    if (!arrive_last(a.ctr + cb, (uint32_t)a.nsplit, &last_flag)) return;
    // the last block of the column block sums the partials in split order, up to kSumU splits
    // per round trip (all their loads issued before the first add; the partials bypass the
    // caches, so no load is issued for splits that do not exist)
    constexpr int kSumU = MT == 1 ? 16 : 8;
    const float* pb = a.part + (size_t)cb * a.nsplit * Mp * 64 + 16 * p + 4 * g;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) out[mt] = f4{0.f, 0.f, 0.f, 0.f};
    for (int s0 = 0; s0 < a.nsplit; s0 += kSumU) {
      f4 pv[kSumU][MT];
#pragma unroll
      for (int u = 0; u < kSumU; ++u)
        if (s0 + u < a.nsplit)
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            const float* q = pb + (size_t)(s0 + u) * Mp * 64 + (16 * mt + c) * 64;
            pv[u][mt] = f4{ld_agent(q), ld_agent(q + 1), ld_agent(q + 2), ld_agent(q + 3)};
          }
#pragma unroll
      for (int u = 0; u < kSumU; ++u)
        if (s0 + u < a.nsplit)
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) out[mt] += pv[u][mt];
    }
  } else if (a.nsplit > 1) {
    // Split-K hand-off through counted fixed-point words, one per output [cb][m][64]: every
    // split adds its partial (value * 2^32 plus 2^56, one count) with a returning atomic, and the
    // split whose add brings the count to nsplit holds the exact total (order-independent, so
    // deterministic), writes the output and clears the word for the next launch.  One round trip
    // per block instead of three (partials stored, arrivals counted, partials read back), at
    // the price of one atomic per output and split: the launcher picks it when those are few.
    uint64_t* wb = a.words + (size_t)cb * a.M * 64 + 16 * p + 4 * g;
    uint64_t add[MT][4], old[MT][4];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float v = out[mt][i];
        if (!fxc_addable(v)) {  // (counted anyway, as zero, so the word still completes)
          if (fin[mt][i]) __hip_atomic_fetch_or((Q35_GLOBAL uint32_t*)a.err, kWsErrRange, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          v = 0.f;
        }
        add[mt][i] = (uint64_t)to_fx(v) + (1ull << 56);
        old[mt][i] = fin[mt][i] ? __hip_atomic_fetch_add((Q35_GLOBAL uint64_t*)(wb + (size_t)(16 * mt + c) * 64 + i),
                                                         add[mt][i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                : 0;
      }
    const uint64_t before = (uint64_t)(a.nsplit - 1) << 56;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        // the word held nsplit - 1 contributions (|value| < 2^55 around its count)
        fin[mt][i] = fin[mt][i] && (old[mt][i] - before + (1ull << 55)) < (1ull << 56);
        if (fin[mt][i]) {
          const uint64_t tot = old[mt][i] + add[mt][i] - ((uint64_t)a.nsplit << 56);
          out[mt][i] = from_fx((fx_t)tot);
          __hip_atomic_store((Q35_GLOBAL uint64_t*)(wb + (size_t)(16 * mt + c) * 64 + i), 0ull, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
        }
      }
  }
  // write (or add) the outputs of rows m < M; residual adds also sum the new rows' squares
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = 16 * mt + c;
    // the squares go to fixed point one by one, so the row's sum is exact whichever block
    // completes which outputs
    fx_t sqs = 0;
    bool bad = false;
    float* yr = sg.y + (size_t)min(m, a.M - 1) * sg.ldy + ncol0;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (fin[mt][i]) {
        float v = out[mt][i];
        if (a.add) v += yold[mt][i];
        yr[i] = v;
        const float q = v * v;
        if (fx_addable(q)) sqs += to_fx(q);
        else bad = true;
      }
    if (a.ss_out) {
      if (bad) __hip_atomic_fetch_or((Q35_GLOBAL uint32_t*)a.err, kWsErrRange, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      sqs += __shfl_xor(sqs, 16);
      sqs += __shfl_xor(sqs, 32);
      if (g == 0) sq[p][m] = sqs;
    }
  }
  if (a.ss_out) {
    __syncthreads();
    // (with split-K, each block that completed some of the row's outputs adds their share)
    if (tid < a.M) {
      const fx_t v = ((sq[0][tid] + sq[1][tid]) + sq[2][tid]) + sq[3][tid];
      if (!a.counted || v != 0)
        __hip_atomic_fetch_add((Q35_GLOBAL unsigned long long*)(a.ss_out + tid), (unsigned long long)v, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// ------------------------------------------------------------------ lm_head over the NK table
struct MbnArgs {
  const int8_t* q;   // the table in load order (mb_lm_table_launch)
  const float* sT;   // scales transposed, [K/64][V]
  int32_t V, K, M;
  const _Float16* xh; const _Float16* xl; int32_t ld16;  // split rows [M][ld16] (hi, lo)
  const float* invf;                                      // [M]
  float* y; int32_t ldy;                                  // logits [M][ldy]
};

// One 16-byte copy per lane from global memory into LDS: lane l writes dst + 16 l (dst is
// wave-uniform).  Counted by vmcnt like any vector load.
Q35_DEV void dma16(const void* src, void* dst) {
  __builtin_amdgcn_global_load_lds((const Q35_GLOBAL void*)src, (__attribute__((address_space(3))) void*)dst, 16, 0, 0);
}

// R rows (M <= R: 16, or 8 so that two blocks fit a CU's LDS) per launch; the split x rows are
// copied into LDS whole, once (lanes of rows past R read row R - 1; their outputs are dropped).
template <int R>
__global__ __launch_bounds__(kT, 1) void mbn_kernel(const MbnArgs a) {
  __shared__ __align__(16) _Float16 xs[2][R * kNLd];  // hi, lo planes
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 4, c = lane & 15;
  const int nbase = (int)blockIdx.x * 256 + 64 * w;  // this wave's 64 vocab rows
  const int nround = a.K / kRound;

  // x rows into LDS: segments of 512 halves (one wave instruction each); rows past M repeat M - 1
  const int spr = a.K / 512, nseg = 2 * R * spr;
  for (int sgi = w; sgi < nseg; sgi += 4) {
    const int pl = sgi / (R * spr), rem = sgi % (R * spr), m = rem / spr, k = (rem % spr) * 512;
    const _Float16* src = (pl ? a.xl : a.xh) + (size_t)min(m, a.M - 1) * a.ld16 + k + 8 * lane;
    dma16(src, &xs[pl][m * kNLd + k]);
  }
  // lane's rows n = nbase + 16 nt + c (not stored past V); the wave's 64-row tile in the copy
  // (clamped: a block's waves past the table read its last tile)
  const int8_t* tile = a.q + (size_t)min(nbase / 64, (a.V + 63) / 64 - 1) * 64 * a.K;
  // the output rows' scales: rows nbase + 16 nt + 4 g .. + 3 of block kb (clamped)
  const int srow = nbase + 4 * g;
  // (rounds past K load the first round again: every round issues the same loads, so the
  // compiler's waits count them exactly)
  q35_u32x4 wr[kNDepth][2][4];
  f4 sr[kNDepth][2][4];
  auto load_round = [&](int r, q35_u32x4 (&wv)[2][4], f4 (&sv)[2][4]) {
    const int rr = r < nround ? r : 0;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) {
        wv[kb][nt] = ldg16v_nt(tile + (size_t)rr * (64 * kRound) + (kb * 4 + nt) * 1024 + 16 * lane);
        sv[kb][nt] = ld4(a.sT + (size_t)(2 * rr + kb) * a.V + min(srow + 16 * nt, a.V - 4));
      }
  };
  static_for<kNDepth>([&](auto d) { load_round(d, wr[d], sr[d]); });
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  f4 acc[4];
#pragma unroll
  for (int nt = 0; nt < 4; ++nt) acc[nt] = f4{0.f, 0.f, 0.f, 0.f};

  static_for<kNKmax / kRound>([&](auto rc) {
    constexpr int r = rc, d = r % kNDepth;
    if (r < nround) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        // k = 128 r + 64 kb + 16 g + 8 s + j: sub-step s takes bytes 8 s .. 8 s + 7 of the lane's 16
        const int kl = r * kRound + 64 * kb + 16 * g;
        h8 bh[2], bl[2];
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          bh[s] = *(const h8*)&xs[0][min(c, R - 1) * kNLd + kl + 8 * s];
          bl[s] = *(const h8*)&xs[1][min(c, R - 1) * kNLd + kl + 8 * s];
        }
        f4 tb[4];
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) {
          const q35_u32x4 wv = wr[d][kb][nt] ^ 0x80808080u;  // int8 -> u = q + 128
          const h8 a0 = a8_from(wv[0], wv[1]), a1 = a8_from(wv[2], wv[3]);
          f4 t = f4{0.f, 0.f, 0.f, 0.f};
          t = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, bh[0], t, 0, 0, 0);
          t = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, bh[1], t, 0, 0, 0);
          t = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, bl[0], t, 0, 0, 0);
          t = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, bl[1], t, 0, 0, 0);
          tb[nt] = t;
        }
        // rows n = nbase + 16 nt + 4 g + i of this 64-k block scale by s[n][kb]
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) acc[nt] += tb[nt] * sr[d][kb][nt];
      }
      if (r + kNDepth < kNKmax / kRound) {
        load_round(r + kNDepth, wr[d], sr[d]);
        asm volatile("" ::: "memory");  // keep the prefetch here (not sunk to its use)
      }
    }
  });
  // lane holds rows n = nbase + 16 nt + 4 g + i of column m = c
  if (c < a.M) {
    const float inv = a.invf[c];
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int n = nbase + 16 * nt + 4 * g + i;
        if (n < a.V) a.y[(size_t)c * a.ldy + n] = acc[nt][i] * inv;
      }
  }
}

// Final RMSNorm of the residual rows (text_modules.rs:800-808) with the lm_head input split:
// y = x * rsqrt(mean(x^2) + eps) * (1 + w), then hi / lo f16 planes of y * 2^e and 2^-e per row.
__global__ __launch_bounds__(kT) void rms_rows_split_kernel(const float* x, int ldx, int K, const float* w, float eps,
                                                            _Float16* yh, _Float16* yl, int ld16, float* invf) {
  __shared__ float sh[4];
  const int m = blockIdx.x;
  const float* xr = x + (size_t)m * ldx;
  float v[kNKmax / kT];
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < kNKmax / kT; ++j) {
    const int k = threadIdx.x + kT * j;
    v[j] = k < K ? xr[k] : 0.f;
    ss += v[j] * v[j];
  }
  ss = block_sum256(ss, sh);
  const float r = rsqrt_f(ss * rcp_f((float)K) + eps);
  float amax = 0.f;
#pragma unroll
  for (int j = 0; j < kNKmax / kT; ++j) {
    const int k = threadIdx.x + kT * j;
    v[j] = k < K ? (v[j] * r) * (1.0f + w[k]) : 0.f;
    amax = fmaxf(amax, fabsf(v[j]));
  }
  __syncthreads();
  // block max (wave max by xor shuffles, then across the 4 waves)
  for (int o = 32; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
  if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(sh[0], sh[1]), fmaxf(sh[2], sh[3]));
  float f, inv;
  split_scale(amax, f, inv);
  if (threadIdx.x == 0) invf[m] = inv;
#pragma unroll
  for (int j = 0; j < kNKmax / kT; ++j) {
    const int k = threadIdx.x + kT * j;
    if (k < K) {
      const float y = v[j] * f;
      const _Float16 h = (_Float16)y;
      yh[(size_t)m * ld16 + k] = h;
      yl[(size_t)m * ld16 + k] = (_Float16)(y - (float)h);
    }
  }
}

// ------------------------------------------------------------------ layout conversion
// Tile-major projection layout (q[t][K][256], scale[t][K][4], the last tile padded to 256
// columns; tiled = 1) or row-major KN (q[K][N], scale[K][N/64]; tiled = 0) -> MB layout (see the
// top).
__global__ void mb_convert_kernel(const int8_t* qt, const float* st, int K, int N, int tiled, int8_t* qb, float* sb) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;  // one 32-byte lane record
  const size_t nrec = (size_t)K * N / 32;
  if (i < nrec) {
    const int lane = (int)(i & 63);
    const size_t blk = i >> 6;  // cb * (K/32) + ks
    const int nks = K >> 5;
    const int cb = (int)(blk / nks), ks = (int)(blk % nks);
    const int g = lane >> 4, c = lane & 15;
    const int t = cb >> 2, cw = (cb & 3) * 64;
    uint32_t dw[8];
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        uint32_t v = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int k = 32 * ks + 8 * g + 4 * h + j;
          const size_t src = tiled ? ((size_t)t * K + k) * 256 + cw + 16 * nt + c : (size_t)k * N + 64 * cb + 16 * nt + c;
          const uint8_t b = (uint8_t)qt[src] ^ 0x80u;  // u = q + 128
          v |= (uint32_t)b << (8 * j);
        }
        dw[2 * nt + h] = v;
      }
    *(uint4*)(qb + i * 32) = make_uint4(dw[0], dw[1], dw[2], dw[3]);
    *(uint4*)(qb + i * 32 + 16) = make_uint4(dw[4], dw[5], dw[6], dw[7]);
  }
  const size_t ns = (size_t)K * (N / 64);
  if (i < ns) {  // scale[cb][k] = st[t][k][cb % 4] (tiled) or st[k][cb]
    const int cb = (int)(i / K), k = (int)(i % K);
    sb[i] = tiled ? st[((size_t)(cb >> 2) * K + k) * 4 + (cb & 3)] : st[(size_t)k * (N / 64) + cb];
  }
}

// The lm_head's table in load order: 16-byte chunk i = ((t * K/128 + r) * 8 + 4 kb + nt) * 64 + l
// holds row 64 t + 16 nt + (l & 15) (the last tile's rows past V repeat row V - 1), bytes
// k = 128 r + 64 kb + 16 (l >> 4) .. + 15.
__global__ void lm_table_kernel(const int8_t* q, int V, int K, int8_t* p, size_t nchunk) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= nchunk) return;
  const int l = (int)(i & 63), q8 = (int)((i >> 6) & 7);
  const size_t rest = i >> 9;
  const int nr = K / kRound, r = (int)(rest % nr);
  const size_t t = rest / nr;
  const int kb = q8 >> 2, nt = q8 & 3;
  const int row = (int)min((size_t)V - 1, 64 * t + 16 * nt + (l & 15));
  const int k = kRound * r + 64 * kb + 16 * (l >> 4);
  *(uint4*)(p + i * 16) = *(const uint4*)(q + (size_t)row * K + k);
}

// MB order -> stream order: 16-byte chunk (record b, lane l, half h) from b * 2048 + 32 l + 16 h
// to b * 2048 + 1024 h + 16 l.
__global__ void mb_stream_kernel(const int8_t* in, int8_t* out, size_t nchunk) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= nchunk) return;
  const size_t b = i >> 7;
  const int l = (int)(i & 63), h = (int)((i >> 6) & 1);
  *(uint4*)(out + b * 2048 + 1024 * h + 16 * l) = *(const uint4*)(in + b * 2048 + 32 * l + 16 * h);
}

// sT[kb][n] = s[n][kb] (the lm_head scales by 64-k block)
__global__ void scale_transpose_kernel(const float* s, int V, int nkb, float* sT) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < (size_t)V * nkb) {
    const int kb = (int)(i / V), n = (int)(i % V);
    sT[i] = s[(size_t)n * nkb + kb];
  }
}

}  // namespace

int mb_stream_launch(const int8_t* q_mb, size_t nbytes, int8_t* q_stream, hipStream_t st) {
  if (!q_mb || !q_stream) return fail(Q35_E_ARG, "mb_stream: null pointer");
  if (nbytes % 2048) return fail(Q35_E_SHAPE, "mb_stream: the MB copy is whole 2 KB records");
  if ((reinterpret_cast<uintptr_t>(q_mb) & 15) || (reinterpret_cast<uintptr_t>(q_stream) & 15))
    return fail(Q35_E_ALIGN, "mb_stream: 16-byte aligned copies");
  const size_t nchunk = nbytes / 16;
  hipLaunchKernelGGL(mb_stream_kernel, dim3((unsigned)((nchunk + 255) / 256)), dim3(256), 0, st, q_mb, q_stream, nchunk);
  Q35_HIP_TRY(hipGetLastError());
  return Q35_OK;
}

int mb_convert_launch(const int8_t* q_tiled, const float* s_tiled, int32_t K, int32_t N, int8_t* q_mb, float* s_mb,
                      hipStream_t st, int tiled) {
  if (!q_tiled || !s_tiled || !q_mb || !s_mb) return fail(Q35_E_ARG, "mb_convert: null pointer");
  if (K < 32 || K % 32 || N < 64 || N % 64) return fail(Q35_E_SHAPE, "mb_convert: need K % 32 == 0, N % 64 == 0");
  const size_t n = std::max((size_t)K * N / 32, (size_t)K * (N / 64));
  hipLaunchKernelGGL(mb_convert_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, q_tiled, s_tiled, K, N,
                     tiled, q_mb, s_mb);
  Q35_HIP_TRY(hipGetLastError());
  return Q35_OK;
}

int mb_scale_transpose_launch(const float* s, int32_t V, int32_t K, float* sT, hipStream_t st) {
  if (!s || !sT || V < 4 || K < 64 || K % 64) return fail(Q35_E_ARG, "mb_scale_transpose: bad arguments");
  const size_t n = (size_t)V * (K / 64);
  hipLaunchKernelGGL(scale_transpose_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, s, V, K / 64, sT);
  Q35_HIP_TRY(hipGetLastError());
  return Q35_OK;
}

namespace {

// Split factors of the RMS direct path: f[cb] = 2^e with sqrt(K) * max|1 + w| * max_k |s[cb][k]|
// * 2^e in [2^13, 2^14) (a bound on |y| of every row, see mbk_kernel).
__global__ __launch_bounds__(kT) void mb_split_factor_kernel(const float* sb, int K, const float* w, float* f) {
  __shared__ float sh[2][kT / 64];
  const int cb = blockIdx.x, t = threadIdx.x;
  float smax = 0.f, wmax = 0.f;
  for (int k = t; k < K; k += kT) {
    smax = fmaxf(smax, fabsf(sb[(size_t)cb * K + k]));
    wmax = fmaxf(wmax, fabsf(1.0f + w[k]));
  }
  for (int o = 32; o > 0; o >>= 1) {
    smax = fmaxf(smax, __shfl_xor(smax, o));
    wmax = fmaxf(wmax, __shfl_xor(wmax, o));
  }
  if ((t & 63) == 0) {
    sh[0][t >> 6] = smax;
    sh[1][t >> 6] = wmax;
  }
  __syncthreads();
  if (t == 0) {
    for (int i = 1; i < kT / 64; ++i) {
      smax = fmaxf(smax, sh[0][i]);
      wmax = fmaxf(wmax, sh[1][i]);
    }
    // (1 + 2^-10: room for the rounding of the row statistic and the products)
    const float bound = sqrtf((float)K) * wmax * smax * (1.0f + 0x1p-10f);
    float fv, inv;
    split_scale(bound, fv, inv);
    f[cb] = fv;
  }
}

}  // namespace

namespace {
__global__ __launch_bounds__(1024) void scale_max_kernel(const float* s, int64_t n, float* out) {
  __shared__ float red[16];
  float mx = 0.f;
  for (int64_t i = threadIdx.x; i < n; i += 1024) mx = fmaxf(mx, fabsf(s[i]));
  for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int i = 1; i < 16; ++i) mx = fmaxf(mx, red[i]);
    out[0] = mx;
  }
}
}  // namespace

namespace {
// ss[m] = fixed-point sum of squares of row m (one block per row), the RMS prologue's statistic
__global__ __launch_bounds__(kT) void mb_row_ss_kernel(const float* x, int32_t ldx, int32_t K, fx_t* ss, uint32_t* err) {
  __shared__ float sh[kT / 64];
  const float* r = x + (size_t)blockIdx.x * ldx;
  float a = 0.f;
  for (int k = threadIdx.x; k < K; k += kT) a += r[k] * r[k];
  a = wave_sum(a);
  if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = a;
  __syncthreads();
  if (threadIdx.x == 0) {
    float t = 0.f;
    for (int w = 0; w < kT / 64; ++w) t += sh[w];
    if (!fx_addable(t)) __hip_atomic_fetch_or((Q35_GLOBAL uint32_t*)err, kWsErrRange, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    ss[blockIdx.x] = fx_addable(t) ? to_fx(t) : 0;
  }
}
}  // namespace

int mb_row_ss_launch(const float* x, int32_t ldx, int32_t K, int32_t M, fx_t* ss, uint32_t* err, hipStream_t st) {
  if (!x || !ss || !err || M < 1 || K < 1) return fail(Q35_E_ARG, "mb_row_ss: bad arguments");
  hipLaunchKernelGGL(mb_row_ss_kernel, dim3((unsigned)M), dim3(kT), 0, st, x, ldx, K, ss, err);
  Q35_HIP_TRY(hipGetLastError());
  return Q35_OK;
}

int mb_scale_max_launch(const float* s, int64_t n, float* out, hipStream_t st) {
  if (!s || !out || n < 1) return fail(Q35_E_ARG, "mb_scale_max: bad arguments");
  hipLaunchKernelGGL(scale_max_kernel, dim3(1), dim3(1024), 0, st, s, n, out);
  Q35_HIP_TRY(hipGetLastError());
  return Q35_OK;
}

int mb_split_factor_launch(const float* s_mb, int32_t K, int32_t N, const float* norm_w, float* f, hipStream_t st) {
  if (!s_mb || !norm_w || !f || K < 1 || N < 64 || N % 64) return fail(Q35_E_ARG, "mb_split_factor: bad arguments");
  hipLaunchKernelGGL(mb_split_factor_kernel, dim3((unsigned)(N / 64)), dim3(kT), 0, st, s_mb, K, norm_w, f);
  Q35_HIP_TRY(hipGetLastError());
  return Q35_OK;
}

// Split-K plan for M rows: the fewest splits of whole 128-row rounds that give >= 160 blocks,
// with at most 1024 / MT rows per block when its x rows are staged in LDS, kDirectKR on the
// direct path.
void mb_plan(int ncb, int K, int M, bool direct, int* nsplit, int* kr) {
  const int nr = K / kRound, rmax = (direct ? kDirectKR : M <= 16 ? 1024 : 512) / kRound;
  int s = (nr + rmax - 1) / rmax;
  while (ncb * s < 160 && s < nr) ++s;
  const int rpb = (nr + s - 1) / s;
  *kr = rpb * kRound;
  *nsplit = (K + *kr - 1) / *kr;
}

size_t mb_part_floats(int ncb, int K, int M) {
  size_t n = 0;
  for (const bool direct : {false, true}) {
    int s, kr;
    mb_plan(ncb, K, M, direct, &s, &kr);
    const int Mp = M <= 16 ? 16 : 32;
    n = std::max(n, s > 1 ? (size_t)ncb * s * Mp * 64 : (size_t)0);
  }
  return n;
}

size_t mb_word_floats(int ncb, int M) { return (size_t)ncb * 64 * M * 2; }

namespace {
// staged prologues of up to 8 rows stage 8 (XBuf)
template <bool SO>
void mbk_dispatch(const MbkArgs& a, int M, int xs, bool direct, dim3 grid, hipStream_t st) {
  if (xs == 2) {  // (staged SwiGLU prologue, <= 16 rows)
    if (M <= 8) hipLaunchKernelGGL(HIP_KERNEL_NAME(mbk_kernel<1, false, 2, 8, SO>), grid, dim3(kT), 0, st, a);
    else hipLaunchKernelGGL(HIP_KERNEL_NAME(mbk_kernel<1, false, 2, 16, SO>), grid, dim3(kT), 0, st, a);
  } else if (M <= 16) {
    if (direct) hipLaunchKernelGGL(HIP_KERNEL_NAME(mbk_kernel<1, true, 1, 16, SO>), grid, dim3(kT), 0, st, a);
    else if (M <= 8) hipLaunchKernelGGL(HIP_KERNEL_NAME(mbk_kernel<1, false, 1, 8, SO>), grid, dim3(kT), 0, st, a);
    else hipLaunchKernelGGL(HIP_KERNEL_NAME(mbk_kernel<1, false, 1, 16, SO>), grid, dim3(kT), 0, st, a);
  } else {
    if (direct) hipLaunchKernelGGL(HIP_KERNEL_NAME(mbk_kernel<2, true, 1, 32, SO>), grid, dim3(kT), 0, st, a);
    else hipLaunchKernelGGL(HIP_KERNEL_NAME(mbk_kernel<2, false, 1, 32, SO>), grid, dim3(kT), 0, st, a);
  }
}
}  // namespace

int mb_launch(const MbCall& c, hipStream_t st) {
  if (c.nseg < 1 || c.nseg > kMbMaxSeg) return fail(Q35_E_ARG, "mb_launch: 1..4 segments");
  if (c.M < 1 || c.M > 32) return fail(Q35_E_SHAPE, "mb_launch: M in [1, 32]");
  if (c.K < kRound || c.K % kRound) return fail(Q35_E_SHAPE, "mb_launch: K must be a positive multiple of 128");
  if (!c.x || c.ldx < c.K) return fail(Q35_E_ARG, "mb_launch: x");
  if ((reinterpret_cast<uintptr_t>(c.x) & 15) || (c.ldx & 3)) return fail(Q35_E_ALIGN, "mb_launch: x rows 16-byte aligned");
  if (c.pro == MB_PRO_RMS && (!c.ss || !c.pw)) return fail(Q35_E_ARG, "mb_launch: RMS needs ss and w");
  if (c.pro == MB_PRO_GATED) {
    const int vpt = c.M <= 8 ? 4 : c.M <= 16 ? 8 : 16;  // values per staging thread (XBuf)
    if (!c.z || !c.pw || c.group < vpt || c.group > kRound || (c.group & (c.group - 1)) || (c.ldz & 3) ||
        (reinterpret_cast<uintptr_t>(c.z) & 15))
      return fail(Q35_E_ARG, "mb_launch: gated prologue needs z (16-byte rows) and a power-of-two group in [vpt, 128]");
  }
  if (c.pro == MB_PRO_SWIGLU && (c.swiglu_off & 3)) return fail(Q35_E_ALIGN, "mb_launch: SwiGLU offset % 4");
  MbkArgs a{};
  a.nseg = c.nseg; a.K = c.K; a.M = c.M;
  int ncb = 0;
  for (int i = 0; i < c.nseg; ++i) {
    const MbSeg& s = c.seg[i];
    if (!s.q || !s.s || !s.y) return fail(Q35_E_ARG, "mb_launch: null segment");
    if (s.N < 64 || s.N % 64) return fail(Q35_E_SHAPE, "mb_launch: segment N % 64");
    if (c.add && ((reinterpret_cast<uintptr_t>(s.y) & 15) || (s.ldy & 3)))
      return fail(Q35_E_ALIGN, "mb_launch: residual rows 16-byte aligned");
    if ((reinterpret_cast<uintptr_t>(s.q) & 15)) return fail(Q35_E_ALIGN, "mb_launch: weights 16-byte aligned");
    a.seg[i] = MbkSeg{s.q, s.s, s.y, s.f, s.N, s.ldy, ncb};
    ncb += s.N / 64;
  }
  for (int i = c.nseg; i < kMbMaxSeg; ++i) {
    a.seg[i] = a.seg[0];
    a.seg[i].cb0 = INT32_MAX;
  }
  a.ncb = ncb;
  bool direct = c.pro == MB_PRO_RMS;
  for (int i = 0; i < c.nseg; ++i) direct = direct && c.seg[i].f;
  mb_plan(ncb, c.K, c.M, direct, &a.nsplit, &a.kr);
  a.x = c.x; a.ldx = c.ldx; a.pro = c.pro; a.pw = c.pw; a.eps = c.eps;
  a.ss = c.pro == MB_PRO_RMS ? c.ss : reinterpret_cast<const fx_t*>(c.x);  // rows of x: >= 8 M bytes
  a.z = c.z; a.ldz = c.ldz; a.group = c.group; a.swiglu_off = c.swiglu_off;
  a.add = c.add; a.ss_out = c.ss_out;
  if (!c.err) return fail(Q35_E_ARG, "mb_launch: null error word");
  a.err = c.err;
  // two-split launches of up to 16 rows without a residual add may leave their partials to the
  // consumer (for 17..32 rows the consumer's doubled staging costs more than the hand-off saves)
  a.dstride = (c.defer_stride > 0 && a.nsplit == 2 && c.M <= 16 && !c.add && !c.ss_out) ? c.defer_stride : 0;
  if (c.deferred_out) *c.deferred_out = a.dstride > 0 ? 1 : 0;
  if (a.dstride)
    for (int i = 0; i < c.nseg; ++i)
      if ((reinterpret_cast<uintptr_t>(c.seg[i].y) & 15) || (c.seg[i].ldy & 3) || (c.defer_stride & 3))
        return fail(Q35_E_ALIGN, "mb_launch: deferred partial rows 16-byte aligned");
  const int xs = c.xsum == 2 ? 2 : 1;
  if (c.xsum != 1 && (c.xsum != 2 || c.pro != MB_PRO_SWIGLU || c.M > 16 || (c.xsstride & 3)))
    return fail(Q35_E_ARG, "mb_launch: a two-partial input is supported for the SwiGLU prologue of <= 16 rows only");
  a.xsstride = xs == 2 ? c.xsstride : 0;
  a.aux_wb = c.aux_wb; a.aux_wa = c.aux_wa; a.aux_nh = c.aux_nh; a.aux_acc = c.aux_acc; a.aux_ldo = c.aux_ldo;
  a.naux = c.aux_acc ? c.K / kRound : 0;
  if (c.aux_acc && (c.aux_nh < 1 || 2 * c.aux_nh > 32 || !c.aux_wb || !c.aux_wa))
    return fail(Q35_E_ARG, "mb_launch: gate side task needs 1..16 heads and both weights");
  if (a.nsplit > 1 && !a.dstride) {
    // the hand-off: counted words when the atomics they cost (one per output and split) are few
    // or the splits many, else partials and an arrival counter
    const size_t np = (size_t)ncb * a.nsplit * (c.M <= 16 ? 16 : 32) * 64, nw = mb_word_floats(ncb, c.M);
    const size_t atomics = (size_t)ncb * 64 * c.M * a.nsplit;
    a.counted = (atomics <= kCountedMax || (atomics <= kCountedMaxSplit && a.nsplit >= 5)) ? 1 : 0;
    if (!c.part || c.part_floats < np || !c.ctr || c.nctr < ncb) return fail(Q35_E_WS, "mb_launch: split-K partials / counters too small");
    if (!c.words || c.word_floats < nw || (reinterpret_cast<uintptr_t>(c.words) & 7))
      return fail(Q35_E_WS, "mb_launch: split-K counted words too small");
    a.part = c.part; a.ctr = c.ctr;
    a.words = reinterpret_cast<uint64_t*>(c.words);
  }
  const dim3 grid((unsigned)(ncb * a.nsplit + a.naux));
  if (c.stream_order) mbk_dispatch<true>(a, c.M, xs, direct, grid, st);
  else mbk_dispatch<false>(a, c.M, xs, direct, grid, st);
  Q35_HIP_TRY(hipGetLastError());
  return Q35_OK;
}

size_t mb_lm_table_bytes(int32_t V, int32_t K) { return (size_t)((V + 63) / 64) * 64 * (size_t)K; }

int mb_lm_table_launch(const int8_t* q, int32_t V, int32_t K, int8_t* p, hipStream_t st) {
  if (!q || !p) return fail(Q35_E_ARG, "mb_lm_table: null pointer");
  if (K < kRound || K % kRound || V < 1) return fail(Q35_E_SHAPE, "mb_lm_table: K must be a multiple of 128");
  if ((reinterpret_cast<uintptr_t>(q) & 15) || (reinterpret_cast<uintptr_t>(p) & 15))
    return fail(Q35_E_ALIGN, "mb_lm_table: 16-byte aligned tables");
  const size_t nchunk = mb_lm_table_bytes(V, K) / 16;
  hipLaunchKernelGGL(lm_table_kernel, dim3((unsigned)((nchunk + 255) / 256)), dim3(256), 0, st, q, V, K, p, nchunk);
  Q35_HIP_TRY(hipGetLastError());
  return Q35_OK;
}

int mb_lm_head_launch(const int8_t* q, const float* sT, int32_t V, int32_t K, const float* h, int32_t ldh,
                      const float* norm_w, float eps, int32_t M, _Float16* split16, float* invf, float* y, int32_t ldy,
                      hipStream_t st) {
  if (!q || !sT || !h || !norm_w || !split16 || !invf || !y) return fail(Q35_E_ARG, "mb_lm_head: null pointer");
  if (M < 1 || M > 32) return fail(Q35_E_SHAPE, "mb_lm_head: M in [1, 32]");
  if (K < 512 || K % 512 || K > kNKmax || V < 4 || V % 4)
    return fail(Q35_E_SHAPE, "mb_lm_head: K must be a multiple of 512, at most 2048, and V of 4");
  if ((reinterpret_cast<uintptr_t>(q) & 15) || (reinterpret_cast<uintptr_t>(split16) & 15))
    return fail(Q35_E_ALIGN, "mb_lm_head: 16-byte aligned table and split rows");
  _Float16* yh = split16;
  _Float16* yl = split16 + (size_t)M * K;
  hipLaunchKernelGGL(rms_rows_split_kernel, dim3(M), dim3(kT), 0, st, h, ldh, K, norm_w, eps, yh, yl, K, invf);
  const dim3 grid((unsigned)((V + 255) / 256));
  for (int m0 = 0; m0 < M; m0 += 16) {  // 16 rows per pass over the table
    MbnArgs a{q, sT, V, K, std::min(16, M - m0), yh + (size_t)m0 * K, yl + (size_t)m0 * K, K, invf + m0,
              y + (size_t)m0 * ldy, ldy};
    if (a.M <= 8) hipLaunchKernelGGL(mbn_kernel<8>, grid, dim3(kT), 0, st, a);
    else hipLaunchKernelGGL(mbn_kernel<16>, grid, dim3(kT), 0, st, a);
  }
  Q35_HIP_TRY(hipGetLastError());
  return Q35_OK;
}

}  // namespace q35
