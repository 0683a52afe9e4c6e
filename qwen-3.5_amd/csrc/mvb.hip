// Batched decode projections on the fp32 matrix cores: Y[m][n] = sum_k X~[m][k] * dequant(W)[k][n]
// for up to 32 decode rows m at once (the B sequences of a batched step), so that every weight
// matrix is streamed once per step for all rows.  The arithmetic is the reference's Linear on a
// QFloat weight (text_modules.rs:500-508, :578-595, :638-647, :880-890, :1003-1005;
// kernels.rs:53-92 for the Q8F block scales): each weight is dequantised to f32 (q * scale, one
// rounding) and multiplied with v_mfma_f32_16x16x4_f32, i.e. f32 products, f32 accumulation.
//
// Weight layout (Q35 "MB", built once from the tile-major projection layout): per 64-column
// block cb and 16-row step ks, 1 KB in which lane l = 16 g + c of a wave finds, as one 16-byte
// load, the bytes u = q + 128 of q[16 ks + 4 g + j][64 cb + 16 nt + c] (j = 0..3) for each of
// the 4 column tiles nt.  Those are exactly its A operands (row c of tile nt, k slot g) for the
// 4 MFMA sub-steps j, with the k order permuted inside the step (the sum is unchanged).  Scales
// are stored per column block, scale[cb][K], so a lane's 4 scales are one 16-byte read.
//
// Block = 4 waves = one column block (64 outputs) x the block's K range (at most 1024 / MT
// rows).  The block first stages its Mp x K-range input rows, transformed by the prologue
// (RMSNorm, gated RMSNorm or SwiGLU of the producer's output), in LDS with one round trip; then
// the waves stream their weights with no further synchronisation: wave p takes the k steps
// 2p and 2p+1 of every 128-row round, its weights loaded 4 rounds ahead, and reads its B
// operands (16-byte reads) from the staged rows.  The 4 waves' accumulators are summed through
// LDS in a fixed order.  A block with the whole K writes its outputs directly; with split-K the
// blocks of a column block publish partials and the last to arrive sums them in split order
// (deterministic).  Residual projections add into the f32 residual rows and accumulate each
// row's sum of squares for the next RMSNorm (fixed point, so the sum is order-independent).
//
// The lm_head (mbn_kernel) reads the tied [V][D] table directly: lane l = 16 g + c takes 16
// consecutive bytes of vocab row c of a tile (k = 16 g .. 16 g + 15 of a 64-wide scale block),
// which are its A operands for 16 sub-steps; the row's block scale is applied to the dequantised
// value.  Blocks of 4 waves x 64 vocab rows copy the 16 normalised x rows whole into LDS.
#include "q35_internal.h"

#include <algorithm>
#include <climits>

namespace q35 {
namespace {

constexpr int kT = 256;            // threads per block (4 waves)
constexpr int kRound = 128;        // K rows per round (4 waves x 2 k steps of 16)
constexpr int kDepth = 4;          // rounds of weights in flight per wave (mbk)
constexpr int kNDepth = 2;         // rounds in flight per wave (mbn)
constexpr int kNKmax = 2048;       // lm_head: largest hidden size (the whole x rows sit in LDS)

typedef float f4 __attribute__((ext_vector_type(4)));

struct MbkSeg {
  const int8_t* q;  // MB layout
  const float* s;   // [N/64][K]
  float* y;
  int32_t N, ldy, cb0;  // cb0: first column block of the segment in the launch
};
struct MbkArgs {
  MbkSeg seg[kMbMaxSeg];
  int32_t nseg, K, M, ncb, nsplit, kr;
  const float* x; int32_t ldx;
  int32_t pro; const float* pw; float eps; const fx_t* ss;
  const float* z; int32_t ldz, group, swiglu_off;
  int32_t add; fx_t* ss_out;
  const float* aux_wb; const float* aux_wa; int32_t aux_nh; fx_t* aux_acc; int32_t aux_ldo, naux;
  float* part; uint32_t* ctr;
};

Q35_DEV f4 ld4(const float* p) { return *(const Q35_GLOBAL f4*)p; }
Q35_DEV f4 lds4(const float* p) { return *(const f4*)p; }

// Byte j of dw holds u = q + 128 (q the int8 weight): f32(q) * s, rounded once, computed as
// fma(u, s, -128 s) (u converts with one instruction; -128 s is exact).
Q35_DEV float dq_byte(uint32_t dw, int j, float s, float neg128s) {
  return __builtin_fmaf((float)((dw >> (8 * j)) & 0xffu), s, neg128s);
}

// A block's x rows live in LDS for its whole K range: at most 1024 / MT rows of Mp = 16 MT rows
// (64 KB), each row padded by 4 floats so that the 16 rows a B-operand read touches start in
// different banks.
template <int MT>
struct XBuf {
  static constexpr int Mp = 16 * MT;
  static constexpr int KR = 1024 / MT;         // rows of K per block
  static constexpr int LD = KR + 4;            // floats per staged x row
  static constexpr int NCH = KR / kRound;      // 128-row chunks
  static constexpr int TPR = kT / Mp;          // staging threads per x row: 16 or 8
  static constexpr int VPT = kRound / TPR;     // values per thread per chunk: 8 or 16
};

// Stage x~ for rows [k0, k0 + klen) (klen a multiple of 128, <= KR) into xs: every load the
// range needs (x, the second operand, the norm weights, the row statistic) is issued first, so
// staging costs one round trip; then each chunk is transformed by the prologue and written.
// Thread t covers row t / TPR of every chunk, columns (t % TPR) * VPT .. + VPT; the rows of the
// chunk past M repeat row M - 1 (their outputs are never stored).  The column block's weight
// scales for the range go to scs.
template <int MT>
Q35_DEV void stage_x(const MbkArgs& a, int k0, int klen, float* xs, float* scs, const float* scl) {
  using X = XBuf<MT>;
  const int t = threadIdx.x, mr = t / X::TPR, m = min(mr, a.M - 1), c0 = (t % X::TPR) * X::VPT;
  const int nch = klen / kRound;
  const bool rms = a.pro == MB_PRO_RMS, gated = a.pro == MB_PRO_GATED, two = gated || a.pro == MB_PRO_SWIGLU;
  const float* xr = a.x + (size_t)m * a.ldx + k0 + c0;
  const float* ur = gated ? a.z + (size_t)m * a.ldz + k0 + c0 : xr + a.swiglu_off;
  float v[X::NCH][X::VPT], u[X::NCH][X::VPT];
  float wg[X::VPT];  // norm weights: gated (the same VPT for every chunk), RMS (into u)
  f4 sc = f4{0.f, 0.f, 0.f, 0.f};
  if (scl && 4 * t < klen) sc = ld4(scl + k0 + 4 * t);
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
      const f4 q = ld4(xr + cc + i);
      v[ci][i] = q[0]; v[ci][i + 1] = q[1]; v[ci][i + 2] = q[2]; v[ci][i + 3] = q[3];
      if (two || rms) {
        const f4 w = ld4(rms ? a.pw + k0 + cc + c0 + i : ur + cc + i);
        u[ci][i] = w[0]; u[ci][i + 1] = w[1]; u[ci][i + 2] = w[2]; u[ci][i + 3] = w[3];
      }
    }
  }
  if (scs && 4 * t < klen) *(f4*)(scs + 4 * t) = sc;
  // y = x * rsqrt(mean(x^2) + eps) * (1 + w)  (text_modules.rs:800-808); the row's sum of
  // squares comes from the projection that produced x
  const float r = rsqrt_f(from_fx(ssv) * rcp_f((float)a.K) + a.eps);
  const int tpg = gated ? a.group / X::VPT : 1;  // gated: threads per group (power of two <= TPR)
#pragma unroll
  for (int ci = 0; ci < X::NCH; ++ci) {
    if (rms) {
#pragma unroll
      for (int i = 0; i < X::VPT; ++i) v[ci][i] = (v[ci][i] * r) * (1.0f + u[ci][i]);
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
    if (ci < nch) {
      float* dst = xs + mr * X::LD + ci * kRound + c0;
#pragma unroll
      for (int i = 0; i < X::VPT; i += 4) *(f4*)(dst + i) = f4{v[ci][i], v[ci][i + 1], v[ci][i + 2], v[ci][i + 3]};
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
template <int MT>
Q35_DEV void mbk_aux(const MbkArgs& a, int ab, float* xs, float* red) {
  using X = XBuf<MT>;
  const int t = threadIdx.x, kc = ab * kRound;
  stage_x<MT>(a, kc, kRound, xs, nullptr, nullptr);
  __syncthreads();
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
    for (int i = 0; i < 16; ++i) acc += xs[m * X::LD + rg * 16 + i] * w[i];
    red[rg * 32 + o] = acc;
    __syncthreads();
    if (t < no) {
      float v = 0.f;
#pragma unroll
      for (int g = 0; g < 8; ++g) v += red[g * 32 + t];
      fx_add(&a.aux_acc[(size_t)m * a.aux_ldo + t], v);
    }
    __syncthreads();
  }
}

template <int MT>
__global__ __launch_bounds__(kT, 1) void mbk_kernel(const MbkArgs a) {
  using X = XBuf<MT>;
  constexpr int Mp = X::Mp;
  __shared__ __align__(16) float xs[Mp * X::LD];  // staged x~; reused for the wave reduction
  __shared__ __align__(16) float scs[X::KR];
  __shared__ __align__(16) float aux_red[256];
  __shared__ float sq[4][Mp];
  __shared__ int last_flag;
  static_assert(4 * 16 * MT * 64 <= Mp * X::LD, "reduction buffer");

  const int nmain = a.ncb * a.nsplit;
  if ((int)blockIdx.x >= nmain) {
    mbk_aux<MT>(a, (int)blockIdx.x - nmain, xs, aux_red);
    return;
  }
  const int tid = threadIdx.x, lane = tid & 63, p = tid >> 6, g = lane >> 4, c = lane & 15;
  const int cb = (int)blockIdx.x / a.nsplit, split = (int)blockIdx.x - cb * a.nsplit;
  const MbkSeg sg = seg_of(a, cb);
  const int lcb = cb - sg.cb0;
  const int k0 = split * a.kr, klen = min(a.kr, a.K - k0);
  const int nround = klen / kRound;
  const int nks = a.K >> 4;
  // wave p's k steps in round r: 8 r + 2 p + e (e = 0, 1), relative to k0
  const int8_t* wq = sg.q + ((size_t)lcb * nks + (k0 >> 4) + 2 * p) * 1024 + lane * 16;

  // Rounds past the block's range load 16 bytes per lane of its (cached) scales instead, so every
  // round issues the same loads and the compiler's waits count them exactly.
  const float* scl = sg.s + (size_t)lcb * a.K;
  const int8_t* dummy = reinterpret_cast<const int8_t*>(scl) + lane * 16;
  q35_u32x4 wr[kDepth][2];
  auto load_round = [&](int r, q35_u32x4 (&w)[2]) {
#pragma unroll
    for (int e = 0; e < 2; ++e) w[e] = ldg16v_nt(r < nround ? wq + ((size_t)r * 8 + e) * 1024 : dummy);
  };
  static_for<kDepth>([&](auto d) { load_round(d, wr[d]); });
  stage_x<MT>(a, k0, klen, xs, scs, scl);
  __syncthreads();

  f4 acc[4][MT];
#pragma unroll
  for (int nt = 0; nt < 4; ++nt)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[nt][mt] = f4{0.f, 0.f, 0.f, 0.f};

  // every round unrolled (at most KR / 128 of them), so the compiler's waits for the weight
  // loads count exactly the rounds still in flight
  static_for<X::NCH>([&](auto rc) {
    constexpr int r = rc, d = r % kDepth;
    if (r < nround) {
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const int kl = r * kRound + 16 * (2 * p + e) + 4 * g;
          f4 xv[MT];
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) xv[mt] = lds4(xs + (16 * mt + c) * X::LD + kl);
          const f4 sv = lds4(scs + kl);
          const q35_u32x4 w = wr[d][e];
          // dequantise the 16 weights first (independent), then issue the MFMAs with the four
          // column tiles' accumulator chains interleaved
          float av[4][4];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const float nb = -128.0f * sv[j];
#pragma unroll
            for (int nt = 0; nt < 4; ++nt) av[nt][j] = dq_byte(w[nt], j, sv[j], nb);
          }
#pragma unroll
          for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int nt = 0; nt < 4; ++nt)
#pragma unroll
              for (int mt = 0; mt < MT; ++mt)
                acc[nt][mt] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[nt][j], xv[mt][j], acc[nt][mt], 0, 0, 0);
        }
        if (r + kDepth < X::NCH) {
          load_round(r + kDepth, wr[d]);
          asm volatile("" ::: "memory");  // keep the prefetch here (not sunk to its use)
        }
    }
  });

  // Sum the 4 waves' partial sums: wave p writes its accumulators, then finalises column tile
  // nt = p (16 columns x Mp rows) from all four in wave order.
  float* red = xs;
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
    out[mt] = v;
  }
  // lane holds columns n = 16 p + 4 g + i (i = 0..3) of row m = 16 mt + c
  const int ncol0 = 64 * lcb + 16 * p + 4 * g;
  if (a.nsplit > 1) {
    float* pp = a.part + ((size_t)cb * a.nsplit + split) * Mp * 64;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i) st_agent(pp + (16 * mt + c) * 64 + 16 * p + 4 * g + i, out[mt][i]);
    if (!arrive_last(a.ctr + cb, (uint32_t)a.nsplit, &last_flag)) return;
    // the last block of the column block sums the partials in split order
    const float* pb = a.part + (size_t)cb * a.nsplit * Mp * 64;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      f4 v = f4{0.f, 0.f, 0.f, 0.f};
      for (int s2 = 0; s2 < a.nsplit; ++s2) {
        const float* q = pb + (size_t)s2 * Mp * 64 + (16 * mt + c) * 64 + 16 * p + 4 * g;
        v += f4{ld_agent(q), ld_agent(q + 1), ld_agent(q + 2), ld_agent(q + 3)};
      }
      out[mt] = v;
    }
  }
  // write (or add) the outputs of rows m < M; residual adds also sum the new rows' squares
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = 16 * mt + c;
    float sqs = 0.f;
    if (m < a.M) {
      float* yr = sg.y + (size_t)m * sg.ldy + ncol0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float v = out[mt][i];
        if (a.add) v += yr[i];
        yr[i] = v;
        sqs += v * v;
      }
    }
    if (a.ss_out) {
      sqs += __shfl_xor(sqs, 16);
      sqs += __shfl_xor(sqs, 32);
      if (g == 0) sq[p][m] = sqs;
    }
  }
  if (a.ss_out) {
    __syncthreads();
    if (tid < a.M) fx_add(a.ss_out + tid, ((sq[0][tid] + sq[1][tid]) + sq[2][tid]) + sq[3][tid]);
  }
}

// ------------------------------------------------------------------ lm_head over the NK table
struct MbnArgs {
  const int8_t* q;  // [V][K]
  const float* s;   // [V][K/64]
  int32_t V, K, M;
  const float* x; int32_t ldx;  // normalised rows [M][ldx]
  float* y; int32_t ldy;        // logits [M][ldy]
};

// One 16-byte copy per lane from global memory into LDS: lane l writes dst + 16 l (dst is
// wave-uniform).  Counted by vmcnt like any vector load.
Q35_DEV void dma16(const void* src, float* dst) {
  __builtin_amdgcn_global_load_lds((const Q35_GLOBAL void*)src, (__attribute__((address_space(3))) void*)dst, 16, 0, 0);
}

// 16 rows (M <= 16) per launch; the whole normalised x rows are copied into LDS once.
__global__ __launch_bounds__(kT, 1) void mbn_kernel(const MbnArgs a) {
  constexpr int LD = kNKmax + 4;
  __shared__ __align__(16) float xs[16 * LD];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 4, c = lane & 15;
  const int nbase = (int)blockIdx.x * 256 + 64 * w;  // this wave's 64 vocab rows
  const int nround = a.K / kRound, nkb = a.K >> 6;

  // x rows into LDS: segments of 256 floats (one wave instruction each), rows past M repeat M - 1
  const int nseg = 16 * (a.K / 256);
  for (int sgi = w; sgi < nseg; sgi += 4) {
    const int m = sgi / (a.K / 256), k = (sgi % (a.K / 256)) * 256;
    dma16(a.x + (size_t)min(m, a.M - 1) * a.ldx + k + 4 * lane, xs + m * LD + k);
  }
  // lane's rows n = nbase + 16 nt + c (clamped for the loads; not stored past V)
  const int8_t* rowp[4];
  const float* srow[4];
#pragma unroll
  for (int nt = 0; nt < 4; ++nt) {
    const int n = min(nbase + 16 * nt + c, a.V - 1);
    rowp[nt] = a.q + (size_t)n * a.K + 16 * g;
    srow[nt] = a.s + (size_t)n * nkb;
  }
  // (rounds past K load the first round again: every round issues the same loads, so the
  // compiler's waits count them exactly)
  q35_u32x4 wr[kNDepth][2][4];
  float sr[kNDepth][2][4];
  auto load_round = [&](int r, q35_u32x4 (&wv)[2][4], float (&sv)[2][4]) {
    const int rr = r < nround ? r : 0;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) {
        wv[kb][nt] = ldg16v_nt(rowp[nt] + rr * kRound + 64 * kb);
        sv[kb][nt] = ldg(srow[nt] + 2 * rr + kb);
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
          // x[c][k + 16 g + i], i = 0..15, k = 128 r + 64 kb
          f4 xv[4];
#pragma unroll
          for (int h = 0; h < 4; ++h) xv[h] = lds4(xs + c * LD + r * kRound + 64 * kb + 16 * g + 4 * h);
#pragma unroll
          for (int h = 0; h < 4; ++h) {  // 4 sub-steps at a time: dequantise, then interleave
            float av[4][4];
#pragma unroll
            for (int nt = 0; nt < 4; ++nt) {
              const float scl = sr[d][kb][nt];
              const uint32_t dw = wr[d][kb][nt][h] ^ 0x80808080u;  // int8 -> u = q + 128
#pragma unroll
              for (int j = 0; j < 4; ++j) av[nt][j] = dq_byte(dw, j, scl, -128.0f * scl);
            }
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
              for (int nt = 0; nt < 4; ++nt)
                acc[nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[nt][j], xv[h][j], acc[nt], 0, 0, 0);
          }
        }
        if (r + kNDepth < kNKmax / kRound) {
          load_round(r + kNDepth, wr[d], sr[d]);
          asm volatile("" ::: "memory");  // keep the prefetch here (not sunk to its use)
        }
    }
  });
  // lane holds rows n = nbase + 16 nt + 4 g + i of column m = c
  if (c < a.M) {
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int n = nbase + 16 * nt + 4 * g + i;
        if (n < a.V) a.y[(size_t)c * a.ldy + n] = acc[nt][i];
      }
  }
}

// ------------------------------------------------------------------ layout conversion
// Tile-major projection layout (q[t][K][256], scale[t][K][4], the last tile padded to 256
// columns) -> MB layout (see the top).
__global__ void mb_convert_kernel(const int8_t* qt, const float* st, int K, int N, int8_t* qb, float* sb) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;  // one 16-byte lane record
  const size_t nrec = (size_t)K * N / 16;
  if (i < nrec) {
    const int lane = (int)(i & 63);
    const size_t blk = i >> 6;  // cb * (K/16) + ks
    const int nks = K >> 4;
    const int cb = (int)(blk / nks), ks = (int)(blk % nks);
    const int g = lane >> 4, c = lane & 15;
    const int t = cb >> 2, cw = (cb & 3) * 64;
    uint32_t dw[4];
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      uint32_t v = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int k = 16 * ks + 4 * g + j;
        const uint8_t b = (uint8_t)qt[((size_t)t * K + k) * 256 + cw + 16 * nt + c] ^ 0x80u;  // u = q + 128
        v |= (uint32_t)b << (8 * j);
      }
      dw[nt] = v;
    }
    *(uint4*)(qb + i * 16) = make_uint4(dw[0], dw[1], dw[2], dw[3]);
  }
  const size_t ns = (size_t)K * (N / 64);
  if (i < ns) {  // scale[cb][k] = st[t][k][cb % 4]
    const int cb = (int)(i / K), k = (int)(i % K);
    sb[i] = st[((size_t)(cb >> 2) * K + k) * 4 + (cb & 3)];
  }
}

}  // namespace

int mb_convert_launch(const int8_t* q_tiled, const float* s_tiled, int32_t K, int32_t N, int8_t* q_mb, float* s_mb,
                      hipStream_t st) {
  if (!q_tiled || !s_tiled || !q_mb || !s_mb) return fail(Q35_E_ARG, "mb_convert: null pointer");
  if (K < 16 || K % 16 || N < 64 || N % 64) return fail(Q35_E_SHAPE, "mb_convert: need K % 16 == 0, N % 64 == 0");
  const size_t n = std::max((size_t)K * N / 16, (size_t)K * (N / 64));
  hipLaunchKernelGGL(mb_convert_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, q_tiled, s_tiled, K, N,
                     q_mb, s_mb);
  Q35_HIP_TRY(hipGetLastError());
  return Q35_OK;
}

// Split-K plan for M rows: the fewest splits of whole 128-row rounds that give >= 160 blocks,
// with at most 1024 / MT rows per block (its x rows sit in LDS).
void mb_plan(int ncb, int K, int M, int* nsplit, int* kr) {
  const int nr = K / kRound, rmax = (M <= 16 ? 1024 : 512) / kRound;
  int s = (nr + rmax - 1) / rmax;
  while (ncb * s < 160 && s < nr) ++s;
  const int rpb = (nr + s - 1) / s;
  *kr = rpb * kRound;
  *nsplit = (K + *kr - 1) / *kr;
}

size_t mb_part_floats(int ncb, int K, int M) {
  int s, kr;
  mb_plan(ncb, K, M, &s, &kr);
  const int Mp = M <= 16 ? 16 : 32;
  return s > 1 ? (size_t)ncb * s * Mp * 64 : 0;
}

int mb_launch(const MbCall& c, hipStream_t st) {
  if (c.nseg < 1 || c.nseg > kMbMaxSeg) return fail(Q35_E_ARG, "mb_launch: 1..4 segments");
  if (c.M < 1 || c.M > 32) return fail(Q35_E_SHAPE, "mb_launch: M in [1, 32]");
  if (c.K < kRound || c.K % kRound) return fail(Q35_E_SHAPE, "mb_launch: K must be a positive multiple of 128");
  if (!c.x || c.ldx < c.K) return fail(Q35_E_ARG, "mb_launch: x");
  if ((reinterpret_cast<uintptr_t>(c.x) & 15) || (c.ldx & 3)) return fail(Q35_E_ALIGN, "mb_launch: x rows 16-byte aligned");
  if (c.pro == MB_PRO_RMS && (!c.ss || !c.pw)) return fail(Q35_E_ARG, "mb_launch: RMS needs ss and w");
  if (c.pro == MB_PRO_GATED) {
    const int vpt = c.M <= 16 ? 8 : 16;
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
    if ((reinterpret_cast<uintptr_t>(s.q) & 15)) return fail(Q35_E_ALIGN, "mb_launch: weights 16-byte aligned");
    a.seg[i] = MbkSeg{s.q, s.s, s.y, s.N, s.ldy, ncb};
    ncb += s.N / 64;
  }
  for (int i = c.nseg; i < kMbMaxSeg; ++i) {
    a.seg[i] = a.seg[0];
    a.seg[i].cb0 = INT32_MAX;
  }
  a.ncb = ncb;
  mb_plan(ncb, c.K, c.M, &a.nsplit, &a.kr);
  a.x = c.x; a.ldx = c.ldx; a.pro = c.pro; a.pw = c.pw; a.eps = c.eps;
  a.ss = c.pro == MB_PRO_RMS ? c.ss : reinterpret_cast<const fx_t*>(c.x);  // rows of x: >= 8 M bytes
  a.z = c.z; a.ldz = c.ldz; a.group = c.group; a.swiglu_off = c.swiglu_off;
  a.add = c.add; a.ss_out = c.ss_out;
  a.aux_wb = c.aux_wb; a.aux_wa = c.aux_wa; a.aux_nh = c.aux_nh; a.aux_acc = c.aux_acc; a.aux_ldo = c.aux_ldo;
  a.naux = c.aux_acc ? c.K / kRound : 0;
  if (c.aux_acc && (c.aux_nh < 1 || 2 * c.aux_nh > 32 || !c.aux_wb || !c.aux_wa))
    return fail(Q35_E_ARG, "mb_launch: gate side task needs 1..16 heads and both weights");
  if (a.nsplit > 1) {
    const size_t need = (size_t)ncb * a.nsplit * (c.M <= 16 ? 16 : 32) * 64;
    if (!c.part || c.part_floats < need || !c.ctr || c.nctr < ncb)
      return fail(Q35_E_WS, "mb_launch: split-K partials / counters too small");
    a.part = c.part; a.ctr = c.ctr;
  }
  const dim3 grid((unsigned)(ncb * a.nsplit + a.naux));
  if (c.M <= 16) hipLaunchKernelGGL(mbk_kernel<1>, grid, dim3(kT), 0, st, a);
  else hipLaunchKernelGGL(mbk_kernel<2>, grid, dim3(kT), 0, st, a);
  Q35_HIP_TRY(hipGetLastError());
  return Q35_OK;
}

int mb_lm_head_launch(const int8_t* q, const float* s, int32_t V, int32_t K, const float* x, int32_t ldx, int32_t M,
                      float* y, int32_t ldy, hipStream_t st) {
  if (!q || !s || !x || !y) return fail(Q35_E_ARG, "mb_lm_head: null pointer");
  if (M < 1 || M > 32) return fail(Q35_E_SHAPE, "mb_lm_head: M in [1, 32]");
  if (K < 256 || K % 256 || K > kNKmax || V < 1)
    return fail(Q35_E_SHAPE, "mb_lm_head: K must be a multiple of 256, at most 2048");
  if ((reinterpret_cast<uintptr_t>(q) & 15) || (reinterpret_cast<uintptr_t>(x) & 15) || (ldx & 3))
    return fail(Q35_E_ALIGN, "mb_lm_head: 16-byte aligned table and rows");
  const dim3 grid((unsigned)((V + 255) / 256));
  for (int m0 = 0; m0 < M; m0 += 16) {  // 16 rows per pass over the table
    MbnArgs a{q, s, V, K, std::min(16, M - m0), x + (size_t)m0 * ldx, ldx, y + (size_t)m0 * ldy, ldy};
    hipLaunchKernelGGL(mbn_kernel, grid, dim3(kT), 0, st, a);
  }
  Q35_HIP_TRY(hipGetLastError());
  return Q35_OK;
}

}  // namespace q35
