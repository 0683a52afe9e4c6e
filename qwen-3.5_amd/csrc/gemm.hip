// Q8F GEMM on the fp32 matrix cores, for the prompt (seq_len > 1) projections:
//   Y[m][n] (+)= sum_k X[m][k] * dequant(W)[k][n],  dequant = f32(q) * scale.
// This is the reference's Linear::forward on a QFloat weight (dequantise to f32, f32 matmul;
// text_modules.rs:500-508, :578-595, :638-647, :880-890, :1003-1005) and its lm_head matmul
// (model.rs:130-138, NK layout).  The weights are dequantised to f32 exactly as the reference
// does (one f32 multiply per element) and multiplied with v_mfma_f32_32x32x2_f32, so the
// arithmetic is f32 products with f32 accumulation, like the reference's f32 matmul.
//
// Block = 4 waves in a 2 x 2 grid over a BM x BN output tile; each wave owns (BM/2) x (BN/2),
// i.e. (BM/64) x (BN/64) MFMA tiles of 32 x 32 (16 accumulator registers each).  K advances
// 32 at a time through double-buffered LDS: the X tile [BM][32] and the dequantised W tile
// stored transposed [BN][32] (k contiguous), both with rows padded to 36 floats so that the
// operand reads (16-byte reads of 8 consecutive k by each lane) are free of bank conflicts.
// Within a 32-wide K step the MFMA k index is permuted: step s of half hh gives lane half h
// (lanes 32h..32h+31) k = 16h + 8hh + s, so each lane reads 8 consecutive floats of its row or
// column; the sum over k is unchanged.  The next K step's global loads are issued before the
// current step's MFMAs and written to the other LDS buffer after them: one barrier per step.
//
// Grid: one block per output tile, over up to 4 segments (weight matrices writing disjoint
// column ranges of Y, e.g. in_proj_qkv | in_proj_z), ordered so that the M tiles sharing a
// weight tile are consecutive; the hardware block index is remapped so that consecutive
// logical tiles land on the same XCD (blocks are dispatched round-robin over the 8 XCDs), which
// keeps a weight tile's re-reads inside one L2.
#include "q35_internal.h"

#include <algorithm>

namespace q35 {
namespace {

constexpr int kGT = 256;
constexpr int kBK = 32;
constexpr int kLd = kBK + 4;  // padded LDS row, floats

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

struct GSeg {
  const int8_t* q;
  const float* s;
  float* y;
  int32_t N, layout, ldy, ntiles, tile0, c0;  // c0: first column in the concatenated partials
  const float* smax;  // MB path: the weights' largest |scale| when known (else the prep pass finds it)
};
struct GArgs {
  GSeg seg[kGemmMaxSeg];
  int32_t nseg;
  const float* x;
  int32_t ldx, M, K, mtiles, accumulate, nblocks;
  int32_t ksplit, kchunk, ncat;  // K splits of kchunk rows; partials part[split][M][ncat]
  float* part;
  float* amax;   // MB path: |x| maximum of each row [M]
  int32_t prep_rows;  // MB path: rows whose maximum the prep pass finds (M, or 0 when given)
  float* act;         // MB path: SwiGLU output of alternating gate / up column blocks (else null)
  float* act_amax;
  int32_t ld_act;
  float* spart;  // MB path: partial maxima of every segment's |scale| [kPrepS]
};

// Logical tile of hardware block b: the blocks of one XCD (b % 8) get consecutive logical ids.
Q35_DEV int xcd_remap(int b, int nb) {
  const int q = nb >> 3, r = nb & 7, x = b & 7, i = b >> 3;
  return x < r ? x * (q + 1) + i : r * (q + 1) + (x - r) * q + i;
}

template <int BM, int BN>
__global__ __launch_bounds__(kGT) void gemm_kernel(const GArgs a) {
  constexpr int WM = BM / 2, WN = BN / 2, TM = WM / 32, TN = WN / 32;
  constexpr int AV = BM / 32;  // float4 loads of the X tile per thread
  __shared__ __align__(16) float As[2][BM * kLd];
  __shared__ __align__(16) float Bs[2][BN * kLd];

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int L = xcd_remap((int)blockIdx.x, a.nblocks);
  // logical block = (tile column, K split, M tile), M fastest: the blocks sharing a weight tile
  // are consecutive (one XCD)
  const int gs = L / a.mtiles, mt = L - gs * a.mtiles;
  const int gt = gs / a.ksplit, split = gs - gt * a.ksplit;
  // the segment of tile gt, selected field by field with constant indices (a dynamic index into
  // the kernel-argument array would copy it to private memory)
  GSeg sg = a.seg[0];
#pragma unroll
  for (int i = 1; i < kGemmMaxSeg; ++i)
    if (i < a.nseg && gt >= a.seg[i].tile0) sg = a.seg[i];
  const int n0 = (gt - sg.tile0) * BN, m0 = mt * BM;
  const int K = a.K;
  const int kbeg = split * a.kchunk, kend = min(K, kbeg + a.kchunk);

  // ---- weight tile addressing
  // KN / KN_TILED: thread (r = tid % 32, c16 = tid / 32) loads row k0 + r, columns c16*16..+15.
  // NK: thread (n = tid / 2, hk = tid % 2) loads column n, k0 + 16 hk .. +15.
  const bool nk = sg.layout == Q35_NK;
  const int8_t* qb;
  const float* sb;
  int64_t qrs;  // bytes between consecutive k rows (KN forms)
  int srs;      // scale entries between consecutive k rows (KN forms)
  const int br = tid & 31, bc = tid >> 5;
  const bool bload = nk ? (tid < 2 * BN) : (bc * 16 < BN);
  if (nk) {
    const int n = tid >> 1, hk = tid & 1;
    qb = sg.q + (int64_t)(n0 + min(n, BN - 1)) * K + 16 * hk;
    sb = sg.s + (int64_t)(n0 + min(n, BN - 1)) * (K >> 6);
    qrs = 0;
    srs = 0;
  } else if (sg.layout == Q35_KN_TILED) {
    const int t = n0 >> 8, c0 = n0 & 255;
    qb = sg.q + (int64_t)t * K * 256 + c0 + bc * 16 + (int64_t)br * 256;
    sb = sg.s + (int64_t)t * K * 4 + ((c0 + bc * 16) >> 6) + br * 4;
    qrs = 256;
    srs = 4;
  } else {
    qb = sg.q + n0 + bc * 16 + (int64_t)br * sg.N;
    sb = sg.s + ((n0 + bc * 16) >> 6) + (int64_t)br * (sg.N >> 6);
    qrs = sg.N;
    srs = sg.N >> 6;
  }
  // ---- X tile addressing: thread loads rows tid/8 + 32 i, floats 4*(tid%8)..+3
  const int ar = tid >> 3, ac = (tid & 7) * 4;
  const float* xb = a.x + (int64_t)(m0 + ar) * a.ldx + ac;

  float4 xa[AV];
  uint4 wq = make_uint4(0, 0, 0, 0);
  float ws = 0.f;
  auto gload = [&](int k0) {
#pragma unroll
    for (int i = 0; i < AV; ++i) {
      const bool ok = m0 + ar + 32 * i < a.M;
      xa[i] = ok ? *(const float4*)(xb + (int64_t)32 * i * a.ldx + k0) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    if (bload) {
      if (nk) {
        wq = ldg16(qb + k0);
        ws = ldg(sb + ((k0 + 16 * (tid & 1)) >> 6));
      } else {
        wq = ldg16(qb + (int64_t)k0 * qrs);
        ws = ldg(sb + (int64_t)k0 * srs);
      }
    }
  };
  auto lstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < AV; ++i) *(float4*)&As[buf][(ar + 32 * i) * kLd + ac] = xa[i];
    if (bload) {
      float f[16];
      unpack16(wq, f);
      if (nk) {
        float* d = &Bs[buf][(tid >> 1) * kLd + 16 * (tid & 1)];
#pragma unroll
        for (int j = 0; j < 16; j += 4) *(float4*)(d + j) = make_float4(f[j] * ws, f[j + 1] * ws, f[j + 2] * ws, f[j + 3] * ws);
      } else {
#pragma unroll
        for (int j = 0; j < 16; ++j) Bs[buf][(bc * 16 + j) * kLd + br] = f[j] * ws;
      }
    }
  };

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  const int wm = w >> 1, wn = w & 1;
  const int li = lane & 31, lh = lane >> 5;
  const int nk_steps = (kend - kbeg) / kBK;
  gload(kbeg);
  lstore(0);
  __syncthreads();
  for (int kb = 0; kb < nk_steps; ++kb) {
    const int buf = kb & 1;
    if (kb + 1 < nk_steps) gload(kbeg + (kb + 1) * kBK);
    const float* Ab = &As[buf][0];
    const float* Bb = &Bs[buf][0];
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const int ko = 16 * lh + 8 * hh;
      f32x4 af[TM][2], bf[TN][2];
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const float* p = Ab + (wm * WM + i * 32 + li) * kLd + ko;
        af[i][0] = *(const f32x4*)p;
        af[i][1] = *(const f32x4*)(p + 4);
      }
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const float* p = Bb + (wn * WN + j * 32 + li) * kLd + ko;
        bf[j][0] = *(const f32x4*)p;
        bf[j][1] = *(const f32x4*)(p + 4);
      }
#pragma unroll
      for (int s = 0; s < 8; ++s)
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[i][s >> 2][s & 3], bf[j][s >> 2][s & 3], acc[i][j], 0, 0, 0);
    }
    if (kb + 1 < nk_steps) lstore(buf ^ 1);
    __syncthreads();
  }

  // ---- epilogue: lane (li, lh), register r holds row 8 (r / 4) + 4 lh + r % 4, column li
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int col = n0 + wn * WN + j * 32 + li;
      float* yc = a.ksplit > 1 ? a.part + (int64_t)split * a.M * a.ncat + sg.c0 + col : sg.y + col;
      const int64_t ld = a.ksplit > 1 ? a.ncat : sg.ldy;
      const bool acc_y = a.accumulate && a.ksplit == 1;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = m0 + wm * WM + i * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
        if (row < a.M) {
          float* p = yc + (int64_t)row * ld;
          *p = acc_y ? *p + acc[i][j][r] : acc[i][j][r];
        }
      }
    }
}

// Split-K finish: y (+)= sum over the splits of part[s][m][c], in split order (deterministic);
// one thread per 4 consecutive columns of one row.
__global__ __launch_bounds__(256) void gemm_reduce_kernel(const GArgs a) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int nq = a.ncat >> 2;
  if (i >= (int64_t)a.M * nq) return;
  const int m = (int)(i / nq), c = (int)(i % nq) * 4;
  GSeg sg = a.seg[0];
#pragma unroll
  for (int s = 1; s < kGemmMaxSeg; ++s)
    if (s < a.nseg && c >= a.seg[s].c0) sg = a.seg[s];
  const float* p = a.part + (int64_t)m * a.ncat + c;
  float4 v = *(const float4*)p;
  for (int s = 1; s < a.ksplit; ++s) {
    const float4 u = *(const float4*)(p + (int64_t)s * a.M * a.ncat);
    v.x += u.x; v.y += u.y; v.z += u.z; v.w += u.w;
  }
  float* y = sg.y + (int64_t)m * sg.ldy + (c - sg.c0);
  if (a.accumulate) {
    v.x += y[0]; v.y += y[1]; v.z += y[2]; v.w += y[3];
  }
  y[0] = v.x; y[1] = v.y; y[2] = v.z; y[3] = v.w;
}

// ------------------------------------------------------------------ f16 matrix cores (Q35_KN_MB)
// The same product on v_mfma_f32_16x16x32_f16 with f32-equivalent arithmetic.  The 8-bit weights
// are exact in f16 (read straight from the MB records, the A operands of four MFMAs per lane);
// the scale of a weight's 64-column block varies along k only, so it multiplies x instead:
// y = x * 2^e * scale[cb][k] (f32, 2^e a power of two per row of x), carried as two f16 halves
// hi + lo (~22 significant bits) whose products with q are exact in the f32 accumulator; the tile
// is scaled back by 2^-e.  2^e is fixed for the whole launch from the row's largest |x| and the
// weights' largest |scale|, so every |y| < 2^14 (f16 overflows at 65504).
//
// Block = 4 waves in a 2 x 2 grid over a BM x 128 tile (launched with BM = 64); wave (wm, wn) owns rows wm*BM/2.. of
// column block n0/64 + wn (4 column tiles of 16) and accumulates (BM/32) x 4 tiles of 16 x 16.
// K advances 64 at a time (two MB steps): the next step's x tile (f32, scaled by 2^e while it is
// written to LDS), weights and scales are loaded while the current step's MFMAs run.  Each lane
// forms its own B operands (x row 16 i + c, 8 consecutive k) from LDS and the column block's
// scales in registers.
constexpr int kHBK = 64;          // K per main-loop step (two 32-row MB steps)
constexpr int kXLd = kHBK + 4;    // padded f32 row of the staged x tile (rows 4 banks apart)
constexpr int kPrepS = 64;        // blocks of the scale-maximum pass (one wave's lanes)

typedef float mf4 __attribute__((ext_vector_type(4)));

// Row maxima of |x| (blocks < prep_rows: one row each, every load issued before the first use)
// and, without precomputed ones, partial maxima of every segment's |scale| (the next kPrepS
// blocks, a strided share each).
__global__ __launch_bounds__(256) void hgemm_prep_kernel(const GArgs a) {
  __shared__ float red[4];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  if ((int)blockIdx.x < a.prep_rows) {
    const float* xr = a.x + (int64_t)blockIdx.x * a.ldx;
    float mx = 0.f;
    for (int k0 = 0; k0 < a.K; k0 += 8 * 1024) {
      mf4 v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int k = k0 + 1024 * u + 4 * tid;
        v[u] = k < a.K ? *(const Q35_GLOBAL mf4*)(xr + k) : mf4{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
      for (int u = 0; u < 8; ++u)
        mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v[u][0]), fabsf(v[u][1])), fmaxf(fabsf(v[u][2]), fabsf(v[u][3]))));
    }
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
    if (lane == 0) red[w] = mx;
    __syncthreads();
    if (tid == 0) a.amax[blockIdx.x] = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    return;
  }
  const int p = (int)blockIdx.x - a.prep_rows;
  float mx = 0.f;
#pragma unroll
  for (int i = 0; i < kGemmMaxSeg; ++i) {
    if (i >= a.nseg) break;
    const float* sc = a.seg[i].s;
    const int64_t n = (int64_t)(a.seg[i].N >> 6) * a.K;
    for (int64_t j = (int64_t)p * 256 + tid; j < n; j += (int64_t)kPrepS * 256) mx = fmaxf(mx, fabsf(sc[j]));
  }
  for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
  if (lane == 0) red[w] = mx;
  __syncthreads();
  if (tid == 0) a.spart[p] = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

template <int BM>
__global__ __launch_bounds__(kGT, 2) void hgemm_kernel(const GArgs a) {
  constexpr int WM = BM / 2, MT = WM / 16;  // rows per wave, 16-row tiles per wave
  constexpr int XV = BM / 16;               // x tile float4 per thread (16 threads per 64-float row)
  __shared__ __align__(16) float Xs[2][BM * kXLd];
  __shared__ float fsh[BM];

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 4, c = lane & 15;
  const int L = xcd_remap((int)blockIdx.x, a.nblocks);
  const int gs = L / a.mtiles, mt = L - gs * a.mtiles;
  const int gt = gs / a.ksplit, split = gs - gt * a.ksplit;
  GSeg sg = a.seg[0];
#pragma unroll
  for (int i = 1; i < kGemmMaxSeg; ++i)
    if (i < a.nseg && gt >= a.seg[i].tile0) sg = a.seg[i];
  const int n0 = (gt - sg.tile0) * 128, m0 = mt * BM;
  const int K = a.K, nks = K >> 5;
  const int kbeg = split * a.kchunk, kend = min(K, kbeg + a.kchunk);
  const int wm = w >> 1, wn = w & 1;
  const int cb = (n0 >> 6) + wn;  // the wave's column block within its segment

  // 2^e of each row: (row max |x|) x (max |scale|) x 2^e < 2^14, with room for rounding
  {
    float S = 0.f;
    if (a.seg[0].smax) {  // precomputed for every segment
#pragma unroll
      for (int i = 0; i < kGemmMaxSeg; ++i)
        if (i < a.nseg) S = fmaxf(S, *a.seg[i].smax);
    } else {
      S = a.spart[lane];
      for (int o = 32; o > 0; o >>= 1) S = fmaxf(S, __shfl_xor(S, o));
    }
    if (tid < BM) {
      float f, inv;
      split_scale(a.amax[min(m0 + tid, a.M - 1)] * S * (1.0f + 0x1p-10f), f, inv);
      fsh[tid] = f;
    }
  }
  __syncthreads();

  // x tile: thread loads rows xr0 + 16 i (clamped to M - 1; zeroed when stored), floats xc..xc+3
  const int xr0 = tid >> 4, xc = (tid & 15) * 4;
  float fx[XV];
  const float* xp[XV];
#pragma unroll
  for (int i = 0; i < XV; ++i) {
    const int r = m0 + xr0 + 16 * i;
    fx[i] = r < a.M ? fsh[xr0 + 16 * i] : 0.f;
    xp[i] = a.x + (int64_t)min(r, a.M - 1) * a.ldx + xc;
  }
  mf4 xa[XV];
  auto xload = [&](int k0) {
#pragma unroll
    for (int i = 0; i < XV; ++i) xa[i] = *(const Q35_GLOBAL mf4*)(xp[i] + k0);
  };
  auto xstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < XV; ++i) *(mf4*)&Xs[buf][(xr0 + 16 * i) * kXLd + xc] = xa[i] * fx[i];
  };
  // weights: the lane's 32 bytes of each 32-row MB step of the wave's column block; scales
  // scale[cb][k] of its 8 k
  const int8_t* wq = sg.q + (int64_t)cb * nks * 2048 + lane * 32;
  const float* sc = sg.s + (int64_t)cb * K + 8 * g;
  q35_u32x4 wr[2][2];
  mf4 sr[2][2];
  auto wload = [&](int k0) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int ks = (k0 >> 5) + h;
      wr[h][0] = *(const Q35_GLOBAL q35_u32x4*)(wq + (int64_t)ks * 2048);
      wr[h][1] = *(const Q35_GLOBAL q35_u32x4*)(wq + (int64_t)ks * 2048 + 16);
      sr[h][0] = *(const Q35_GLOBAL mf4*)(sc + 32 * ks);
      sr[h][1] = *(const Q35_GLOBAL mf4*)(sc + 32 * ks + 4);
    }
  };

  mf4 acc[4][MT];
#pragma unroll
  for (int nt = 0; nt < 4; ++nt)
#pragma unroll
    for (int i = 0; i < MT; ++i) acc[nt][i] = mf4{0.f, 0.f, 0.f, 0.f};

  const int nsteps = (kend - kbeg) / kHBK;
  xload(kbeg);
  wload(kbeg);
  xstore(0);
  __syncthreads();
  for (int kb = 0; kb < nsteps; ++kb) {
    const int buf = kb & 1;
    q35_u32x4 wc[2][2];
    mf4 scur[2][2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      wc[h][0] = wr[h][0]; wc[h][1] = wr[h][1];
      scur[h][0] = sr[h][0]; scur[h][1] = sr[h][1];
    }
    if (kb + 1 < nsteps) {
      xload(kbeg + (kb + 1) * kHBK);
      wload(kbeg + (kb + 1) * kHBK);
    }
    const float* Xb = &Xs[buf][0];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const q35_h8 aw[4] = {a8_from(wc[h][0][0], wc[h][0][1]), a8_from(wc[h][0][2], wc[h][0][3]),
                            a8_from(wc[h][1][0], wc[h][1][1]), a8_from(wc[h][1][2], wc[h][1][3])};
      // every LDS read of this half step first, so one wait covers them
      mf4 xv[MT][2];
#pragma unroll
      for (int i = 0; i < MT; ++i) {
        const float* xr = Xb + (wm * WM + 16 * i + c) * kXLd + 32 * h + 8 * g;
        xv[i][0] = *(const mf4*)xr;
        xv[i][1] = *(const mf4*)(xr + 4);
      }
      __builtin_amdgcn_sched_barrier(0);  // (the scheduler would sink each read to its use)
      // the wave issues its MFMAs at raised priority, so that the SIMD's other waves fill the
      // MFMAs' shadow with their vector-ALU work rather than delay them (4-5% on the prompt GEMMs)
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int i = 0; i < MT; ++i) {
        const mf4 x0 = xv[i][0], x1 = xv[i][1];
        uint32_t hi[4], lo[4];
        split2(x0[0] * scur[h][0][0], x0[1] * scur[h][0][1], hi[0], lo[0]);
        split2(x0[2] * scur[h][0][2], x0[3] * scur[h][0][3], hi[1], lo[1]);
        split2(x1[0] * scur[h][1][0], x1[1] * scur[h][1][1], hi[2], lo[2]);
        split2(x1[2] * scur[h][1][2], x1[3] * scur[h][1][3], hi[3], lo[3]);
        const q35_h8 bh = __builtin_bit_cast(q35_h8, q35_u32x4{hi[0], hi[1], hi[2], hi[3]});
        const q35_h8 bl = __builtin_bit_cast(q35_h8, q35_u32x4{lo[0], lo[1], lo[2], lo[3]});
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) acc[nt][i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(aw[nt], bh, acc[nt][i], 0, 0, 0);
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) acc[nt][i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(aw[nt], bl, acc[nt][i], 0, 0, 0);
      }
    }
    __builtin_amdgcn_s_setprio(0);
    if (kb + 1 < nsteps) xstore(buf ^ 1);
    __syncthreads();
  }

  // lane holds D[n = 16 nt + 4 g + r][m = 16 i + c] of the wave's tile: 4 consecutive columns of
  // one row per (nt, i)
  if (a.act) {
    // SwiGLU: the tile's column blocks are gate (wave wn = 0) and up (wn = 1) of the same 64 act
    // columns, at the same lane positions; the up wave hands its values over through LDS (the x
    // staging buffer, idle after the loop's last barrier)
    float* ex = &Xs[0][0] + wm * (MT * 4 * 4 * 64);
    if (wn == 1) {
#pragma unroll
      for (int i = 0; i < MT; ++i) {
        const float inv = __int_as_float((254 << 23) - __float_as_int(fsh[wm * WM + 16 * i + c]));
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) *(mf4*)(ex + ((i * 4 + nt) * 64 + lane) * 4) = acc[nt][i] * inv;
      }
    }
    __syncthreads();
    if (wn == 1) return;
#pragma unroll
    for (int i = 0; i < MT; ++i) {
      const int rl = wm * WM + 16 * i + c, row = m0 + rl;
      const float inv = __int_as_float((254 << 23) - __float_as_int(fsh[rl]));
      float mx = 0.f;
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) {
        const mf4 gt4 = acc[nt][i] * inv, up = *(const mf4*)(ex + ((i * 4 + nt) * 64 + lane) * 4);
        mf4 v;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          v[r] = up[r] * silu_f(gt4[r]);
          mx = fmaxf(mx, fabsf(v[r]));
        }
        if (row < a.M) *(mf4*)(a.act + (int64_t)row * a.ld_act + (n0 >> 1) + 16 * nt + 4 * g) = v;
      }
      mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      if (g == 0 && row < a.M)  // (non-negative floats order as their bit patterns)
        __hip_atomic_fetch_max((Q35_GLOBAL uint32_t*)(a.act_amax + row), __float_as_uint(mx), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < MT; ++i) {
    const int rl = wm * WM + 16 * i + c, row = m0 + rl;
    if (row >= a.M) continue;
    const float inv = __int_as_float((254 << 23) - __float_as_int(fsh[rl]));  // 2^-e, exact
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      const int col = n0 + wn * 64 + 16 * nt + 4 * g;
      mf4 v = acc[nt][i] * inv;
      if (a.ksplit > 1) {
        *(mf4*)(a.part + ((int64_t)split * a.M + row) * a.ncat + sg.c0 + col) = v;
      } else {
        mf4* y = (mf4*)(sg.y + (int64_t)row * sg.ldy + col);
        if (a.accumulate) v += *y;
        *y = v;
      }
    }
  }
}

int g_cus = 0;
int device_cus() {
  if (g_cus > 0) return g_cus;
  int dev = 0, n = 0;
  if (hipGetDevice(&dev) == hipSuccess && hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
    g_cus = n;
  else
    g_cus = 256;
  return g_cus;
}

template <int BM, int BN>
int launch_tile(const GemmCall& c, int ksplit, hipStream_t st) {
  GArgs a{};
  a.nseg = c.nseg;
  a.x = c.x; a.ldx = c.ldx; a.M = c.M; a.K = c.K; a.accumulate = c.accumulate;
  a.mtiles = (c.M + BM - 1) / BM;
  int tiles = 0, ncat = 0;
  for (int i = 0; i < c.nseg; ++i) {
    const GemmSeg& s = c.seg[i];
    a.seg[i] = GSeg{s.q, s.s, s.y, s.N, s.layout, s.ldy, s.N / BN, tiles, ncat};
    tiles += s.N / BN;
    ncat += s.N;
  }
  a.ksplit = ksplit;
  a.kchunk = ((c.K / kBK + ksplit - 1) / ksplit) * kBK;
  a.ncat = ncat;
  a.part = c.part;
  a.nblocks = tiles * ksplit * a.mtiles;
  hipLaunchKernelGGL((gemm_kernel<BM, BN>), dim3(a.nblocks), dim3(kGT), 0, st, a);
  Q35_HIP_TRY(hipGetLastError());
  if (ksplit > 1) {
    const int64_t n = (int64_t)c.M * (ncat / 4);
    hipLaunchKernelGGL(gemm_reduce_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, a);
    Q35_HIP_TRY(hipGetLastError());
  }
  return Q35_OK;
}

template <int BM>
int launch_mb(const GemmCall& c, int ksplit, hipStream_t st) {
  GArgs a{};
  a.nseg = c.nseg;
  a.x = c.x; a.ldx = c.ldx; a.M = c.M; a.K = c.K; a.accumulate = c.accumulate;
  a.mtiles = (c.M + BM - 1) / BM;
  int tiles = 0, ncat = 0;
  for (int i = 0; i < c.nseg; ++i) {
    const GemmSeg& s = c.seg[i];
    a.seg[i] = GSeg{s.q, s.s, s.y, s.N, s.layout, s.ldy, s.N / 128, tiles, ncat, s.smax};
    tiles += s.N / 128;
    ncat += s.N;
  }
  a.ksplit = ksplit;
  a.kchunk = ((c.K / kHBK + ksplit - 1) / ksplit) * kHBK;
  a.ncat = ncat;
  a.part = c.part;
  a.nblocks = tiles * ksplit * a.mtiles;
  a.act = c.act;
  a.act_amax = c.act_amax;
  a.ld_act = c.ld_act;
  a.amax = c.amax ? const_cast<float*>(c.amax) : c.aux;
  a.prep_rows = c.amax ? 0 : c.M;
  a.spart = c.aux + (gemm_aux_floats(c.M) - kPrepS);
  bool smax = true;
  for (int i = 0; i < c.nseg; ++i) smax = smax && c.seg[i].smax;
  if (!smax)
    for (int i = 0; i < c.nseg; ++i) a.seg[i].smax = nullptr;
  const int prep_blocks = a.prep_rows + (smax ? 0 : kPrepS);
  if (prep_blocks > 0) hipLaunchKernelGGL(hgemm_prep_kernel, dim3((unsigned)prep_blocks), dim3(256), 0, st, a);
  hipLaunchKernelGGL((hgemm_kernel<BM>), dim3(a.nblocks), dim3(kGT), 0, st, a);
  Q35_HIP_TRY(hipGetLastError());
  const bool defer = c.defer_reduce && c.nseg == 1;
  if (c.ksplit_out) *c.ksplit_out = defer ? ksplit : 1;  // partial sums the caller must add
  if (ksplit > 1 && !defer) {
    const int64_t n = (int64_t)c.M * (ncat / 4);
    hipLaunchKernelGGL(gemm_reduce_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, a);
    Q35_HIP_TRY(hipGetLastError());
  }
  return Q35_OK;
}

// MB path: 64 x 128 tiles (64-row tiles measured faster than 128-row ones at every prompt shape:
// their 35 KB of LDS lets three or four blocks share a CU, so a launch spreads evenly over the
// CUs) and the K split of least estimated time.  Measured at 512 rows: a block alone on a CU takes
// ~1.09 us per 64-row K step, and a CU holding two or more blocks retires one block-step every
// ~0.91 us; a split adds the reduction kernel (reads every split's partials, writes y: ~4 TB/s,
// plus a launch).
void gemm_pick_mb(const GemmCall& c, int* bm, int* ksplit) {
  int64_t ncat = 0, tiles = 0;
  for (int i = 0; i < c.nseg; ++i) {
    ncat += c.seg[i].N;
    tiles += c.seg[i].N / 128;
  }
  tiles *= (c.M + 63) / 64;
  const int cus = device_cus();
  double best = 1e300;
  *bm = 64;
  *ksplit = 1;
  if (c.act) return;  // (the SwiGLU epilogue needs whole sums)
  for (int ks = 1; ks <= kGemmMaxSplit; ks *= 2) {
    if (ks > 1 && (!c.part || c.part_floats < (size_t)ks * c.M * ncat || c.K / kHBK < 2 * ks)) break;
    const int steps = (c.K / kHBK + ks - 1) / ks;
    const long long per_cu = (tiles * ks + cus - 1) / cus;
    double cost = per_cu <= 1 ? steps * 1.09e-6 : (double)per_cu * steps * 0.91e-6;
    if (ks > 1) cost += (double)c.M * ncat * (ks + 1) * 4.0 / 4e12 + 3e-6;
    if (cost < best * 0.97) { best = cost; *ksplit = ks; }
  }
}

}  // namespace

// Tile shape and K splits: the least estimated time.  A launch takes ceil(blocks / CUs) rounds,
// each the block's MFMA work at the efficiency measured for its tile (128 x 128: 0.70 of peak per
// CU, 64-wide tiles 0.67 / 0.45: they read more LDS operands per MFMA); split K adds a second
// kernel that reads the splits' partials and writes y (~4 TB/s, plus a launch).
int gemm_pick(const GemmCall& c, int* bm, int* bn, int* ksplit) {
  bool n128 = true;
  int64_t ncat = 0;
  for (int i = 0; i < c.nseg; ++i) {
    n128 = n128 && (c.seg[i].N % 128 == 0);
    ncat += c.seg[i].N;
  }
  const int cus = device_cus();
  const double cu_flops = 157.3e12 / 256.0;
  double best = 1e300;
  const int cand[4][2] = {{128, 128}, {64, 128}, {128, 64}, {64, 64}};
  for (const auto& t : cand) {
    if (t[1] == 128 && !n128) continue;
    long long tiles = 0;
    for (int i = 0; i < c.nseg; ++i) tiles += c.seg[i].N / t[1];
    tiles *= (c.M + t[0] - 1) / t[0];
    const double eff = (t[0] == 128 && t[1] == 128) ? 0.70 : (t[0] == 64 && t[1] == 64) ? 0.45 : 0.67;
    for (int ks = 1; ks <= kGemmMaxSplit; ks *= 2) {
      if (ks > 1 && (!c.part || c.part_floats < (size_t)ks * c.M * ncat || c.K / kBK < 2 * ks)) break;
      const int kch = ((c.K / kBK + ks - 1) / ks) * kBK;
      const long long blocks = tiles * ks;
      const double rounds = (double)((blocks + cus - 1) / cus);
      double cost = rounds * 2.0 * t[0] * t[1] * kch / (cu_flops * eff);
      if (ks > 1) cost += (double)c.M * ncat * (ks + 1) * 4.0 / 4e12 + 3e-6;
      if (cost < best * 0.97) { best = cost; *bm = t[0]; *bn = t[1]; *ksplit = ks; }
    }
  }
  return Q35_OK;
}

int gemm_launch(const GemmCall& c, hipStream_t st) {
  if (!c.x || c.nseg < 1 || c.nseg > kGemmMaxSeg) return fail(Q35_E_ARG, "gemm: bad arguments");
  int nmb = 0;
  for (int i = 0; i < c.nseg; ++i) nmb += c.seg[i].layout == Q35_KN_MB;
  if (nmb) {
    if (nmb != c.nseg) return fail(Q35_E_ARG, "gemm: Q35_KN_MB segments cannot be mixed with other layouts");
    if (!c.aux) return fail(Q35_E_WS, "gemm: Q35_KN_MB needs a workspace");
    if (c.M < 1 || c.K < kHBK || (c.K % kHBK) != 0) return fail(Q35_E_SHAPE, "gemm: Q35_KN_MB needs K a multiple of 64");
    if ((c.ldx % 4) != 0 || (reinterpret_cast<uintptr_t>(c.x) & 15) != 0)
      return fail(Q35_E_ALIGN, "gemm: x rows must be 16-byte aligned");
    for (int i = 0; i < c.nseg; ++i) {
      const GemmSeg& s = c.seg[i];
      if (!s.q || !s.s || !s.y) return fail(Q35_E_ARG, "gemm: null segment pointer");
      if (s.N < 128 || (s.N % 128) != 0) return fail(Q35_E_SHAPE, "gemm: Q35_KN_MB needs N a multiple of 128");
      if ((reinterpret_cast<uintptr_t>(s.q) & 15) || (reinterpret_cast<uintptr_t>(s.s) & 15) ||
          (reinterpret_cast<uintptr_t>(s.y) & 15) || (s.ldy % 4))
        return fail(Q35_E_ALIGN, "gemm: Q35_KN_MB needs 16-byte aligned q, scales and y rows");
    }
    if (c.act && (c.nseg != 1 || !c.act_amax || (c.ld_act % 4) != 0 || (reinterpret_cast<uintptr_t>(c.act) & 15)))
      return fail(Q35_E_ARG, "gemm: the SwiGLU output needs one segment, row maxima and 16-byte aligned rows");
    int bm = 64, ks = 1;
    gemm_pick_mb(c, &bm, &ks);
    return launch_mb<64>(c, ks, st);
  }
  if (c.M < 1 || c.K < kBK || (c.K % 64) != 0) return fail(Q35_E_SHAPE, "gemm: M >= 1 and K a multiple of 64 required");
  if ((c.ldx % 4) != 0 || (reinterpret_cast<uintptr_t>(c.x) & 15) != 0)
    return fail(Q35_E_ALIGN, "gemm: x rows must be 16-byte aligned");
  for (int i = 0; i < c.nseg; ++i) {
    const GemmSeg& s = c.seg[i];
    if (!s.q || !s.s || !s.y) return fail(Q35_E_ARG, "gemm: null segment pointer");
    if (s.N < 64 || (s.N % 64) != 0) return fail(Q35_E_SHAPE, "gemm: N must be a multiple of 64");
    if (s.layout != Q35_KN && s.layout != Q35_KN_TILED && s.layout != Q35_NK) return fail(Q35_E_ARG, "gemm: layout");
    if ((reinterpret_cast<uintptr_t>(s.q) & 15) != 0) return fail(Q35_E_ALIGN, "gemm: q not 16-byte aligned");
  }
  int bm = 128, bn = 128, ks = 1;
  gemm_pick(c, &bm, &bn, &ks);
  if (bm == 128 && bn == 128) return launch_tile<128, 128>(c, ks, st);
  if (bm == 64 && bn == 128) return launch_tile<64, 128>(c, ks, st);
  if (bm == 128 && bn == 64) return launch_tile<128, 64>(c, ks, st);
  return launch_tile<64, 64>(c, ks, st);
}

}  // namespace q35
