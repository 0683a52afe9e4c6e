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
};
struct GArgs {
  GSeg seg[kGemmMaxSeg];
  int32_t nseg;
  const float* x;
  int32_t ldx, M, K, mtiles, accumulate, nblocks;
  int32_t ksplit, kchunk, ncat;  // K splits of kchunk rows; partials part[split][M][ncat]
  float* part;
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
