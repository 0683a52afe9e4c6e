// Q8F matvec on the panel layout (Q35_KN_PANEL): the reference projection W[K][N] (blocks of 64
// along N, kernels.rs:53-92,103-165) stored as 16-column panels, q[N/16][K][16], with the block
// scales transposed to scale[N/64][K].  One block computes one panel (16 outputs) over all K rows,
// so every output is finished inside its block: no split-K, no cross-block reduction, no atomics,
// no workspace, one launch that writes f32 y directly, and a fixed summation order
// (bit-reproducible).
//
// Memory pattern: lane l of wave w reads row k = tid + 512 j of the panel (16 bytes), so a wave's
// load instruction covers 64 consecutive rows = 1 KB contiguous of int8 plus 256 contiguous bytes of
// scales; every row of the block is requested before the first is used (all of K for M <= 1 and
// K <= 8192), so the whole panel is in flight at once.  x[k] is read per row from global memory
// (it is small and shared by every panel, so it is served by the caches).  The 16 column partials
// of a lane are folded across the wave with a transposed butterfly, then across the 8 waves
// through LDS.
#include "q35_internal.h"

namespace q35 {

namespace {

constexpr int kT = 512;  // threads per block
constexpr int kNW = kT / 64;
constexpr int kP = 16;   // columns per panel

struct MvpArgs {
  const int8_t* q;  // [N/16][K][16]
  const float* s;   // [N/64][K]
  const float* x;   // [M][ldx]
  float* y;         // [M][ldy]
  int32_t K, N, M, ldx, ldy;
};

// J rows per thread in flight per pass, MR input rows per launch.
template <int MR, int J>
__global__ __launch_bounds__(kT) void mvp_kernel(const MvpArgs a) {
  __shared__ float red[kNW][MR][kP];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int panel = blockIdx.x;
  const int K = a.K;
  const int8_t* qp = a.q + (size_t)panel * K * kP;
  const float* sp = a.s + (size_t)(panel >> 2) * K;
  float acc[MR][kP];
#pragma unroll
  for (int m = 0; m < MR; ++m)
#pragma unroll
    for (int c = 0; c < kP; ++c) acc[m][c] = 0.f;

  for (int k0 = 0; k0 < K; k0 += kT * J) {
    uint4 w[J];
    float sc[J];
    float xv[MR][J];
    // issue every load of the pass first (rows clamped into the matrix; masked below)
#pragma unroll
    for (int j = 0; j < J; ++j) {
      if (k0 + kT * j >= K) break;  // uniform
      const int k = min(k0 + tid + kT * j, K - 1);
      w[j] = ldg16_nt(qp + (size_t)k * kP);
      sc[j] = ldg_nt(sp + k);
#pragma unroll
      for (int m = 0; m < MR; ++m) xv[m][j] = ldg(a.x + (size_t)min(m, a.M - 1) * a.ldx + k);
    }
#pragma unroll
    for (int j = 0; j < J; ++j) {
      if (k0 + kT * j >= K) break;
      const bool ok = k0 + tid + kT * j < K;
      float f[16];
      unpack16(w[j], f);
#pragma unroll
      for (int m = 0; m < MR; ++m) {
        const float cm = ok ? xv[m][j] * sc[j] : 0.f;
#pragma unroll
        for (int c = 0; c < kP; ++c) acc[m][c] += f[c] * cm;
      }
    }
  }
  // wave: each lane ends with the wave's full sum of column lane / 4
#pragma unroll
  for (int m = 0; m < MR; ++m) {
    const float v = fold_rows<kP>(acc[m], lane);
    if ((lane & 3) == 0) red[wid][m][lane >> 2] = v;
  }
  __syncthreads();
  if (tid < MR * kP) {
    const int m = tid / kP, c = tid % kP;
    if (m < a.M) {
      float v = 0.f;
#pragma unroll
      for (int w2 = 0; w2 < kNW; ++w2) v += red[w2][m][c];
      a.y[(size_t)m * a.ldy + panel * kP + c] = v;
    }
  }
}

}  // namespace

int mvp_launch(const int8_t* q, const float* s, int32_t K, int32_t N, const float* x, int32_t ldx, int32_t M,
               float* y, int32_t ldy, hipStream_t st) {
  if (!q || !s || !x || !y) return fail(Q35_E_ARG, "q8_gemv (panel): null pointer");
  if (K < 1 || N < 64 || (N % 64) != 0) return fail(Q35_E_SHAPE, "q8_gemv (panel): N must be a positive multiple of 64");
  if (M < 1 || M > 8) return fail(Q35_E_SHAPE, "q8_gemv (panel): M in [1, 8] per launch");
  if ((reinterpret_cast<uintptr_t>(q) & 15) != 0) return fail(Q35_E_ALIGN, "q8_gemv (panel): q not 16-byte aligned");
  MvpArgs a{q, s, x, y, K, N, M, ldx, ldy};
  const dim3 grid(N / kP), block(kT);
  if (M == 1) hipLaunchKernelGGL((mvp_kernel<1, 16>), grid, block, 0, st, a);
  else if (M == 2) hipLaunchKernelGGL((mvp_kernel<2, 8>), grid, block, 0, st, a);
  else if (M <= 4) hipLaunchKernelGGL((mvp_kernel<4, 4>), grid, block, 0, st, a);
  else hipLaunchKernelGGL((mvp_kernel<8, 4>), grid, block, 0, st, a);
  Q35_HIP_TRY(hipGetLastError());
  return Q35_OK;
}

}  // namespace q35
