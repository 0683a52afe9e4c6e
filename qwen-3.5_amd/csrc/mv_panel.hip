// Q8F matvec on the panel layout (Q35_KN_PANEL): the reference projection W[K][N] (blocks of 64
// along N, kernels.rs:53-92,103-165) stored as 16-column panels, q[N/16][K][16], with the block
// scales transposed to scale[N/64][K].  One block computes one panel (16 outputs) over all K rows,
// so every output is finished inside its block: no split-K, no cross-block reduction, no atomics,
// no workspace, one launch that writes f32 y directly, and a fixed summation order
// (bit-reproducible).
//
// Memory pattern: lane l of wave w reads row k = tid + T j of the panel (16 bytes), so a wave's
// load instruction covers 64 consecutive rows = 1 KB contiguous of int8 plus 256 contiguous bytes of
// scales; every row of the block is requested before the first is used, so the whole panel is in
// flight at once.  The weights carry the non-temporal hint (read once); the scales do not: the 4
// panels of one 64-column scale block read the same scale row, and the panel order below puts
// those 4 blocks on one XCD (workgroups go to the 8 XCDs round-robin), so 3 of the 4 reads hit
// that XCD's L2.  x[k] is read per row from global memory (small and shared by every panel).
//
// Reduction of a lane's 16 column partials over the wave: two gfx950 lane swaps
// (v_permlane32_swap, v_permlane16_swap) leave each 16-lane row with 4 columns summed over 4 lanes,
// then DPP row rotations sum the 16 lanes of the row — all VALU, no LDS crossbar round trips; the
// waves' results are added through LDS in a fixed order.
#include "q35_internal.h"

namespace q35 {

namespace {

constexpr int kP = 16;  // columns per panel

struct MvpArgs {
  const int8_t* q;  // [N/16][K][16]
  const float* s;   // [N/64][K]
  const float* x;   // [M][ldx]
  float* y;         // [M][ldy]
  int32_t K, N, M, ldx, ldy;
  int32_t remap;    // 1: XCD-aware panel order ((N/16) % 32 == 0)
};

Q35_DEV float swap32_sum(float a, float b) {  // lanes < 32: a(l) + a(l+32); lanes >= 32: b(l-32) + b(l)
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
Q35_DEV float swap16_sum(float a, float b) {  // within each 32-lane half: rows 0 / 2 keep a, 1 / 3 keep b
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
Q35_DEV float row_sum16(float v) {
  v += row_ror<8>(v);
  v += row_ror<4>(v);
  v += row_ror<2>(v);
  v += row_ror<1>(v);
  return v;
}

// Sum of acc[c] over the 64 lanes; on return every lane of 16-lane row r holds columns 4r .. 4r+3
// in o[0..3].
Q35_DEV void fold16(const float (&acc)[kP], float (&o)[4]) {
  float s8[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) s8[j] = swap32_sum(acc[j], acc[j + 8]);  // column j (lanes < 32) or j + 8
#pragma unroll
  for (int j = 0; j < 4; ++j) o[j] = row_sum16(swap16_sum(s8[j], s8[j + 4]));  // column 4r + j
}

// T threads, J rows per thread in flight per pass, MR input rows per launch.  EXACT: K is a
// multiple of T*J, so no row is clamped or masked and no load is skipped; the compiler then knows
// how many loads are outstanding and starts on row j as soon as it lands (with data-dependent
// early exits it waits for every load of the pass first).
template <int T, int MR, int J, bool EXACT>
__global__ __launch_bounds__(T) void mvp_kernel(const MvpArgs a) {
  constexpr int NW = T / 64;
  __shared__ __align__(16) float red[NW][MR][kP];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  int panel = blockIdx.x;
  if (a.remap) {  // panels 4g .. 4g+3 (one scale block) on blocks b with equal b % 8, i.e. one XCD
    const int b = blockIdx.x, xcd = b & 7, slot = b >> 3;
    panel = 4 * ((slot >> 2) * 8 + xcd) + (slot & 3);
  }
  const int K = a.K;
  const int8_t* qp = a.q + (size_t)panel * K * kP;
  const float* sp = a.s + (size_t)(panel >> 2) * K;
  float acc[MR][kP];
#pragma unroll
  for (int m = 0; m < MR; ++m)
#pragma unroll
    for (int c = 0; c < kP; ++c) acc[m][c] = 0.f;

  for (int k0 = 0; k0 < K; k0 += T * J) {
    uint4 w[J];
    float sc[J];
    float xv[MR][J];
    // every load of the pass is issued first (rows clamped into the matrix; masked below)
#pragma unroll
    for (int j = 0; j < J; ++j) {
      if (!EXACT && k0 + T * j >= K) break;  // uniform
      const int k = EXACT ? k0 + tid + T * j : min(k0 + tid + T * j, K - 1);
      w[j] = ldg16_nt(qp + (size_t)k * kP);
      sc[j] = ldg(sp + k);
#pragma unroll
      for (int m = 0; m < MR; ++m) xv[m][j] = ldg(a.x + (size_t)min(m, a.M - 1) * a.ldx + k);
    }
#pragma unroll
    for (int j = 0; j < J; ++j) {
      if (!EXACT && k0 + T * j >= K) break;
      const bool ok = EXACT || k0 + tid + T * j < K;
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
#pragma unroll
  for (int m = 0; m < MR; ++m) {
    float o[4];
    fold16(acc[m], o);
    if ((lane & 15) == 0)
      *reinterpret_cast<float4*>(&red[wid][m][4 * (lane >> 4)]) = make_float4(o[0], o[1], o[2], o[3]);
  }
  __syncthreads();
  if (tid < MR * kP) {
    const int m = tid / kP, c = tid % kP;
    if (m < a.M) {
      float v = 0.f;
#pragma unroll
      for (int w2 = 0; w2 < NW; ++w2) v += red[w2][m][c];
      a.y[(size_t)m * a.ldy + panel * kP + c] = v;
    }
  }
}

template <int T, int MR, int J, bool EXACT>
void launch_one(const MvpArgs& a, hipStream_t st) {
  hipLaunchKernelGGL((mvp_kernel<T, MR, J, EXACT>), dim3(a.N / kP), dim3(T), 0, st, a);
}

// The first J of the list that splits K into exactly as many full passes of T*J rows as the
// generic kernel (J = Jmax, the list's first entry) needs: an exact kernel with no more passes.
// Otherwise the generic kernel.
template <int T, int MR, int Jmax, int J, int... Js>
void launch_pick(const MvpArgs& a, hipStream_t st) {
  const int passes = (a.K + T * Jmax - 1) / (T * Jmax);
  if (a.K % (T * J) == 0 && a.K / (T * J) == passes) launch_one<T, MR, J, true>(a, st);
  else if constexpr (sizeof...(Js) > 0) launch_pick<T, MR, Jmax, Js...>(a, st);
  else launch_one<T, MR, Jmax, false>(a, st);
}
template <int T, int MR, int Jmax, int... Js>
void launch_exact(const MvpArgs& a, hipStream_t st) {
  launch_pick<T, MR, Jmax, Jmax, Js...>(a, st);
}

}  // namespace

int mvp_launch(const int8_t* q, const float* s, int32_t K, int32_t N, const float* x, int32_t ldx, int32_t M,
               float* y, int32_t ldy, hipStream_t st) {
  if (!q || !s || !x || !y) return fail(Q35_E_ARG, "q8_gemv (panel): null pointer");
  if (K < 1 || N < 64 || (N % 64) != 0) return fail(Q35_E_SHAPE, "q8_gemv (panel): N must be a positive multiple of 64");
  if (M < 1 || M > 8) return fail(Q35_E_SHAPE, "q8_gemv (panel): M in [1, 8] per launch");
  if ((reinterpret_cast<uintptr_t>(q) & 15) != 0) return fail(Q35_E_ALIGN, "q8_gemv (panel): q not 16-byte aligned");
  const int npanel = N / kP;
  MvpArgs a{q, s, x, y, K, N, M, ldx, ldy, (npanel % 32) == 0 ? 1 : 0};
  // M = 1: 512 threads, all of K (<= 8192, in one pass) in flight; M > 1: 256-thread blocks (the
  // accumulators take more registers, and two blocks per CU keep every panel of a 6144-wide
  // matrix resident).  The first J of each list that divides K / T gives an exact kernel.
  if (M == 1) launch_exact<512, 1, 16, 12, 8, 6, 4, 3, 2, 1>(a, st);
  else if (M == 2) launch_exact<256, 2, 8, 6, 4, 3, 2, 1>(a, st);
  else if (M <= 4) launch_exact<256, 4, 8, 6, 4, 3, 2, 1>(a, st);
  else launch_exact<256, 8, 4, 3, 2, 1>(a, st);
  Q35_HIP_TRY(hipGetLastError());
  return Q35_OK;
}

}  // namespace q35
