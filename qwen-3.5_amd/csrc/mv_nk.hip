// Q8F matvec with rows contiguous along K (NK: W[N][K] int8, scale[N][K/64]) — the tied
// embedding table used as lm_head (kernels.rs:251-291) — plus the greedy argmax
// (kernels.rs:298-371) fused into its epilogue, the standalone argmax and the embedding
// lookup (kernels.rs:15-45).
//
// lm_head decomposition: each wave owns R rows per step; lane l reads the 16-byte chunks
// k = 16*(l + 64c), c < CPW = K/1024, of every row, so a wave reads 1 KB contiguous per row per
// chunk and keeps R*CPW loads (16 for K = 2048) in flight per lane.  x (after the optional final
// RMSNorm) is staged once per block in LDS.  The R row partials of a lane are folded with a
// transposed butterfly (each xor stage exchanges half of the remaining rows, then the lanes
// sharing a row finish the sum): log2(R) + log2(64/R) exchanges for R rows.  Blocks stride over
// row groups.  The argmax keeps the best (value, index) per lane -> wave -> block under the
// reference's order (ArgOrder: larger value, ties by the reference's scan order); the last block
// to finish reduces the block results; the order is total, so the result does not depend on the
// reduction order.
#include "q35_internal.h"
#include <climits>

namespace q35 {

namespace {

constexpr int kThreads = 256;
constexpr int kMaxCpw = 8;        // 16-byte chunks per lane per row: K <= 8192
constexpr int kMaxGrid = 2048;
constexpr size_t kStaticLds = 256;  // the kernel's own shared variables, beside the staged x

// rows per wave per step: 16 loads in flight per lane
template <int CPW> constexpr int kRowsPerWave = CPW >= 8 ? 2 : (CPW >= 4 ? 4 : 8);

struct NkArgs {
  const int8_t* q; const float* s;
  int32_t N, K, M;
  const float* x; const fx_t* xf; int32_t ldx;
  float* y; int32_t ldy;
  int32_t pro; const float* pw; float eps;
  int32_t* argmax_out; int32_t* pos_inc; int32_t* hist;
  float* part_v; int32_t* part_i; uint32_t* counter;
  ArgOrder ord;
};

Q35_DEV float nk_in(const NkArgs& a, int m, int k) {
  const size_t i = (size_t)m * a.ldx + k;
  return a.xf ? from_fx(a.xf[i]) : a.x[i];
}

// best (value, index) over the n published block results, 8 loads in flight per thread.
Q35_DEV void reduce_published(const float* pv, const int32_t* pi, int n, float& v, int& i, const ArgOrder& o) {
  v = -INFINITY;
  i = INT_MAX;
  for (int b0 = threadIdx.x; b0 < n; b0 += 8 * kThreads) {
    float vv[8];
    int ii[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int b = b0 + j * kThreads;
      vv[j] = (b < n) ? ld_agent(&pv[b]) : -INFINITY;
      ii[j] = (b < n) ? ld_agent(&pi[b]) : INT_MAX;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (argmax_better(vv[j], ii[j], v, i, o)) { v = vv[j]; i = ii[j]; }
  }
}

// Block-wide argmax reduction; result valid in all threads.
Q35_DEV void block_argmax(float& v, int& i, float* shv, int* shi, const ArgOrder& o) {
  wave_argmax(v, i, o);
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) { shv[wid] = v; shi[wid] = i; }
  __syncthreads();
  v = shv[0]; i = shi[0];
#pragma unroll
  for (int w = 1; w < 4; ++w)
    if (argmax_better(shv[w], shi[w], v, i, o)) { v = shv[w]; i = shi[w]; }
}

template <int MR, int CPW>
__global__ __launch_bounds__(kThreads) void nk_kernel(const NkArgs a) {
  constexpr int R = kRowsPerWave<CPW>;
  constexpr int kRowsPerBlock = 4 * R;
  extern __shared__ __align__(16) float xs[];  // [MR][K]
  __shared__ float sh[4];
  __shared__ float shv[4];
  __shared__ int shi[4];
  __shared__ int flag;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int K = a.K, nbK = K >> 6;

  // prologue: thread t loads x[t + 256 j] for all j at once (one round trip), normalises, stages
#pragma unroll
  for (int m = 0; m < MR; ++m) {
    if (m >= a.M) break;
    float v[CPW * 4];
#pragma unroll
    for (int j = 0; j < CPW * 4; ++j) {
      const int k = tid + kThreads * j;
      v[j] = (k < K) ? nk_in(a, m, k) : 0.f;
    }
    float r = 1.0f;
    if (a.pro == PRO_RMS) {
      float ss = 0.f;
#pragma unroll
      for (int j = 0; j < CPW * 4; ++j) ss += v[j] * v[j];
      ss = block_sum256(ss, sh);
      r = rsqrt_f(ss / (float)K + a.eps);
    }
#pragma unroll
    for (int j = 0; j < CPW * 4; ++j) {
      const int k = tid + kThreads * j;
      if (k < K) xs[m * K + k] = (a.pro == PRO_RMS) ? (v[j] * r) * (1.0f + a.pw[k]) : v[j];
    }
  }
  __syncthreads();

  float best_v = -INFINITY;
  int best_i = INT_MAX;
  const int nrb = (a.N + kRowsPerBlock - 1) / kRowsPerBlock;
  for (int rb = blockIdx.x; rb < nrb; rb += gridDim.x) {
    const int row0 = rb * kRowsPerBlock + wid * R;
    uint4 wv[R][CPW];
    float sv[R][CPW];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int row = row0 + r;
#pragma unroll
      for (int c = 0; c < CPW; ++c) {
        const int k = 16 * (lane + 64 * c);
        const bool ok = row < a.N && k < K;
        wv[r][c] = ok ? ldg16_nt(a.q + (size_t)row * K + k) : make_uint4(0, 0, 0, 0);
        sv[r][c] = ok ? ldg_nt(a.s + (size_t)row * nbK + (k >> 6)) : 0.f;
      }
    }
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      if (m >= a.M) break;
      float p[R];
#pragma unroll
      for (int r = 0; r < R; ++r) p[r] = 0.f;
#pragma unroll
      for (int c = 0; c < CPW; ++c) {
        const int k = 16 * (lane + 64 * c);
        if (k >= K) continue;
        float xv[16];
        const float4* xp = reinterpret_cast<const float4*>(&xs[m * K + k]);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float4 t = xp[q];
          xv[4 * q] = t.x; xv[4 * q + 1] = t.y; xv[4 * q + 2] = t.z; xv[4 * q + 3] = t.w;
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
          float f[16];
          unpack16(wv[r][c], f);
          float d = 0.f;
#pragma unroll
          for (int j = 0; j < 16; ++j) d += f[j] * xv[j];
          p[r] += d * sv[r][c];
        }
      }
      const float v = fold_rows<R>(p, lane);
      const int row = row0 + lane / (64 / R);
      if ((lane % (64 / R)) == 0 && row < a.N) {
        if (a.y) a.y[(size_t)m * a.ldy + row] = v;
        if (m == 0 && argmax_better(v, row, best_v, best_i, a.ord)) { best_v = v; best_i = row; }
      }
    }
  }

  if (!a.argmax_out) return;
  block_argmax(best_v, best_i, shv, shi, a.ord);
  if (tid == 0) { st_agent(&a.part_v[blockIdx.x], best_v); st_agent(&a.part_i[blockIdx.x], best_i); }
  if (!arrive_last_grid(a.counter, &flag)) return;
  float v;
  int i;
  reduce_published(a.part_v, a.part_i, gridDim.x, v, i, a.ord);
  block_argmax(v, i, shv, shi, a.ord);
  if (tid == 0) {
    const int32_t tok = (i == INT_MAX) ? 0 : i;
    *a.argmax_out = tok;
    if (a.pos_inc) {
      const int32_t p = *a.pos_inc;
      if (a.hist) a.hist[p] = tok;
      *a.pos_inc = p + 1;
    }
  }
}

__global__ __launch_bounds__(kThreads) void argmax_kernel(const float* v, int64_t n, float* part_v, int32_t* part_i,
                                                         uint32_t* counter, int32_t* out, const ArgOrder ord) {
  __shared__ float shv[4];
  __shared__ int shi[4];
  __shared__ int flag;
  const int tid = threadIdx.x;
  float bv = -INFINITY;
  int bi = INT_MAX;
  for (int64_t i = (int64_t)blockIdx.x * kThreads + tid; i < n; i += (int64_t)gridDim.x * kThreads) {
    const float x = v[i];
    if (argmax_better(x, (int)i, bv, bi, ord)) { bv = x; bi = (int)i; }
  }
  block_argmax(bv, bi, shv, shi, ord);
  if (tid == 0) { st_agent(&part_v[blockIdx.x], bv); st_agent(&part_i[blockIdx.x], bi); }
  if (!arrive_last_grid(counter, &flag)) return;
  float rv;
  int ri;
  reduce_published(part_v, part_i, gridDim.x, rv, ri, ord);
  block_argmax(rv, ri, shv, shi, ord);
  if (tid == 0) *out = (ri == INT_MAX) ? 0 : ri;
}

__global__ __launch_bounds__(kThreads) void embed_kernel(const int8_t* q, const float* s, int32_t D, const int32_t* ids,
                                                        int32_t n, float* out) {
  const int64_t total = (int64_t)n * (D / 16);
  for (int64_t e = (int64_t)blockIdx.x * kThreads + threadIdx.x; e < total; e += (int64_t)gridDim.x * kThreads) {
    const int i = (int)(e / (D / 16));
    const int d = (int)(e % (D / 16)) * 16;
    const int64_t id = ids[i];
    const uint4 w = *reinterpret_cast<const uint4*>(q + id * D + d);
    const float sc = s[id * (D / 64) + d / 64];
    float f[16];
    unpack16(w, f);
    float4* o = reinterpret_cast<float4*>(out + (size_t)i * D + d);
#pragma unroll
    for (int j = 0; j < 4; ++j) o[j] = make_float4(f[4 * j] * sc, f[4 * j + 1] * sc, f[4 * j + 2] * sc, f[4 * j + 3] * sc);
  }
}

int cpw_of(int K) {
  const int need = (K + 1023) / 1024;
  return need <= 1 ? 1 : (need <= 2 ? 2 : (need <= 4 ? 4 : 8));
}

int nk_grid(int N, int K) {
  const int rows_per_block = 4 * (cpw_of(K) >= 8 ? 2 : (cpw_of(K) >= 4 ? 4 : 8));
  const int nrb = (N + rows_per_block - 1) / rows_per_block;
  return nrb < kMaxGrid ? nrb : kMaxGrid;
}

// Shared memory one block may use on the current device (160 KB on gfx950), queried once per device.
size_t lds_per_block() {
  static size_t cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 65536;
  if (!cache[dev]) {
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess || v <= 0) v = 65536;
    cache[dev] = (size_t)v;
  }
  return cache[dev];
}

template <int MR, int CPW>
void launch_one(dim3 g, size_t lds, hipStream_t st, const NkArgs& a) {
  if (lds > 65536)  // staging beyond 64 KB of dynamic LDS has to be allowed per kernel
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(nk_kernel<MR, CPW>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  hipLaunchKernelGGL((nk_kernel<MR, CPW>), g, dim3(kThreads), lds, st, a);
}

template <int MR>
void launch_mr(int cpw, dim3 g, size_t lds, hipStream_t st, const NkArgs& a) {
  if (cpw == 1) launch_one<MR, 1>(g, lds, st, a);
  else if (cpw == 2) launch_one<MR, 2>(g, lds, st, a);
  else if (cpw == 4) launch_one<MR, 4>(g, lds, st, a);
  else launch_one<MR, 8>(g, lds, st, a);
}

}  // namespace

int nk_max_rows(int K) {
  int g = 8;
  while (g > 1 && (size_t)g * K * sizeof(float) + kStaticLds > lds_per_block()) g /= 2;
  return g;
}

size_t nk_ws_bytes(const NkCall& c) {
  const size_t g = (size_t)nk_grid(c.N, c.K);
  return kCounterBytes + align256(g * 4) * 2;
}

int nk_launch(const NkCall& c, void* ws, size_t ws_bytes, hipStream_t st) {
  if (!c.q || !c.s || (!c.x && !c.xf)) return fail(Q35_E_ARG, "nk: null pointer");
  if (c.N <= 0 || c.K <= 0 || (c.K % 64) != 0) return fail(Q35_E_SHAPE, "nk: K must be a positive multiple of 64");
  if (c.K > 1024 * kMaxCpw) return fail(Q35_E_SHAPE, "nk: K > 8192");
  if (c.M < 1 || c.M > 8) return fail(Q35_E_SHAPE, "nk: M in [1,8]");
  const int MR = c.M == 1 ? 1 : (c.M == 2 ? 2 : (c.M <= 4 ? 4 : 8));
  if ((size_t)MR * c.K * sizeof(float) + kStaticLds > lds_per_block())
    return fail(Q35_E_SHAPE, "nk: M*K too large for LDS staging");
  if ((reinterpret_cast<uintptr_t>(c.q) & 15) != 0) return fail(Q35_E_ALIGN, "nk: weights not 16-byte aligned");
  if (c.pro == PRO_RMS && !c.pw) return fail(Q35_E_ARG, "nk: RMSNorm needs weight");
  if (c.argmax_out && c.M != 1) return fail(Q35_E_SHAPE, "nk: fused argmax needs M == 1");
  if (!c.y && !c.argmax_out) return fail(Q35_E_ARG, "nk: no output");
  NkArgs a;
  a.q = c.q; a.s = c.s; a.N = c.N; a.K = c.K; a.M = c.M;
  a.x = c.x; a.xf = c.xf; a.ldx = c.ldx; a.y = c.y; a.ldy = c.ldy;
  a.pro = c.pro; a.pw = c.pw; a.eps = c.eps;
  a.argmax_out = c.argmax_out; a.pos_inc = c.pos_inc; a.hist = c.hist;
  a.ord = make_arg_order(c.N);
  const int grid = nk_grid(c.N, c.K);
  a.counter = nullptr; a.part_v = nullptr; a.part_i = nullptr;
  if (c.argmax_out) {
    if (!ws || ws_bytes < nk_ws_bytes(c)) return fail(Q35_E_WS, "nk: workspace too small");
    char* base = ws_scratch(ws);
    const size_t pb = align256((size_t)grid * 4);
    a.counter = ws_counters(ws);
    a.part_v = reinterpret_cast<float*>(base);
    a.part_i = reinterpret_cast<int32_t*>(base + pb);
  }
  const size_t lds = (size_t)MR * c.K * sizeof(float);
  const int cpw = cpw_of(c.K);
  if (MR == 1) launch_mr<1>(cpw, dim3(grid), lds, st, a);
  else if (MR == 2) launch_mr<2>(cpw, dim3(grid), lds, st, a);
  else if (MR == 4) launch_mr<4>(cpw, dim3(grid), lds, st, a);
  else launch_mr<8>(cpw, dim3(grid), lds, st, a);
  Q35_HIP_TRY(hipGetLastError());
  return Q35_OK;
}

size_t argmax_ws_bytes(int64_t n) {
  (void)n;
  return kCounterBytes + 2 * 1024 * 4;
}

int argmax_launch(const float* v, int64_t n, int32_t* out, void* ws, size_t ws_bytes, hipStream_t st) {
  if (!v || !out) return fail(Q35_E_ARG, "argmax: null pointer");
  if (n <= 0 || n > INT_MAX) return fail(Q35_E_SHAPE, "argmax: n out of range");
  if (!ws || ws_bytes < argmax_ws_bytes(n)) return fail(Q35_E_WS, "argmax: workspace too small");
  int64_t g = (n + kThreads * 8 - 1) / (kThreads * 8);
  if (g > 1024) g = 1024;
  if (g < 1) g = 1;
  char* base = ws_scratch(ws);
  hipLaunchKernelGGL(argmax_kernel, dim3((unsigned)g), dim3(kThreads), 0, st, v, n,
                     reinterpret_cast<float*>(base), reinterpret_cast<int32_t*>(base + 4096),
                     ws_counters(ws), out, make_arg_order(n));
  Q35_HIP_TRY(hipGetLastError());
  return Q35_OK;
}

int embed_launch(const int8_t* q, const float* s, int32_t V, int32_t D, const int32_t* ids, int32_t n,
                 float* out, hipStream_t st) {
  (void)V;
  if (!q || !s || !ids || !out) return fail(Q35_E_ARG, "embedding: null pointer");
  if (D <= 0 || (D % 64) != 0 || n < 0) return fail(Q35_E_SHAPE, "embedding: D must be a multiple of 64");
  if (n == 0) return Q35_OK;
  const int64_t total = (int64_t)n * (D / 16);
  int64_t g = (total + kThreads - 1) / kThreads;
  if (g > 4096) g = 4096;
  hipLaunchKernelGGL(embed_kernel, dim3((unsigned)g), dim3(kThreads), 0, st, q, s, D, ids, n, out);
  Q35_HIP_TRY(hipGetLastError());
  return Q35_OK;
}

}  // namespace q35
