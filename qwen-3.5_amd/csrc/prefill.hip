// Prompt (seq_len > 1) kernels besides the GEMM: row RMSNorm, the Gated DeltaNet prompt path
// (causal conv over the prompt continuing the cached state, then the chunked gated delta rule
// in two launches), gated RMSNorm, SwiGLU, and the attention prompt path (q/k norms, RoPE and
// KV append, then causal attention over the cache).
//
// Chunked gated delta rule (burn_chunk_gated_delta_rule, text_modules.rs:189-363; chunk 64,
// :640).  Everything that does not involve the recurrent state is independent per chunk, so
// the first launch (gdn_chunk_prep) runs one block per (chunk, head) in parallel: conv + SiLU of
// the head's q/k/v channels (:164-182 with the cached state prepended, :531-554), l2norm and
// the 128^-1/2 query scale (:219-223), cumulative decay, the strictly lower system
// -(k_beta k^T) * exp(cum_i - cum_j) and its forward substitution (:282-296), then
// new_values = U (v beta), k_cumdecay = U (k beta e^cum), the intra-chunk attention
// (q k^T) * exp(cum_i - cum_j) (j <= i), q e^cum, k e^(cum_last - cum) and e^cum_last; all go to
// a scratch buffer.  The second launch (gdn_chunk_state) walks the chunks in order (:313-349):
// the state's value columns are independent, so one block per (head, 16-column slice) keeps its
// S[:, slice] in LDS and per chunk forms v_new = new_values - k_cumdecay S, the output
// q_e S + intra v_new, and S = S e^cum_last + k_d^T v_new.
#include "q35_internal.h"

#include <cmath>

namespace q35 {
namespace {

constexpr int kPT = 256;
constexpr int kC = kGdnChunk;     // 64
constexpr int kDk = 128;          // key and value head dim
constexpr int kLdq = kDk + 4;     // padded LDS row (floats)
constexpr int kSl = 16;           // value columns per state-pass block
constexpr int kNsl = kDk / kSl;   // 8 slices per head
// scratch per (head, chunk)
constexpr int kScrNv = 0, kScrKcd = kC * kDk, kScrQe = 2 * kC * kDk, kScrKd = 3 * kC * kDk;
constexpr int kScrIntra = 4 * kC * kDk, kScrCd = kScrIntra + kC * kC;
static_assert(kScrCd + 64 == kGdnScratchPerChunk, "scratch layout");
// Element order of the scratch matrices: the state pass reads them as MFMA operands, each lane
// l = 16 g + c16 of a wave taking 4 consecutive k as one float4, so they are stored lane-major
// (every load of a wave is 1 KB contiguous).  k_cumdecay and q_e [row i][key e]: wave tile (i/16,
// e/64), step (e/16) % 4, lane (g = (e/4) % 4, c16 = i % 16), k = e % 4.  k_d [row l][key e], read
// as k_d^T: wave e/16, step l/16, lane (g = (l/4) % 4, c16 = e % 16), k = l % 4.  intra [i][j]:
// tile i/16, step j/16, lane (g = (j/4) % 4, c16 = i % 16), k = j % 4.  New values [i][column d]
// (an output-tile operand): slice d/16, tile i/16, lane (g = (i/4) % 4, c16 = d % 16), r = i % 4.
Q35_DEV int scr_a(int i, int e) {
  return ((((i >> 4) * 2 + (e >> 6)) * 4 + ((e >> 4) & 3)) * 64 + ((e >> 2) & 3) * 16 + (i & 15)) * 4 + (e & 3);
}
Q35_DEV int scr_kd(int l, int e) { return (((e >> 4) * 4 + (l >> 4)) * 64 + ((l >> 2) & 3) * 16 + (e & 15)) * 4 + (l & 3); }
Q35_DEV int scr_in(int i, int j) { return (((i >> 4) * 4 + (j >> 4)) * 64 + ((j >> 2) & 3) * 16 + (i & 15)) * 4 + (j & 3); }
Q35_DEV int scr_nv(int i, int d) { return (((d >> 4) * 4 + (i >> 4)) * 64 + ((i >> 2) & 3) * 16 + (d & 15)) * 4 + (i & 3); }

// Largest value over a 256-thread block (every thread passes one); thread 0 stores it.
Q35_DEV void block_max256_store(float v, float* sh, float* dst) {
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
  __syncthreads();
  if (threadIdx.x == 0) *dst = fmaxf(fmaxf(sh[0], sh[1]), fmaxf(sh[2], sh[3]));
}

// y[m] = x[m] * rsqrt(mean(x[m]^2) + eps) * (1 + w)  (text_modules.rs:800-808).  amax (optional):
// max |y[m]| of each row, the row maxima the matrix-core GEMM that consumes y needs.  With nsplit >
// 1, x[m] is first replaced by ((part_0 + part_1) + ...) + x[m], the K splits of the GEMM that
// accumulates into x added in split order as its reduction kernel would.  clear (optional): set to
// zero per row (the next GEMM's SwiGLU row maxima, raised by atomics).  Rows of up to
// kRmsHeld * 4 * 256 floats (K a multiple of 4, rows 16-byte aligned) stay in registers between
// the sum of squares and the scaling (one read of x); longer ones are read twice.
constexpr int kRmsHeld = 4;  // float4 per thread held
__global__ __launch_bounds__(kPT) void rms_rows_kernel(float* x, int ldx, int K, const float* w, float eps,
                                                       float* y, int ldy, float* amax, const float* part,
                                                       int nsplit, int64_t sstride, int ldp, float* clear) {
  __shared__ float sh[4];
  const int m = blockIdx.x;
  if (clear && threadIdx.x == 0) clear[m] = 0.f;
  float* xr = x + (int64_t)m * ldx;
  float* yr = y + (int64_t)m * ldy;
  const float* pr = part ? part + (int64_t)m * ldp : nullptr;
  float mx = 0.f;
  if (K <= kRmsHeld * 4 * kPT && (K & 3) == 0 &&
      ((reinterpret_cast<uintptr_t>(xr) | reinterpret_cast<uintptr_t>(yr) | reinterpret_cast<uintptr_t>(w) |
        reinterpret_cast<uintptr_t>(pr)) & 15) == 0 && (nsplit <= 1 || (sstride & 3) == 0)) {
    float4 v[kRmsHeld];
    float ss = 0.f;
#pragma unroll
    for (int u = 0; u < kRmsHeld; ++u) {
      const int k = 4 * (threadIdx.x + u * kPT);
      v[u] = k < K ? *(const float4*)(xr + k) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    if (nsplit > 1) {
#pragma unroll
      for (int u = 0; u < kRmsHeld; ++u) {
        const int k = 4 * (threadIdx.x + u * kPT);
        if (k < K) {
          float4 t = *(const float4*)(pr + k);
          for (int s = 1; s < nsplit; ++s) {
            const float4 q = *(const float4*)(pr + s * sstride + k);
            t.x += q.x; t.y += q.y; t.z += q.z; t.w += q.w;
          }
          v[u] = make_float4(t.x + v[u].x, t.y + v[u].y, t.z + v[u].z, t.w + v[u].w);
          *(float4*)(xr + k) = v[u];
        }
      }
    }
#pragma unroll
    for (int u = 0; u < kRmsHeld; ++u) ss += ((v[u].x * v[u].x + v[u].y * v[u].y) + v[u].z * v[u].z) + v[u].w * v[u].w;
    ss = block_sum256(ss, sh);
    const float r = rsqrt_f(ss * rcp_f((float)K) + eps);
#pragma unroll
    for (int u = 0; u < kRmsHeld; ++u) {
      const int k = 4 * (threadIdx.x + u * kPT);
      if (k < K) {
        const float4 wv = *(const float4*)(w + k);
        const float4 o = make_float4((v[u].x * r) * (1.0f + wv.x), (v[u].y * r) * (1.0f + wv.y),
                                     (v[u].z * r) * (1.0f + wv.z), (v[u].w * r) * (1.0f + wv.w));
        *(float4*)(yr + k) = o;
        mx = fmaxf(mx, fmaxf(fmaxf(fabsf(o.x), fabsf(o.y)), fmaxf(fabsf(o.z), fabsf(o.w))));
      }
    }
  } else {
    float ss = 0.f;
    for (int k = threadIdx.x; k < K; k += kPT) {
      float v = xr[k];
      if (nsplit > 1) {
        float t = pr[k];
        for (int s = 1; s < nsplit; ++s) t += pr[s * sstride + k];
        v = t + v;
        xr[k] = v;
      }
      ss += v * v;
    }
    ss = block_sum256(ss, sh);
    const float r = rsqrt_f(ss * rcp_f((float)K) + eps);
    for (int k = threadIdx.x; k < K; k += kPT) {
      const float v = (xr[k] * r) * (1.0f + w[k]);
      yr[k] = v;
      mx = fmaxf(mx, fabsf(v));
    }
  }
  if (amax) block_max256_store(mx, sh, amax + m);
}

// ------------------------------------------------------------------ Gated DeltaNet, prompt
// [beta | g] of 4 prompt rows per block (text_modules.rs:578-595).  Four groups of 256 threads
// take the 512-column chunks of K in turn (all four chunks of a 2048-wide row in one round trip).
// In a group, thread (output o = tid % 32, K group kg = tid / 32) loads one weight W[k][o] per k
// of its group and multiplies it with the block's rows' x[t][k] (LDS), keeping a sum per row; the groups'
// and K groups' sums are then added in LDS in a fixed order.  Softplus takes its identity branch
// when its input exceeds 20 (the prompt branch's rule).
constexpr int kGateRows = 4, kGateK = 512, kGateGroups = kPT / 32, kGateCG = 4, kGateT = kGateCG * kPT;
__global__ __launch_bounds__(kGateT) void gate_prompt_kernel(const float* x, int ldx, int T, int K, const float* wb,
                                                             const float* wa, const float* alog, const float* dtb,
                                                             int nh, float* out) {
  __shared__ float xs[kGateCG][kGateRows][kGateK + 4];
  __shared__ float red[kGateCG][kGateGroups][kGateRows][33];
  const int cg = threadIdx.x / kPT, tid = threadIdx.x % kPT, o = tid & 31, kg = tid >> 5;
  const int t0 = blockIdx.x * kGateRows;
  const int nout = 2 * nh, oo = min(o, nout - 1), h = oo % nh;
  const float* W = (oo < nh ? wb : wa) + h;
  float acc[kGateRows];
#pragma unroll
  for (int r = 0; r < kGateRows; ++r) acc[r] = 0.f;
  constexpr int kIt = kGateK / (8 * kGateGroups);
  for (int kb = 0; kb < K; kb += kGateCG * kGateK) {  // (the same trip count in every group)
    const int k0 = kb + cg * kGateK;
    const int kn = max(0, min(kGateK, K - k0));  // a multiple of 64; 0 past the end
    __syncthreads();
    // all of the chunk's loads are issued before any is used (one round trip): the x rows, and
    // the weights of the thread's 8-row groups kb = 8 kg + 64 it (rows clamped inside the chunk)
    constexpr int kL = kGateRows * kGateK / 4 / kPT;  // float4 per thread (8)
    float4 v[kL];
#pragma unroll
    for (int u = 0; u < kL; ++u) {
      const int e = tid + u * kPT, i = e / (kGateK / 4), kk = (e % (kGateK / 4)) * 4, t = t0 + i;
      v[u] = (t < T && kk < kn) ? *(const float4*)(x + (int64_t)t * ldx + k0 + kk) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    float w[kIt][8];
#pragma unroll
    for (int it = 0; it < kIt; ++it)
#pragma unroll
      for (int u = 0; u < 8; ++u) w[it][u] = kn > 0 ? W[(int64_t)(k0 + min(kg * 8 + 64 * it, kn - 8) + u) * nh] : 0.f;
#pragma unroll
    for (int u = 0; u < kL; ++u) {
      const int e = tid + u * kPT, i = e / (kGateK / 4), kk = (e % (kGateK / 4)) * 4;
      xs[cg][i][kk] = v[u].x; xs[cg][i][kk + 1] = v[u].y; xs[cg][i][kk + 2] = v[u].z; xs[cg][i][kk + 3] = v[u].w;
    }
    __syncthreads();
#pragma unroll
    for (int it = 0; it < kIt; ++it) {
      const int kq = kg * 8 + 64 * it;
      if (kq < kn) {
#pragma unroll
        for (int u = 0; u < 8; ++u)
#pragma unroll
          for (int r = 0; r < kGateRows; ++r) acc[r] += xs[cg][r][kq + u] * w[it][u];
      }
    }
  }
#pragma unroll
  for (int r = 0; r < kGateRows; ++r) red[cg][kg][r][o] = acc[r];
  __syncthreads();
  for (int e = threadIdx.x; e < kGateRows * 32; e += kGateT) {
    const int r = e >> 5, oc = e & 31, t = t0 + r;
    if (t >= T || oc >= nout) continue;
    float sv = 0.f;
#pragma unroll
    for (int c = 0; c < kGateCG; ++c)
#pragma unroll
      for (int g = 0; g < kGateGroups; ++g) sv += red[c][g][r][oc];
    float res;
    if (oc < nh) {
      res = sigmoid_f(sv);
    } else {
      const int hh = oc - nh;
      const float xg = sv + dtb[hh];
      res = -expf(alog[hh]) * (xg > 20.0f ? xg : logf(expf(xg) + 1.0f));
    }
    out[(int64_t)t * nout + oc] = res;
  }
}

typedef float mfma_f4 __attribute__((ext_vector_type(4)));

// 16 x 16 tile product on the f32 matrix cores: acc += A B over 16 k, A(i, k) and B(k, j) read by
// the callers' accessors; lane l = 16 g + c16 feeds k = 4 g + m to step m and holds
// D[4 g + r][c16] (register r).
template <typename FA, typename FB>
Q35_DEV mfma_f4 tile_mm16(FA A, FB B, mfma_f4 acc) {
  const int c16 = threadIdx.x & 15, g = (threadIdx.x >> 4) & 3;
#pragma unroll
  for (int m = 0; m < 4; ++m) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(A(c16, 4 * g + m), B(4 * g + m, c16), acc, 0, 0, 0);
  return acc;
}

// X = (I - N)^-1 for N strictly lower 64 x 64 in U (in place: U ends as X minus its unit
// diagonal; zero above it), by blocks on the f32 matrix cores (the reference's row recurrence,
// text_modules.rs:282-290, solves the same system): waves 0-3 each invert a 16 x 16 diagonal block
// as (I + N)(I + N^2)(I + N^4)(I + N^8) (N^16 = 0 for a strictly lower 16 x 16 block), then
// X_BA = X_BB N_BA X_AA joins 16-blocks into 32-blocks and those into the 64-block
// (for [[I - N_AA, 0], [-N_BA, I - N_BB]]).  Tm: 64 x 65 scratch.
Q35_DEV void tri_inverse(float (*U)[kC + 1], float (*Tm)[kC + 1]) {
  const int tid = threadIdx.x, wid = tid >> 6, c16 = tid & 15, g = (tid >> 4) & 3;
  const mfma_f4 z = {0.f, 0.f, 0.f, 0.f};
  auto put = [&](float (*D)[kC + 1], int r0, int c0, mfma_f4 v) {
#pragma unroll
    for (int r = 0; r < 4; ++r) D[r0 + 4 * g + r][c0 + c16] = v[r];
  };
  if (wid < 4) {  // diagonal block b0; scratch: Tm rows b0 .. b0 + 15 (blocks 0..3 of columns)
    const int b0 = 16 * wid;
    auto N = [&](int i, int k) { return U[b0 + i][b0 + k]; };
    auto S = [&](int q) { return [=](int i, int k) { return Tm[b0 + i][16 * q + k]; }; };
    put(Tm, b0, 16, tile_mm16(N, N, z));              // N^2
    put(Tm, b0, 32, tile_mm16(S(1), S(1), z));        // N^4
    put(Tm, b0, 48, tile_mm16(S(2), S(2), z));        // N^8
    {  // X1 = N + N^2 + N N^2  (= (I + N)(I + N^2) - I)
      const mfma_f4 p = tile_mm16(N, S(1), z);
      mfma_f4 v;
#pragma unroll
      for (int r = 0; r < 4; ++r) v[r] = (N(4 * g + r, c16) + Tm[b0 + 4 * g + r][16 + c16]) + p[r];
      put(Tm, b0, 0, v);
    }
    {  // X2 = X1 + N^4 + X1 N^4
      const mfma_f4 p = tile_mm16(S(0), S(2), z);
      mfma_f4 v;
#pragma unroll
      for (int r = 0; r < 4; ++r) v[r] = (Tm[b0 + 4 * g + r][c16] + Tm[b0 + 4 * g + r][32 + c16]) + p[r];
      put(Tm, b0, 16, v);
    }
    {  // X3 = X2 + N^8 + X2 N^8
      const mfma_f4 p = tile_mm16(S(1), S(3), z);
      mfma_f4 v;
#pragma unroll
      for (int r = 0; r < 4; ++r) v[r] = (Tm[b0 + 4 * g + r][16 + c16] + Tm[b0 + 4 * g + r][48 + c16]) + p[r];
      put(U, b0, b0, v);
    }
  }
  __syncthreads();
  // 16 -> 32: blocks (1,0) and (3,2) of 16, a wave each: Tm_BA = N_BA (I + L_A), X_BA = (I + L_B) Tm_BA
  if (wid < 2) {
    const int ra = 32 * wid, rb = ra + 16;
    auto NBA = [&](int i, int k) { return U[rb + i][ra + k]; };
    auto IA = [&](int k, int j) { return U[ra + k][ra + j] + (k == j ? 1.0f : 0.0f); };
    put(Tm, rb, ra, tile_mm16(NBA, IA, z));
    auto IB = [&](int i, int k) { return U[rb + i][rb + k] + (i == k ? 1.0f : 0.0f); };
    auto T = [&](int k, int j) { return Tm[rb + k][ra + j]; };
    put(U, rb, ra, tile_mm16(IB, T, z));
  }
  __syncthreads();
  // 32 -> 64: block (1,0) of 32, a wave per 16 x 16 output tile (rt, ct)
  if (wid < 4) {
    const int rt = wid >> 1, ct = wid & 1;
    mfma_f4 acc = z;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      auto A = [&](int i, int k) { return U[32 + 16 * rt + i][16 * kb + k]; };
      auto B = [&](int k, int j) { return U[16 * kb + k][16 * ct + j] + (16 * kb + k == 16 * ct + j ? 1.0f : 0.0f); };
      acc = tile_mm16(A, B, acc);
    }
    put(Tm, 32 + 16 * rt, 16 * ct, acc);
  }
  __syncthreads();
  if (wid < 4) {
    const int rt = wid >> 1, ct = wid & 1;
    mfma_f4 acc = z;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      auto A = [&](int i, int k) { return U[32 + 16 * rt + i][32 + 16 * kb + k] + (16 * rt + i == 16 * kb + k ? 1.0f : 0.0f); };
      auto B = [&](int k, int j) { return Tm[32 + 16 * kb + k][16 * ct + j]; };
      acc = tile_mm16(A, B, acc);
    }
    put(U, 32 + 16 * rt, 16 * ct, acc);
  }
  __syncthreads();
}

constexpr int kPP = 512;  // threads of the prep pass
__global__ __launch_bounds__(kPP) void gdn_chunk_prep_kernel(const GdnPrefill a) {
  __shared__ __align__(16) float Qs[kC][kLdq];
  __shared__ __align__(16) float Ks[kC][kLdq];
  __shared__ __align__(16) float Vs[kC][kLdq];
  __shared__ float U[kC][kC + 1];
  __shared__ float Tm[kC][kC + 1];
  __shared__ float cum[kC], bet[kC], ecum[kC];

  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int c = blockIdx.x % a.nchunk, h = blockIdx.x / a.nchunk;
  const int t0 = c * kC;
  float* scr = a.scr + ((int64_t)h * a.nchunk + c) * kGdnScratchPerChunk;

  // causal conv (cached state prepended) + SiLU: one channel of the head's 3 x 128 per thread
  // pass, a sliding window of the last three inputs in registers
  for (int jj = tid; jj < 3 * kDk; jj += kPP) {
    const int part = jj >> 7, cc = jj & 127;
    const int ch = part == 0 ? h * kDk + cc : (part == 1 ? a.key_dim + h * kDk + cc : 2 * a.key_dim + h * kDk + cc);
    float (*dst)[kLdq] = part == 0 ? Qs : (part == 1 ? Ks : Vs);
    const float* wp = a.conv_w + (int64_t)ch * 4;
    const float w0 = wp[0], w1 = wp[1], w2 = wp[2], w3 = wp[3];
    float x0, x1, x2;
    {
      float xw[3];
#pragma unroll
      for (int u = 0; u < 3; ++u) {
        const int tt = t0 - 3 + u;
        xw[u] = tt >= 0 ? a.raw[(int64_t)tt * a.ld_raw + ch] : a.conv_state[(int64_t)ch * 3 + 3 + tt];
      }
      x0 = xw[0]; x1 = xw[1]; x2 = xw[2];
    }
    // all of the chunk's inputs of the channel in flight at once (rows clamped, masked below)
    float xv[kC];
#pragma unroll
    for (int u = 0; u < kC; ++u) xv[u] = a.raw[(int64_t)min(t0 + u, a.T - 1) * a.ld_raw + ch];
#pragma unroll
    for (int u = 0; u < kC; ++u) {
      const int t = t0 + u;
      const float xin = t < a.T ? xv[u] : 0.f;
      const float y = ((w0 * x0 + w1 * x1) + w2 * x2) + w3 * xin;
      dst[u][cc] = t < a.T ? silu_f(y) : 0.f;
      x0 = x1; x1 = x2; x2 = xin;
    }
  }
  if (tid < kC) {
    const int t = t0 + tid;
    bet[tid] = t < a.T ? a.bg[(int64_t)t * a.ld_bg + h] : 0.f;
    cum[tid] = t < a.T ? a.bg[(int64_t)t * a.ld_bg + a.nh + h] : 0.f;  // g for now
  }
  for (int e = tid; e < kC * kC; e += kPP) U[e >> 6][e & 63] = 0.f;
  __syncthreads();
  // l2norm of q (times dk^-1/2) and k rows
  for (int r = wid; r < 2 * kC; r += kPP / 64) {
    float* row = r < kC ? Qs[r] : Ks[r - kC];
    const float v0 = row[lane], v1 = row[lane + 64];
    const float rn = rsqrt_f(wave_sum(v0 * v0 + v1 * v1) + 1e-6f);
    const float f = r < kC ? a.qscale : 1.0f;
    row[lane] = (v0 * rn) * f;
    row[lane + 64] = (v1 * rn) * f;
  }
  if (wid == 0) {  // cumulative decay inside the chunk (padded steps add 0): a wave scan
    float v = cum[lane];
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const float o = __shfl_up(v, off, 64);
      if (lane >= off) v += o;
    }
    cum[lane] = v;
    ecum[lane] = expf(v);
  }
  __syncthreads();
  // N = -(beta_i k_i.k_j) e^(cum_i - cum_j) for j < i; intra = (q_i.k_j) e^(cum_i - cum_j) for j <= i:
  // the 10 16 x 16 tiles on and below the diagonal of K K^T and Q K^T on the f32 matrix cores (a
  // wave per tile; lane l = 16 g + c16 feeds keys 16 kk + 4 g + m to step m of both operands), the 6
  // tiles above it zero
  float* intra = scr + kScrIntra;
  {
    const int g = lane >> 4, c16 = lane & 15;
    for (int e = tid; e < 6 * 64; e += kPP) {
      const int t = e >> 6, ti = t < 3 ? 0 : (t < 5 ? 1 : 2), tj = t < 3 ? t + 1 : (t < 5 ? t - 1 : 3);
      *(float4*)(intra + ((ti * 4 + tj) * 64 + (e & 63)) * 4) = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    for (int tt = wid; tt < 10; tt += kPP / 64) {
      const int ti = tt >= 6 ? 3 : (tt >= 3 ? 2 : (tt >= 1 ? 1 : 0)), tj = tt - ti * (ti + 1) / 2;
      mfma_f4 gk = {0.f, 0.f, 0.f, 0.f}, gq = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < kDk / 16; ++kk) {
        const int e0 = 16 * kk + 4 * g;
        const mfma_f4 ka = *(const mfma_f4*)&Ks[16 * ti + c16][e0];
        const mfma_f4 qa = *(const mfma_f4*)&Qs[16 * ti + c16][e0];
        const mfma_f4 kb = *(const mfma_f4*)&Ks[16 * tj + c16][e0];
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          gk = __builtin_amdgcn_mfma_f32_16x16x4f32(ka[m], kb[m], gk, 0, 0, 0);
          gq = __builtin_amdgcn_mfma_f32_16x16x4f32(qa[m], kb[m], gq, 0, 0, 0);
        }
      }
      const int jj = 16 * tj + c16;  // the lane's column; rows 16 ti + 4 g + r
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int ii = 16 * ti + 4 * g + r;
        const float dec = jj <= ii ? expf(cum[ii] - cum[jj]) : 0.f;
        if (jj < ii) U[ii][jj] = -((bet[ii] * gk[r]) * dec);
        intra[scr_in(ii, jj)] = jj <= ii ? gq[r] * dec : 0.f;
      }
    }
  }
  // k_d = k e^(cum_last - cum): 4 chunk rows of one key per float4 of its lane-major layout
  for (int e = tid; e < kC * kDk / 4; e += kPP) {
    const int w = e >> 8, lb = (e >> 6) & 3, ln = e & 63, g = ln >> 4, c16 = ln & 15;
    const int l = 16 * lb + 4 * g, k = 16 * w + c16;
    float kv[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) kv[m] = Ks[l + m][k] * expf(cum[kC - 1] - cum[l + m]);
    *(float4*)(scr + kScrKd + scr_kd(l, k)) = make_float4(kv[0], kv[1], kv[2], kv[3]);
  }
  __syncthreads();
  tri_inverse(U, Tm);
  // new_values = (I + X) (beta v), k_cumdecay = (I + X) (beta e^cum k) on the f32 matrix cores (X:
  // the strictly lower inverse in U, zero elsewhere): wave = 16 value / key columns, the four row
  // tiles over the column blocks up to the diagonal
  {
    const int g = lane >> 4, c16 = lane & 15, dcol = 16 * wid + c16;
#pragma unroll
    for (int ti = 0; ti < 4; ++ti) {
      mfma_f4 an = {0.f, 0.f, 0.f, 0.f}, ak = {0.f, 0.f, 0.f, 0.f};
      const int il = 16 * ti + c16;
      for (int lb = 0; lb <= ti; ++lb) {
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          const int ll = 16 * lb + 4 * g + m;
          const float av = U[il][ll] + (ll == il ? 1.0f : 0.0f);
          const float b = bet[ll];
          an = __builtin_amdgcn_mfma_f32_16x16x4f32(av, b * Vs[ll][dcol], an, 0, 0, 0);
          ak = __builtin_amdgcn_mfma_f32_16x16x4f32(av, (b * ecum[ll]) * Ks[ll][dcol], ak, 0, 0, 0);
        }
      }
      // lane: rows 16 ti + 4 g + r of column dcol
      *(float4*)(scr + kScrNv + scr_nv(16 * ti + 4 * g, dcol)) = make_float4(an[0], an[1], an[2], an[3]);
#pragma unroll
      for (int r = 0; r < 4; ++r) scr[kScrKcd + scr_a(16 * ti + 4 * g + r, dcol)] = ak[r];
    }
    // q_e = q e^cum
    for (int e = tid; e < kC * kDk / 4; e += kPP) {
      const int i = e >> 5, d = (e & 31) * 4;
      const float eq = ecum[i];
      const float4 q = *(const float4*)&Qs[i][d];
      *(float4*)(scr + kScrQe + scr_a(i, d)) = make_float4(q.x * eq, q.y * eq, q.z * eq, q.w * eq);
    }
    if (tid == 0) scr[kScrCd] = ecum[kC - 1];
  }
}

// The chunk recurrence on the f32 matrix cores (v_mfma_f32_16x16x4_f32: f32 products, f32
// accumulation, like the reference's f32 matmuls).  Block = one head's 16-column slice of the value
// dimension, 8 waves.  Per chunk:
//   v_new = new_values - k_cumdecay S    (wave: 16 chunk rows x half of the 128 key rows)
//   S'    = S e^cum_last + k_d^T v_new    (wave: 16 key rows)          } concurrently: S' goes to
//   out   = q_e S + intra v_new          (wave: 16 chunk rows x half)  } the other state buffer
// The halves of each key-row sum are added as (lower + upper), then the intra-chunk term, in a fixed
// order.  Each lane takes 4 consecutive k of its operand rows and feeds them to 4 MFMAs (k = 4 g + m
// in step m), the same k order on both operands, so the products summed are exactly those of the
// plain sum.  Every k_cumdecay / q_e / k_d / intra / new-value element is used by one wave only, so
// the waves load theirs straight into registers (the next chunk's while the current one is
// computed); only the state slice (transposed, [column][key row], double-buffered) and v_new
// (transposed) are shared through LDS.  Three barriers per chunk.
constexpr int kST = 512;
constexpr int kStLd = kDk + 4;  // transposed state rows (key rows contiguous)
constexpr int kInLd = kC + 4;   // transposed v_new rows
struct StateOps {  // one wave's operands of one chunk, in MFMA layout
  mfma_f4 ka[4], qa[4], ia[4];  // k_cumdecay / q_e rows 16 rt + c16, keys 64 kh + 16 kk + 4 g + m;
                                // intra rows 16 rt + c16, columns 16 lb + 4 g + m
  float kd[4][4];               // k_d[16 lb + 4 g + m][16 w + c16]
  float vn0[4];                 // new values [16 rt + 4 g + r][c0 + c16]
  float cd;
};
__global__ __launch_bounds__(kST) void gdn_chunk_state_kernel(const GdnPrefill a) {
  __shared__ __align__(16) float St[2][kSl][kStLd];
  __shared__ __align__(16) float VnT[kSl][kInLd];  // v_new, transposed
  __shared__ __align__(16) mfma_f4 RedV[4][64];    // upper halves' v_new partials
  __shared__ __align__(16) mfma_f4 RedO[4][64];    // upper halves' output partials

  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, c16 = l & 15, g = l >> 4;
  const int sl = blockIdx.x % kNsl, h = blockIdx.x / kNsl;
  const int c0 = sl * kSl;
  float* S = a.S + (int64_t)h * kDk * kDk;
  // the new conv state of the head's channels: the last 3 inputs (older ones from the old state
  // when the prompt is shorter than 3); the prep launch has read the old state already
  if (sl == 0 && a.conv_state_out) {
    for (int e = tid; e < 3 * kDk; e += kST) {
      const int part = e >> 7, jj = e & 127;
      const int ch = part == 0 ? h * kDk + jj : (part == 1 ? a.key_dim + h * kDk + jj : 2 * a.key_dim + h * kDk + jj);
      float* st = a.conv_state_out + (int64_t)ch * 3;
      float n[3];
#pragma unroll
      for (int k = 0; k < 3; ++k) {
        const int src = k + a.T;  // index into [old s0, s1, s2, x_0, x_1, ...]
        n[k] = src < 3 ? st[src] : a.raw[(int64_t)(src - 3) * a.ld_raw + ch];
      }
      st[0] = n[0]; st[1] = n[1]; st[2] = n[2];
    }
  }
  // thread (e4 = tid / 4, j4 = 4 (tid % 4)): S rows e4, columns j4..j4+3 of the slice
  const int e4 = tid >> 2, j4 = (tid & 3) * 4;
  {
    const float4 v = *(const float4*)(S + (int64_t)e4 * kDk + c0 + j4);
    St[0][j4][e4] = v.x; St[0][j4 + 1][e4] = v.y; St[0][j4 + 2][e4] = v.z; St[0][j4 + 3][e4] = v.w;
  }
  const int rt = w & 3, kh = w >> 2;  // chunk-row tile and key-row half of the wave
  auto load_ops = [&](int c, StateOps& o) {
    const float* scr = a.scr + ((int64_t)h * a.nchunk + c) * kGdnScratchPerChunk;
    const float* kr = scr + kScrKcd + (rt * 2 + kh) * 4 * 256 + 4 * l;
    const float* qr = scr + kScrQe + (rt * 2 + kh) * 4 * 256 + 4 * l;
    const float* ir = scr + kScrIntra + rt * 4 * 256 + 4 * l;
    const float* dr = scr + kScrKd + w * 4 * 256 + 4 * l;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      o.ka[kk] = *(const mfma_f4*)(kr + 256 * kk);
      o.qa[kk] = *(const mfma_f4*)(qr + 256 * kk);
      o.ia[kk] = *(const mfma_f4*)(ir + 256 * kk);
      const mfma_f4 dv = *(const mfma_f4*)(dr + 256 * kk);
#pragma unroll
      for (int m = 0; m < 4; ++m) o.kd[kk][m] = dv[m];
    }
    const mfma_f4 nv = *(const mfma_f4*)(scr + kScrNv + (sl * 4 + rt) * 256 + 4 * l);
#pragma unroll
    for (int r = 0; r < 4; ++r) o.vn0[r] = nv[r];
    o.cd = scr[kScrCd];
  };
  StateOps cur, nxt;
  load_ops(0, cur);
  __syncthreads();
  int sb = 0;  // state buffer of the current chunk
  for (int c = 0; c < a.nchunk; ++c) {
    if (c + 1 < a.nchunk) load_ops(c + 1, nxt);
    // v_new: rows 16 rt + 4 g + r, column c16; key rows [64 kh, 64 kh + 64)
    {
      mfma_f4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const mfma_f4 bv = *(const mfma_f4*)&St[sb][c16][64 * kh + 16 * kk + 4 * g];
#pragma unroll
        for (int m = 0; m < 4; ++m) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(cur.ka[kk][m], bv[m], acc, 0, 0, 0);
      }
      if (kh == 1) RedV[rt][l] = acc;
      __syncthreads();
      if (kh == 0) {
        const mfma_f4 up = RedV[rt][l];
        mfma_f4 v;
#pragma unroll
        for (int r = 0; r < 4; ++r) v[r] = cur.vn0[r] - (acc[r] + up[r]);
        *(mfma_f4*)&VnT[c16][16 * rt + 4 * g] = v;
      }
      __syncthreads();
    }
    // S' rows 16 w + 4 g + r (column c16) into the other buffer; out partials of (rt, kh)
    {
      mfma_f4 sacc = *(const mfma_f4*)&St[sb][c16][16 * w + 4 * g] * cur.cd;
#pragma unroll
      for (int lb = 0; lb < 4; ++lb) {
        const mfma_f4 bv = *(const mfma_f4*)&VnT[c16][16 * lb + 4 * g];
#pragma unroll
        for (int m = 0; m < 4; ++m) sacc = __builtin_amdgcn_mfma_f32_16x16x4f32(cur.kd[lb][m], bv[m], sacc, 0, 0, 0);
      }
      mfma_f4 oacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const mfma_f4 bv = *(const mfma_f4*)&St[sb][c16][64 * kh + 16 * kk + 4 * g];
#pragma unroll
        for (int m = 0; m < 4; ++m) oacc = __builtin_amdgcn_mfma_f32_16x16x4f32(cur.qa[kk][m], bv[m], oacc, 0, 0, 0);
      }
      mfma_f4 pacc = {0.f, 0.f, 0.f, 0.f};
      if (kh == 0) {
#pragma unroll
        for (int lb = 0; lb < 4; ++lb) {
          if (lb > rt) break;  // (the intra matrix is zero past the diagonal)
          const mfma_f4 bv = *(const mfma_f4*)&VnT[c16][16 * lb + 4 * g];
#pragma unroll
          for (int m = 0; m < 4; ++m) pacc = __builtin_amdgcn_mfma_f32_16x16x4f32(cur.ia[lb][m], bv[m], pacc, 0, 0, 0);
        }
      }
      *(mfma_f4*)&St[sb ^ 1][c16][16 * w + 4 * g] = sacc;
      if (kh == 1) RedO[rt][l] = oacc;
      __syncthreads();
      if (kh == 0) {
        const mfma_f4 up = RedO[rt][l];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int t = c * kC + 16 * rt + 4 * g + r;
          if (t < a.T) a.out[(int64_t)t * a.ld_out + h * kDk + c0 + c16] = (oacc[r] + up[r]) + pacc[r];
        }
      }
    }
    // (no barrier here: the next chunk writes VnT, RedV, RedO and St[sb] only after barriers that
    // every read of them in this chunk precedes)
    cur = nxt;
    sb ^= 1;
  }
  __syncthreads();
  *(float4*)(S + (int64_t)e4 * kDk + c0 + j4) =
      make_float4(St[sb][j4][e4], St[sb][j4 + 1][e4], St[sb][j4 + 2][e4], St[sb][j4 + 3][e4]);
}

// out[t][h*G + i] = (w[i] * (o * rsqrt(mean_h(o^2) + eps))) * silu(z)  (text_modules.rs:91-100);
// amax (optional): max |out[t]| of each row
__global__ __launch_bounds__(kPT) void gated_norm_rows_kernel(const float* o, int ldo, const float* z, int ldz,
                                                              const float* w, int nh, float eps, float* out,
                                                              int ldout, float* amax) {
  __shared__ float sh[4];
  const int t = blockIdx.x, lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  float mx = 0.f;
  for (int h = wid; h < nh; h += 4) {
    const float* orow = o + (int64_t)t * ldo + h * kDk;
    const float* zrow = z + (int64_t)t * ldz + h * kDk;
    const float v0 = orow[lane], v1 = orow[lane + 64];
    const float r = rsqrt_f(wave_sum(v0 * v0 + v1 * v1) / (float)kDk + eps);
    float* dst = out + (int64_t)t * ldout + h * kDk;
    const float y0 = (w[lane] * (v0 * r)) * silu_f(zrow[lane]);
    const float y1 = (w[lane + 64] * (v1 * r)) * silu_f(zrow[lane + 64]);
    dst[lane] = y0;
    dst[lane + 64] = y1;
    mx = fmaxf(mx, fmaxf(fabsf(y0), fabsf(y1)));
  }
  if (amax) block_max256_store(mx, sh, amax + t);
}

// ------------------------------------------------------------------ attention, prompt
// Block (t, slot): slot < nh normalises and rotates query head `slot` into qbuf[t][slot]; slot
// nh + g does kv head g: k_norm + RoPE into the K cache row p0 + t, v copied to the V cache.
__global__ __launch_bounds__(kPT) void attn_prefill_prep_kernel(const AttnPrefill a) {
  __shared__ float sh[4];
  __shared__ float xs[kHdP];
  const int t = blockIdx.x / (a.nh + a.nkv), slot = blockIdx.x % (a.nh + a.nkv);
  const int tid = threadIdx.x;
  const int pos = a.p0 + t;
  const float* src;
  const float* nw;
  if (slot < a.nh) {
    src = a.qg + (int64_t)t * a.ld_qg + (int64_t)slot * 2 * kHdP;
    nw = a.qnw;
  } else {
    src = a.k + (int64_t)t * a.ld_kv + (int64_t)(slot - a.nh) * kHdP;
    nw = a.knw;
  }
  const float v = src[tid];
  const float ss = block_sum256(v * v, sh);
  const float r = rsqrt_f(ss / (float)kHdP + a.eps);
  xs[tid] = (v * r) * (1.0f + nw[tid]);
  __syncthreads();
  float y = xs[tid];
  if (tid < a.rot) {
    const int half = a.rot / 2;
    const float rh = tid < half ? -xs[tid + half] : xs[tid - half];
    y = xs[tid] * a.rcos[(int64_t)pos * a.rot + tid] + rh * a.rsin[(int64_t)pos * a.rot + tid];
  }
  if (slot < a.nh) {
    a.qbuf[((int64_t)t * a.nh + slot) * kHdP + tid] = y;
  } else {
    const int g = slot - a.nh;
    const int64_t row = ((int64_t)g * a.tmax + pos) * kHdP;
    a.kc[row + tid] = y;
    a.vc[row + tid] = a.v[(int64_t)t * a.ld_kv + (int64_t)g * kHdP + tid];
  }
}

// Causal GQA attention of the prompt rows on the f32 matrix cores (v_mfma_f32_16x16x4_f32: f32
// products and accumulation, like the f32 matmuls of the reference's attention).  Block (query
// tile, kv head g): 16 rows = QT tokens x rep query heads of g (QT = 16 / rep), so a 512-token
// prompt gives 128 x kv_heads blocks.  Its 4 waves take every 4th 16-key tile, each with its own
// online softmax (f32, log2 units), and merge their (max, sum, output) in wave order at the end.
// A wave computes S^T = K Q^T for its tile (lane l = 16 g + c16: keys 4 g + r of query row c16)
// and O^T += V^T P^T, whose lane holds dims 16 i + 4 g + r of the same row c16: the row's running
// max, sum and rescale stay in the lane (the 16 keys of a row sit in lanes c16 + 16 g, reduced by
// two exchanges).  Keys and values pass through a per-wave LDS slot, the next tile's loaded into
// registers while the current one is computed; the block's 16 query rows sit in LDS.
constexpr int kRows = 16;          // query rows per block
constexpr int kAW = 4;             // waves per block
constexpr int kAT = 64 * kAW;
constexpr int kKvLd = kHdP + 4;    // padded key / value / query rows in LDS (rows 4 banks apart)
__global__ __launch_bounds__(kAT, 1) void attn_prefill_kernel(const AttnPrefill a) {
  __shared__ __align__(16) float Qs[kRows][kKvLd];
  __shared__ __align__(16) float KV[kAW][2][16][kKvLd];  // per wave: key tile, value tile
  __shared__ float Mw[kAW][kRows], Lw[kAW][kRows];
  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, c16 = l & 15, g = l >> 4;
  const int rep = a.nh / a.nkv, QT = kRows / rep;
  const int qt = blockIdx.x / a.nkv, gk = blockIdx.x % a.nkv;
  const int t = qt * QT + c16 / rep;  // the lane's query row c16: token t
  const int lim = a.p0 + min(t, a.T - 1);  // last key row c16 may see (rows past T are discarded)
  const int tmax_blk = min(a.T, (qt + 1) * QT) - 1;
  const int nkeys = a.p0 + tmax_blk + 1;
  for (int e = tid; e < kRows * kHdP / 4; e += kAT) {
    const int r = e >> 6, d = (e & 63) * 4;
    const int tr = min(qt * QT + r / rep, a.T - 1), hr = gk * rep + r % rep;
    *(q35_f32x4*)&Qs[r][d] = *(const q35_f32x4*)(a.qbuf + ((int64_t)tr * a.nh + hr) * kHdP + d);
  }
  const float* Kg = a.kc + (int64_t)gk * a.tmax * kHdP;
  const float* Vg = a.vc + (int64_t)gk * a.tmax * kHdP;
  float (*Kt)[kKvLd] = KV[w][0];
  float (*Vt)[kKvLd] = KV[w][1];
  q35_f32x4 nk[16], nv[16];  // the next tile: key row u, dims 4 l .. 4 l + 3
  auto load_tile = [&](int k0) {
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const int kj = min(k0 + u, nkeys - 1);
      nk[u] = *(const q35_f32x4*)(Kg + (int64_t)kj * kHdP + 4 * l);
      nv[u] = *(const q35_f32x4*)(Vg + (int64_t)kj * kHdP + 4 * l);
    }
  };
  mfma_f4 o[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) o[i] = mfma_f4{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, lsum = 0.f;
  const float sl2 = a.scale * 1.44269504088896341f;
  int k0 = 16 * w;
  if (k0 < nkeys) load_tile(k0);
  __syncthreads();  // Qs
  for (; k0 < nkeys; k0 += 16 * kAW) {
    // (the wave's reads of its slot in the previous tile precede these stores: LDS is in order)
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      *(q35_f32x4*)&Kt[u][4 * l] = nk[u];
      *(q35_f32x4*)&Vt[u][4 * l] = nv[u];
    }
    if (k0 + 16 * kAW < nkeys) load_tile(k0 + 16 * kAW);
    mfma_f4 sc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < kHdP / 16; ++kk) {
      const mfma_f4 ka = *(const mfma_f4*)&Kt[c16][16 * kk + 4 * g];
      const mfma_f4 qb = *(const mfma_f4*)&Qs[c16][16 * kk + 4 * g];
#pragma unroll
      for (int mm = 0; mm < 4; ++mm) sc = __builtin_amdgcn_mfma_f32_16x16x4f32(ka[mm], qb[mm], sc, 0, 0, 0);
    }
    float sv[4], bm = -INFINITY;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      sv[r] = (k0 + 4 * g + r <= lim) ? sc[r] * sl2 : -INFINITY;
      bm = fmaxf(bm, sv[r]);
    }
    bm = fmaxf(bm, __shfl_xor(bm, 16, 64));
    bm = fmaxf(bm, __shfl_xor(bm, 32, 64));
    const float mn = fmaxf(m, bm);
    float p[4], alpha = 1.f;
    if (mn == -INFINITY) {  // nothing visible yet for this row
      p[0] = p[1] = p[2] = p[3] = 0.f;
    } else {
      alpha = __builtin_amdgcn_exp2f(m - mn);
#pragma unroll
      for (int r = 0; r < 4; ++r) p[r] = __builtin_amdgcn_exp2f(sv[r] - mn);
      m = mn;
    }
    float ps = (p[0] + p[1]) + (p[2] + p[3]);
    ps += __shfl_xor(ps, 16, 64);
    ps += __shfl_xor(ps, 32, 64);
    lsum = lsum * alpha + ps;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      o[i] *= alpha;
#pragma unroll
      for (int mm = 0; mm < 4; ++mm)
        o[i] = __builtin_amdgcn_mfma_f32_16x16x4f32(Vt[4 * g + mm][16 * i + c16], p[mm], o[i], 0, 0, 0);
    }
  }
  // merge the waves' states (key 0, in wave 0's first tile, is visible to every row, so wave 0's
  // maximum is finite)
  __syncthreads();
  float* Om = &KV[0][0][0][0];  // [kAW][kRows][kKvLd]
#pragma unroll
  for (int i = 0; i < 16; ++i) *(mfma_f4*)&Om[(w * kRows + c16) * kKvLd + 16 * i + 4 * g] = o[i];
  if (g == 0) {
    Mw[w][c16] = m;
    Lw[w][c16] = lsum;
  }
  __syncthreads();
  const int q = tid >> 4, d0 = (tid & 15) * 16;
  const int tq = qt * QT + q / rep, hq = gk * rep + q % rep;
  if (tq >= a.T) return;
  float M = Mw[0][q];
#pragma unroll
  for (int ww = 1; ww < kAW; ++ww) M = fmaxf(M, Mw[ww][q]);
  float f[kAW], L = 0.f;
#pragma unroll
  for (int ww = 0; ww < kAW; ++ww) {
    f[ww] = __builtin_amdgcn_exp2f(Mw[ww][q] - M);  // (-inf: 0)
    L += Lw[ww][q] * f[ww];
  }
  const float* gate = a.qg + (int64_t)tq * a.ld_qg + (int64_t)hq * 2 * kHdP + kHdP + d0;
  float* dst = a.out + (int64_t)tq * a.ld_out + (int64_t)hq * kHdP + d0;
#pragma unroll
  for (int d = 0; d < 16; d += 4) {
    q35_f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ww = 0; ww < kAW; ++ww) acc += *(const q35_f32x4*)&Om[(ww * kRows + q) * kKvLd + d0 + d] * f[ww];
    const float4 gv = *(const float4*)(gate + d);
    *(float4*)(dst + d) = make_float4((acc[0] / L) * sigmoid_f(gv.x), (acc[1] / L) * sigmoid_f(gv.y),
                                      (acc[2] / L) * sigmoid_f(gv.z), (acc[3] / L) * sigmoid_f(gv.w));
  }
}

__global__ void store_i32_kernel(int32_t* p, int32_t v) {
  if (threadIdx.x == 0) *p = v;
}

}  // namespace

int store_i32_launch(int32_t* p, int32_t v, hipStream_t st) {
  hipLaunchKernelGGL(store_i32_kernel, dim3(1), dim3(64), 0, st, p, v);
  Q35_HIP_TRY(hipGetLastError());
  return Q35_OK;
}

int rms_rows_launch(float* x, int ldx, int M, int K, const float* w, float eps, float* y, int ldy,
                    hipStream_t st, float* amax, const float* part, int nsplit, int64_t sstride, int ldp,
                    float* clear) {
  if (M < 1) return Q35_OK;
  if (nsplit > 1 && !part) return fail(Q35_E_ARG, "rms_rows: split partials missing");
  hipLaunchKernelGGL(rms_rows_kernel, dim3(M), dim3(kPT), 0, st, x, ldx, K, w, eps, y, ldy, amax,
                     nsplit > 1 ? part : nullptr, nsplit, sstride, ldp, clear);
  Q35_HIP_TRY(hipGetLastError());
  return Q35_OK;
}

int gate_prompt_launch(const float* x, int ldx, int T, int K, const float* wb, const float* wa, const float* alog,
                       const float* dtb, int nh, float* out, hipStream_t st) {
  if (!x || !wb || !wa || !alog || !dtb || !out) return fail(Q35_E_ARG, "gate_proj_prompt: null pointer");
  if (T < 1 || K < 64 || (K % 64) != 0 || nh < 1 || 2 * nh > 32)
    return fail(Q35_E_SHAPE, "gate_proj_prompt: K a multiple of 64 and 2 heads <= 32");
  if ((ldx % 4) != 0 || (reinterpret_cast<uintptr_t>(x) & 15) != 0) return fail(Q35_E_ALIGN, "gate_proj_prompt: x rows must be 16-byte aligned");
  hipLaunchKernelGGL(gate_prompt_kernel, dim3((T + kGateRows - 1) / kGateRows), dim3(kGateT), 0, st, x, ldx, T, K, wb,
                     wa, alog, dtb, nh, out);
  Q35_HIP_TRY(hipGetLastError());
  return Q35_OK;
}

int gdn_prefill_launch(const GdnPrefill& a, hipStream_t st) {
  if (!a.raw || !a.conv_state || !a.conv_w || !a.bg || !a.scr || !a.S || !a.out) return fail(Q35_E_ARG, "gdn_prefill: null pointer");
  if (a.T < 1 || a.nh < 1 || a.nchunk != (a.T + kC - 1) / kC) return fail(Q35_E_SHAPE, "gdn_prefill: bad T / chunks");
  if ((a.ld_out % 4) != 0) return fail(Q35_E_ALIGN, "gdn_prefill: output rows must be 16-byte aligned");
  hipLaunchKernelGGL(gdn_chunk_prep_kernel, dim3(a.nchunk * a.nh), dim3(kPP), 0, st, a);
  Q35_HIP_TRY(hipGetLastError());
  hipLaunchKernelGGL(gdn_chunk_state_kernel, dim3(kNsl * a.nh), dim3(kST), 0, st, a);
  Q35_HIP_TRY(hipGetLastError());
  return Q35_OK;
}

int gated_norm_rows_launch(const float* o, int ldo, const float* z, int ldz, const float* w, int T, int nh, float eps,
                           float* out, int ldout, hipStream_t st, float* amax) {
  if (T < 1) return Q35_OK;
  hipLaunchKernelGGL(gated_norm_rows_kernel, dim3(T), dim3(kPT), 0, st, o, ldo, z, ldz, w, nh, eps, out, ldout, amax);
  Q35_HIP_TRY(hipGetLastError());
  return Q35_OK;
}

int attn_prefill_launch(const AttnPrefill& a, hipStream_t st) {
  if (!a.qg || !a.k || !a.v || !a.qnw || !a.knw || !a.rcos || !a.rsin || !a.kc || !a.vc || !a.qbuf || !a.out)
    return fail(Q35_E_ARG, "attention prefill: null pointer");
  if (a.T < 1) return Q35_OK;
  if (a.nkv < 1 || a.nh % a.nkv != 0 || kRows % (a.nh / a.nkv) != 0) return fail(Q35_E_SHAPE, "attention prefill: heads");
  if (a.p0 < 0 || (int64_t)a.p0 + a.T > a.tmax) return fail(Q35_E_SHAPE, "attention prefill: positions past tmax");
  if (a.rot < 2 || a.rot > kHdP || (a.rot % 2) != 0) return fail(Q35_E_SHAPE, "attention prefill: rotary dims");
  if ((a.ld_qg % 4) != 0 || (a.ld_out % 4) != 0) return fail(Q35_E_ALIGN, "attention prefill: row alignment");
  hipLaunchKernelGGL(attn_prefill_prep_kernel, dim3(a.T * (a.nh + a.nkv)), dim3(kPT), 0, st, a);
  Q35_HIP_TRY(hipGetLastError());
  const int QT = kRows / (a.nh / a.nkv);
  const int nqt = (a.T + QT - 1) / QT;
  hipLaunchKernelGGL(attn_prefill_kernel, dim3(nqt * a.nkv), dim3(kAT), 0, st, a);
  Q35_HIP_TRY(hipGetLastError());
  return Q35_OK;
}

}  // namespace q35
