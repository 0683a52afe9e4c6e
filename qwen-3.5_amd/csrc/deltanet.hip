// Gated DeltaNet single-token step (text_modules.rs:134-162 causal_conv1d_update,
// :184-187 l2norm, :365-443 burn_recurrent_gated_delta_rule), plus the standalone gate
// projection (kernels.rs:174-247) and the causal-conv state shift.
//
// Step block (b, head h, slice of 32 or, for many rows, all 128 columns of the value dim): 256
// threads.  Threads 0..255 run the 4-tap depthwise conv + SiLU for the head's 128 q and 128 k
// channels, the first threads the slice's v channels; q and k are L2-normalised in LDS.  The
// state slice S[h][0:128][j0:j0+CS] (16 or 64 KB) is held in registers, 16 rows per thread (one
// column, or a float4 of columns): decay, S^T k (8-way
// LDS reduction), delta = (v - S^T k) * beta, rank-1 update, S^T q, write back.  Every value
// column is independent, so slices need no cross-block reduction; the per-head gated RMSNorm
// is applied by the out_proj matvec prologue.  All slices of a head read the same q/k conv
// channels, so the conv state can only be advanced once every slice has read it: with a
// counter per (row, head) (head_ctr), the last slice block of the head to finish shifts the head's
// 2*dk + dv channels itself; otherwise it is advanced afterwards by conv_shift or by a side task
// of the next matvec launch.
#include "q35_internal.h"

namespace q35 {

namespace {

constexpr int kThreads = 256;
constexpr int kDk = 128;
constexpr int kRowGroups = kThreads / 32;  // 8 row groups of 32 column groups
constexpr int kRowsPerThread = kDk / kRowGroups;  // 16

struct GdnArgs {
  GdnCall c;
  int32_t conv_dim, key_dim, nslice;
  float qscale;
};

// QF: the mixed qkv rows are fixed-point accumulator words (else f32).  A compile-time choice:
// a load inside a runtime branch is joined by a wait for every load in flight (the state slice).
template <bool QF>
Q35_DEV float qkv_at(const GdnCall& c, int b, int ch) {
  const size_t i = (size_t)b * c.ld_qkv + ch;
  if constexpr (QF) return from_fx(c.qkv_f[i]);
  else return c.qkv[i];
}

Q35_DEV float conv4_silu(float xin, const float* st, const float* w) {
  const float acc = ((w[0] * st[0] + w[1] * st[1]) + w[2] * st[2]) + w[3] * xin;
  return silu_f(acc);
}

// One channel's conv inputs in registers (loaded ahead of any use), and the same conv + SiLU.
struct ConvIn {
  float x, s[3], w[4];
};
template <bool QF>
Q35_DEV ConvIn conv_in(const GdnCall& a, const float* cs, int b, int c) {
  ConvIn r;
  r.x = qkv_at<QF>(a, b, c);
  const float* st = cs + (size_t)c * 3;
  const float* w = a.conv_w + (size_t)c * 4;
  r.s[0] = st[0]; r.s[1] = st[1]; r.s[2] = st[2];
  r.w[0] = w[0]; r.w[1] = w[1]; r.w[2] = w[2]; r.w[3] = w[3];
  return r;
}
Q35_DEV float conv4_silu(const ConvIn& r) { return conv4_silu(r.x, r.s, r.w); }

// BF: the gates arrive as raw fixed-point projections (else activated f32 [beta | g]).
template <int CS, bool QF, bool BF>
__global__ __launch_bounds__(kThreads) void gdn_step_kernel(const GdnArgs A) {
  constexpr int VW = CS / 32;  // value columns per thread (4: one float4)
  const GdnCall& a = A.c;
  __shared__ float qk[2 * kDk];
  __shared__ float qh[kDk];
  __shared__ float kh[kDk];
  __shared__ float vv[CS];
  __shared__ float wsum[4];
  __shared__ float red[kRowGroups * CS];
  __shared__ int last_flag;

  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int slice = blockIdx.x % A.nslice;
  const int h = (blockIdx.x / A.nslice) % a.nh;
  const int b = blockIdx.x / (A.nslice * a.nh);
  const float* cs = a.conv_state + (size_t)b * A.conv_dim * 3;

  // state slice loads first: their latency overlaps the conv / norm work.  Thread (column group
  // jq = tid % 32, row group ig = tid / 32): columns VW jq .. VW jq + VW - 1, rows 16 ig .. + 15
  const int jq = tid % 32, ig = tid / 32, j0 = VW * jq;
  const int i0 = ig * kRowsPerThread;
  float* Sp = a.S + (((size_t)b * a.nh + h) * kDk) * a.dv + slice * CS + j0;
  float sr[kRowsPerThread][VW];
#pragma unroll
  for (int r = 0; r < kRowsPerThread; ++r) {
    if constexpr (VW == 4) {
      const float4 v = *(const float4*)(Sp + (size_t)(i0 + r) * a.dv);
      sr[r][0] = v.x; sr[r][1] = v.y; sr[r][2] = v.z; sr[r][3] = v.w;
    } else {
      sr[r][0] = Sp[(size_t)(i0 + r) * a.dv];
    }
  }

  // the gate inputs too (independent of everything above: one round trip for all; kept raw
  // until used, so that no wait for them sits before the conv loads)
  fx_t g_bx = 0, g_ax = 0;
  float g_b = 0.f, g_a = 0.f, g_dt = 0.f, g_al = 0.f;
  if constexpr (BF) {
    g_bx = a.ba_f[(size_t)b * a.ld_bg + h];
    g_ax = a.ba_f[(size_t)b * a.ld_bg + a.nh + h];
    g_dt = a.dt_bias[h];
    g_al = a.a_log[h];
  } else {
    g_b = a.bg[(size_t)b * a.ld_bg + h];
    g_a = a.bg[(size_t)b * a.ld_bg + a.nh + h];
  }

  // the conv inputs of the thread's q (tid < 128) or k channel of head h and of the slice's v
  // channel (clamped: every thread loads, the first CS use it), all issued before any is used,
  // so the state slice, the gates and the conv inputs take one round trip; no divergent branch
  // around a load (its join would wait for every load in flight)
  const ConvIn in_qk = conv_in<QF>(a, cs, b, (tid < kDk) ? h * kDk + tid : A.key_dim + h * kDk + (tid - kDk));
  const ConvIn in_v = conv_in<QF>(a, cs, b, 2 * A.key_dim + h * a.dv + slice * CS + min(tid, CS - 1));
  __builtin_amdgcn_sched_barrier(0);  // (the scheduler would interleave the conv math and its waits)
  qk[tid] = conv4_silu(in_qk);
  if (tid < CS) vv[tid] = conv4_silu(in_v);
  __syncthreads();
  {
    const float v = qk[tid];
    const float ss = wave_sum(v * v);
    if (lane == 0) wsum[wid] = ss;
  }
  __syncthreads();
  const float rq = rsqrt_f((wsum[0] + wsum[1]) + 1e-6f);
  const float rk = rsqrt_f((wsum[2] + wsum[3]) + 1e-6f);
  if (tid < kDk) qh[tid] = (qk[tid] * rq) * A.qscale;
  else kh[tid - kDk] = qk[tid] * rk;

  float beta, g;
  if constexpr (BF) {  // raw projections: beta = sigmoid(b); g = -exp(A_log) * softplus(a + dt_bias)
    beta = sigmoid_f(from_fx(g_bx));
    const float xg = from_fx(g_ax) + g_dt;
    const float pre = logf(expf(xg) + 1.0f);
    g = -expf(g_al) * (pre > 20.0f ? xg : pre);
  } else {
    beta = g_b;
    g = g_a;
  }
  const float decay = expf(g);
  __syncthreads();

  float mp[VW];
#pragma unroll
  for (int u = 0; u < VW; ++u) mp[u] = 0.f;
#pragma unroll
  for (int r = 0; r < kRowsPerThread; ++r)
#pragma unroll
    for (int u = 0; u < VW; ++u) {
      sr[r][u] = sr[r][u] * decay;
      mp[u] += sr[r][u] * kh[i0 + r];
    }
#pragma unroll
  for (int u = 0; u < VW; ++u) red[ig * CS + j0 + u] = mp[u];
  __syncthreads();
  float delta[VW];
#pragma unroll
  for (int u = 0; u < VW; ++u) {
    float m = 0.f;
#pragma unroll
    for (int i = 0; i < kRowGroups; ++i) m += red[i * CS + j0 + u];
    delta[u] = (vv[j0 + u] - m) * beta;
  }
  __syncthreads();
  float op[VW];
#pragma unroll
  for (int u = 0; u < VW; ++u) op[u] = 0.f;
#pragma unroll
  for (int r = 0; r < kRowsPerThread; ++r) {
#pragma unroll
    for (int u = 0; u < VW; ++u) {
      sr[r][u] = sr[r][u] + kh[i0 + r] * delta[u];
      op[u] += sr[r][u] * qh[i0 + r];
    }
    if constexpr (VW == 4) {
      *(float4*)(Sp + (size_t)(i0 + r) * a.dv) = make_float4(sr[r][0], sr[r][1], sr[r][2], sr[r][3]);
    } else {
      Sp[(size_t)(i0 + r) * a.dv] = sr[r][0];
    }
  }
#pragma unroll
  for (int u = 0; u < VW; ++u) red[ig * CS + j0 + u] = op[u];
  __syncthreads();
  if (tid < CS) {
    float o = 0.f;
#pragma unroll
    for (int i = 0; i < kRowGroups; ++i) o += red[i * CS + tid];
    a.o[(size_t)b * a.ld_o + h * a.dv + slice * CS + tid] = o;
  }
  if (!a.head_ctr) return;
  // conv state advance, [s0, s1, s2] <- [s1, s2, x], from the registers loaded above: each slice
  // owns its CS v channels and advances them now; the q/k channels are read by every slice of
  // (b, h), so the last slice to get here advances them
  float* cw = a.conv_state + (size_t)b * A.conv_dim * 3;
  if (tid < CS) {
    float* st = cw + (size_t)(2 * A.key_dim + h * a.dv + slice * CS + tid) * 3;
    st[0] = in_v.s[1]; st[1] = in_v.s[2]; st[2] = in_v.x;
  }
  if (!arrive_last(&a.head_ctr[b * a.nh + h], (uint32_t)A.nslice, &last_flag)) return;
  {
    float* st = cw + (size_t)((tid < kDk) ? h * kDk + tid : A.key_dim + h * kDk + (tid - kDk)) * 3;
    st[0] = in_qk.s[1]; st[1] = in_qk.s[2]; st[2] = in_qk.x;
  }
}

__global__ __launch_bounds__(kThreads) void conv_shift_kernel(float* state, const float* x, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads) {
    float* st = state + i * 3;
    const float s1 = st[1], s2 = st[2];
    st[0] = s1; st[1] = s2; st[2] = x[i];
  }
}

// Standalone gate projection: one block per batch row; thread t owns output t % (2*nh) and a
// strided subset of the input rows, partial sums are reduced in LDS in a fixed order, then
// sigmoid / -exp(A_log)*softplus are applied.  The softplus switches to the identity when its
// result exceeds 20 (the decode kernel, kernels.rs:238-243) or, with input_rule, when its input
// does (the prompt path, text_modules.rs:587-592).
__global__ __launch_bounds__(kThreads) void gate_proj_kernel(const float* x, int32_t in_dim, const float* wb,
                                                            const float* wa, const float* alog, const float* dtb,
                                                            int32_t nh, float* out, int32_t input_rule) {
  __shared__ float red[kThreads];
  const int tid = threadIdx.x, b = blockIdx.x;
  const int nout = 2 * nh, subs = kThreads / nout;
  const int o = tid % nout, sub = tid / nout, h = o % nh;
  const float* W = (o < nh) ? wb : wa;
  const float* xb = x + (size_t)b * in_dim;
  float acc = 0.f;
  for (int k = sub; k < in_dim; k += subs) acc += xb[k] * W[(size_t)k * nh + h];
  red[sub * nout + o] = acc;
  __syncthreads();
  if (tid < nout) {
    float s = 0.f;
    for (int j = 0; j < subs; ++j) s += red[j * nout + tid];
    float r;
    if (tid < nh) {
      r = sigmoid_f(s);
    } else {
      const float xg = s + dtb[h];
      const float pre = logf(expf(xg) + 1.0f);
      r = -expf(alog[h]) * ((input_rule ? xg : pre) > 20.0f ? xg : pre);
    }
    out[(size_t)b * nout + tid] = r;
  }
}

}  // namespace

int gate_proj_simple_launch(const float* x, int32_t B, int32_t in_dim, const float* wb, const float* wa,
                            const float* alog, const float* dtb, int32_t nh, float* out, hipStream_t st,
                            int32_t input_rule) {
  if (!x || !wb || !wa || !alog || !dtb || !out) return fail(Q35_E_ARG, "gate_proj: null pointer");
  if (B < 1 || in_dim < 1 || nh < 1) return fail(Q35_E_SHAPE, "gate_proj: B, in_dim, n_heads must be >= 1");
  if (2 * nh > kThreads || (kThreads % (2 * nh)) != 0) return fail(Q35_E_SHAPE, "gate_proj: 2*n_heads must divide 256");
  hipLaunchKernelGGL(gate_proj_kernel, dim3(B), dim3(kThreads), 0, st, x, in_dim, wb, wa, alog, dtb, nh, out,
                     input_rule);
  Q35_HIP_TRY(hipGetLastError());
  return Q35_OK;
}

int gdn_step_launch(const GdnCall& c, hipStream_t st) {
  if ((!c.qkv && !c.qkv_f) || !c.conv_state || !c.conv_w || !c.S || !c.o) return fail(Q35_E_ARG, "gdn_step: null pointer");
  if (!c.bg && !(c.ba_f && c.a_log && c.dt_bias)) return fail(Q35_E_ARG, "gdn_step: need bg, or ba_f with a_log and dt_bias");
  if (c.dk != kDk) return fail(Q35_E_SHAPE, "gdn_step: key head dim must be 128");
  if (c.dv <= 0 || (c.dv % 32) != 0) return fail(Q35_E_SHAPE, "gdn_step: value head dim must be a multiple of 32");
  if (c.conv_k != 4) return fail(Q35_E_SHAPE, "gdn_step: conv kernel must be 4");
  if (c.B < 1 || c.nh < 1) return fail(Q35_E_SHAPE, "gdn_step: B and heads must be >= 1");
  GdnArgs a;
  a.c = c;
  a.key_dim = c.nh * c.dk;
  a.conv_dim = 2 * a.key_dim + c.nh * c.dv;
  a.qscale = powf((float)c.dk, -0.5f);
  // whole-head blocks (128 columns, a float4 per thread and row: long row segments, the head's
  // q / k conv and norms done once) when there are enough of them to fill the GPU; 32-column
  // slices otherwise
  // whole value heads per block once there are enough blocks without slicing (B * nh >= 512: B =
  // 32 at 16 heads; at B = 16 the 32-column slices measured 0.3% faster)
  const bool wide = (c.dv % 128) == 0 && (int64_t)c.B * c.nh >= 512 &&
                    (reinterpret_cast<uintptr_t>(c.S) & 15) == 0 && (c.dv % 4) == 0;
  a.nslice = c.dv / (wide ? 128 : 32);
  const int grid = c.B * c.nh * a.nslice;
  const void* k;
  if (c.qkv_f)
    k = c.ba_f ? (wide ? (const void*)gdn_step_kernel<128, true, true> : (const void*)gdn_step_kernel<32, true, true>)
               : (wide ? (const void*)gdn_step_kernel<128, true, false> : (const void*)gdn_step_kernel<32, true, false>);
  else
    k = c.ba_f ? (wide ? (const void*)gdn_step_kernel<128, false, true> : (const void*)gdn_step_kernel<32, false, true>)
               : (wide ? (const void*)gdn_step_kernel<128, false, false> : (const void*)gdn_step_kernel<32, false, false>);
  void* params[] = {&a};
  Q35_HIP_TRY(hipLaunchKernel(k, dim3(grid), dim3(kThreads), params, 0, st));
  Q35_HIP_TRY(hipGetLastError());
  return Q35_OK;
}

int conv_shift_launch(float* state, const float* x, int32_t B, int32_t ch, hipStream_t st) {
  if (!state || !x) return fail(Q35_E_ARG, "conv_shift: null pointer");
  const int64_t n = (int64_t)B * ch;
  if (n <= 0) return Q35_OK;
  int64_t g = (n + kThreads - 1) / kThreads;
  if (g > 1024) g = 1024;
  hipLaunchKernelGGL(conv_shift_kernel, dim3((unsigned)g), dim3(kThreads), 0, st, state, x, n);
  Q35_HIP_TRY(hipGetLastError());
  return Q35_OK;
}

}  // namespace q35
