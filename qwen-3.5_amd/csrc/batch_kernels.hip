// Kernels of the batched decode step that the single-sequence kernels do not cover: the
// per-sequence token selection + embedding into the fixed-point residual rows, and the
// per-sequence greedy argmax over the logits rows (the reference's tie order), which advances
// each sequence's position and history.
#include "q35_internal.h"

#include <climits>

namespace q35 {
namespace {

constexpr int kBT = 256;

// Row b: the prompt id at pos[b] while pos[b] < plen[b], else the row's last argmax; its
// dequantised embedding row goes to the residual row h[b] (fixed point).
__global__ __launch_bounds__(kBT) void batch_embed_kernel(const int8_t* q, const float* s, int D,
                                                         const int32_t* token, const int32_t* prompt, int ldp,
                                                         const int32_t* plen, const int32_t* pos, fx_t* h) {
  const int b = blockIdx.y;
  const int p = pos[b];
  const int tok = p < plen[b] ? prompt[(int64_t)b * ldp + p] : token[b];
  const int8_t* qr = q + (int64_t)tok * D;
  const float* sr = s + (int64_t)tok * (D / 64);
  for (int k = blockIdx.x * kBT + threadIdx.x; k < D; k += gridDim.x * kBT)
    h[(int64_t)b * D + k] = to_fx((float)qr[k] * sr[k >> 6]);
}

// f32 residual rows for the batched step on the matrix cores: row b's embedding (as above) into
// h[b] and its sum of squares into ss[b] (the first RMSNorm's statistic); every block also
// clears its share of zero_ptr[0 .. zero_n) (accumulators the step adds into).
__global__ __launch_bounds__(kBT) void batch_embed_f32_kernel(const int8_t* q, const float* s, int D,
                                                             const int32_t* token, const int32_t* prompt, int ldp,
                                                             const int32_t* plen, const int32_t* pos, float* h, fx_t* ss,
                                                             fx_t* zero_ptr, int64_t zero_n, uint32_t* err) {
  __shared__ float sh[4];
  for (int64_t i = (int64_t)blockIdx.x * kBT + threadIdx.x; i < zero_n; i += (int64_t)gridDim.x * kBT) zero_ptr[i] = 0;
  const int b = blockIdx.x;
  const int p = pos[b];
  const int tok = p < plen[b] ? prompt[(int64_t)b * ldp + p] : token[b];
  const int8_t* qr = q + (int64_t)tok * D;
  const float* sr = s + (int64_t)tok * (D / 64);
  float acc = 0.f;
  for (int k = threadIdx.x; k < D; k += kBT) {
    const float e = (float)qr[k] * sr[k >> 6];
    h[(int64_t)b * D + k] = e;
    acc += e * e;
  }
  acc = block_sum256(acc, sh);
  if (threadIdx.x == 0) {
    if (!fx_addable(acc)) __hip_atomic_fetch_or((Q35_GLOBAL uint32_t*)err, kWsErrRange, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    ss[b] = fx_addable(acc) ? to_fx(acc) : 0;
  }
}

Q35_DEV void block_argmax256(float& v, int& i, float* shv, int* shi, const ArgOrder& o) {
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

// Block (b, g) reduces values [g*span, (g+1)*span) of logits row b to one partial.
__global__ __launch_bounds__(kBT) void batch_argmax_part_kernel(const float* logits, int V, int G, int span,
                                                               float* pv, int32_t* pi, const ArgOrder ord) {
  __shared__ float shv[4];
  __shared__ int shi[4];
  const int b = blockIdx.x / G, g = blockIdx.x % G;
  const float* row = logits + (int64_t)b * V;
  const int lo = g * span, hi = min(V, lo + span);
  float v = -INFINITY;
  int ix = INT_MAX;
  for (int i = lo + threadIdx.x; i < hi; i += kBT) {
    const float x = row[i];
    if (argmax_better(x, i, v, ix, ord)) { v = x; ix = i; }
  }
  block_argmax256(v, ix, shv, shi, ord);
  if (threadIdx.x == 0) {
    pv[blockIdx.x] = v;
    pi[blockIdx.x] = ix;
  }
}

// Block b: the row's argmax from its G partials -> token[b], hist[b][pos[b]], pos[b] + 1.
__global__ __launch_bounds__(kBT) void batch_argmax_final_kernel(const float* pv, const int32_t* pi, int G,
                                                                int32_t* token, int32_t* pos, int32_t* hist, int ldh,
                                                                const ArgOrder ord) {
  __shared__ float shv[4];
  __shared__ int shi[4];
  const int b = blockIdx.x;
  float v = -INFINITY;
  int ix = INT_MAX;
  for (int g = threadIdx.x; g < G; g += kBT)
    if (argmax_better(pv[b * G + g], pi[b * G + g], v, ix, ord)) { v = pv[b * G + g]; ix = pi[b * G + g]; }
  block_argmax256(v, ix, shv, shi, ord);
  if (threadIdx.x == 0) {
    const int tok = ix == INT_MAX ? 0 : ix;
    const int p = pos[b];
    token[b] = tok;
    hist[(int64_t)b * ldh + p] = tok;
    pos[b] = p + 1;
  }
}

}  // namespace

int batch_embed_f32_launch(const int8_t* q, const float* s, int D, const int32_t* token, const int32_t* prompt, int ldp,
                           const int32_t* plen, const int32_t* pos, float* h, fx_t* ss, fx_t* zero_ptr, int64_t zero_n,
                           uint32_t* err, int B, hipStream_t st) {
  hipLaunchKernelGGL(batch_embed_f32_kernel, dim3(B), dim3(kBT), 0, st, q, s, D, token, prompt, ldp, plen, pos, h, ss,
                     zero_ptr, zero_n, err);
  Q35_HIP_TRY(hipGetLastError());
  return Q35_OK;
}

int batch_embed_launch(const int8_t* q, const float* s, int D, const int32_t* token, const int32_t* prompt, int ldp,
                       const int32_t* plen, const int32_t* pos, fx_t* h, int B, hipStream_t st) {
  const int gx = std::min((D + kBT - 1) / kBT, 8);
  hipLaunchKernelGGL(batch_embed_kernel, dim3(gx, B), dim3(kBT), 0, st, q, s, D, token, prompt, ldp, plen, pos, h);
  Q35_HIP_TRY(hipGetLastError());
  return Q35_OK;
}

int batch_argmax_groups(int V) { return std::max(1, std::min(64, (V + 4095) / 4096)); }

int batch_argmax_launch(const float* logits, int V, int B, float* pv, int32_t* pi, int32_t* token, int32_t* pos,
                        int32_t* hist, int ldh, hipStream_t st) {
  const int G = batch_argmax_groups(V), span = (V + G - 1) / G;
  const ArgOrder ord = make_arg_order(V);
  hipLaunchKernelGGL(batch_argmax_part_kernel, dim3(B * G), dim3(kBT), 0, st, logits, V, G, span, pv, pi, ord);
  Q35_HIP_TRY(hipGetLastError());
  hipLaunchKernelGGL(batch_argmax_final_kernel, dim3(B), dim3(kBT), 0, st, pv, pi, G, token, pos, hist, ldh, ord);
  Q35_HIP_TRY(hipGetLastError());
  return Q35_OK;
}

}  // namespace q35
