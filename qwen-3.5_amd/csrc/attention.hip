// Gated GQA attention for one decode token (text_modules.rs:842-944): per-head q/k RMSNorm
// (1+w), partial RoPE on the first rot dims (rotate_half, :739-774), K/V append at the
// current position, softmax(q K^T / sqrt(d)) V over the cache with GQA (q head h reads kv
// head h / (nh/nkv), repeat_kv :776-792) and the sigmoid output gate (:936) — one kernel.
//
// Split-T ("flash decoding"): block (b, kv head g, chunk c) handles `chunk` cached tokens for
// all rep = nh/nkv query heads that share kv head g, so each K/V row is read once for rep
// heads.  Waves take tokens round-robin; a lane owns 4 of the 256 dims (one float4 of every
// K/V row, 1 KB coalesced per wave per token).  Each block publishes (max, sum, o[rep][d]);
// the last block of the (b, g) group merges the chunks in order and applies the gate.
// The grid covers tmax so a captured graph stays valid as the position advances; blocks past
// the current length exit at once.
#include "q35_internal.h"

namespace q35 {

namespace {

constexpr int kThreads = 256;
constexpr int kHd = 256;
constexpr int kMaxRep = 4;
constexpr int kMaxChunk = 256;     // tokens per block
constexpr int kMaxChunks = 1024;   // chunks per (b, kv head): the merge weights live in LDS

struct AttnArgs {
  AttnCall c;
  float scale;
  int32_t chunk, nchunk;
  uint32_t* counters;  // [B*nkv] completion counters; counters[kWsErrWord] the sticky error word
  float* part_ml;      // [B*nkv][nchunk][2][kMaxRep]
  float* part_o;       // [B*nkv][nchunk][kMaxRep][hd]
};

Q35_DEV float4 ld4(const float* f, const fx_t* x, size_t i) {
  if (x) return make_float4(from_fx(x[i]), from_fx(x[i + 1]), from_fx(x[i + 2]), from_fx(x[i + 3]));
  return *reinterpret_cast<const float4*>(f + i);
}
Q35_DEV float ld1(const float* f, const fx_t* x, size_t i) { return x ? from_fx(x[i]) : f[i]; }

__global__ __launch_bounds__(kThreads) void attn_decode_kernel(const AttnArgs A) {
  const AttnCall& a = A.c;
  __shared__ __align__(16) float qn[kMaxRep][kHd];
  __shared__ __align__(16) float kn[kHd];
  __shared__ __align__(16) float vn[kHd];
  __shared__ float rtmp[kMaxRep + 1][kHd];
  __shared__ float sc[kMaxRep][kMaxChunk];
  __shared__ __align__(16) float ored[4][kMaxRep][kHd];
  __shared__ float hm[kMaxRep], hl[kMaxRep];
  __shared__ int flag;

  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int c = blockIdx.x % A.nchunk;
  const int g = (blockIdx.x / A.nchunk) % a.nkv;
  const int b = blockIdx.x / (A.nchunk * a.nkv);
  const int rep = a.nh / a.nkv;
  const int pos = a.pos[b];
  if (pos < 0 || pos >= a.tmax) {  // no cache row or rotary row exists for it: report, touch nothing
    if (tid == 0 && c == 0 && g == 0) ws_raise(A.counters, kWsErrPos);
    return;
  }
  const int T = pos + 1;
  const int nact = (T + A.chunk - 1) / A.chunk;
  if (c >= nact) return;
  const int t0 = c * A.chunk;
  const int len = min(A.chunk, T - t0);
  const bool has_new = (c == nact - 1);

  // 1. q heads (wave w -> head g*rep + w), plus k/v of the new token in the chunk holding it
  for (int w = wid; w < rep + (has_new ? 2 : 0); w += 4) {
    if (w < rep) {
      const int hq = g * rep + w;
      const float4 v = ld4(a.qg, a.qg_f, (size_t)b * a.ld_qg + (size_t)hq * 2 * kHd + 4 * lane);
      const float ss = wave_sum(v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w);
      const float r = rsqrt_f(ss / (float)kHd + a.eps);
      const int d = 4 * lane;
      qn[w][d + 0] = (v.x * r) * (1.0f + a.qnw[d + 0]);
      qn[w][d + 1] = (v.y * r) * (1.0f + a.qnw[d + 1]);
      qn[w][d + 2] = (v.z * r) * (1.0f + a.qnw[d + 2]);
      qn[w][d + 3] = (v.w * r) * (1.0f + a.qnw[d + 3]);
    } else if (w == rep) {
      const float4 v = ld4(a.k, a.k_f, (size_t)b * a.ld_kv + (size_t)g * kHd + 4 * lane);
      const float ss = wave_sum(v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w);
      const float r = rsqrt_f(ss / (float)kHd + a.eps);
      const int d = 4 * lane;
      kn[d + 0] = (v.x * r) * (1.0f + a.knw[d + 0]);
      kn[d + 1] = (v.y * r) * (1.0f + a.knw[d + 1]);
      kn[d + 2] = (v.z * r) * (1.0f + a.knw[d + 2]);
      kn[d + 3] = (v.w * r) * (1.0f + a.knw[d + 3]);
    } else {
      const float4 v = ld4(a.v, a.v_f, (size_t)b * a.ld_kv + (size_t)g * kHd + 4 * lane);
      *reinterpret_cast<float4*>(&vn[4 * lane]) = v;
    }
  }
  __syncthreads();
  // 2. RoPE on dims [0, rot): x' = x*cos + rotate_half(x)*sin (computed into rtmp, then copied)
  const int half = a.rot / 2;
  const float* cs = a.rcos + (size_t)pos * a.rot;
  const float* sn = a.rsin + (size_t)pos * a.rot;
  const int nrot_heads = rep + (has_new ? 1 : 0);
  for (int e = tid; e < nrot_heads * a.rot; e += kThreads) {
    const int hh = e / a.rot, i = e % a.rot;
    const float* src = (hh < rep) ? qn[hh] : kn;
    const float rh = (i < half) ? -src[i + half] : src[i - half];
    rtmp[hh][i] = src[i] * cs[i] + rh * sn[i];
  }
  __syncthreads();
  for (int e = tid; e < nrot_heads * a.rot; e += kThreads) {
    const int hh = e / a.rot, i = e % a.rot;
    if (hh < rep) qn[hh][i] = rtmp[hh][i];
    else kn[i] = rtmp[hh][i];
  }
  __syncthreads();
  const size_t cache_off = (((size_t)b * a.nkv + g) * a.tmax) * kHd;
  const float* Kc = a.kc + cache_off;
  const float* Vc = a.vc + cache_off;
  if (has_new) {  // append (post-RoPE k, raw v) at row `pos`
    a.kc[cache_off + (size_t)pos * kHd + tid] = kn[tid];
    a.vc[cache_off + (size_t)pos * kHd + tid] = vn[tid];
  }

  // 3. scores: wave w takes tokens w, w+4, ...
  float q4[kMaxRep][4];
#pragma unroll
  for (int h = 0; h < kMaxRep; ++h)
#pragma unroll
    for (int i = 0; i < 4; ++i) q4[h][i] = (h < rep) ? qn[h][4 * lane + i] : 0.f;
  for (int tt = wid; tt < len; tt += 4) {
    const int t = t0 + tt;
    const float4 kv = (t == pos) ? *reinterpret_cast<const float4*>(&kn[4 * lane])
                                 : *reinterpret_cast<const float4*>(Kc + (size_t)t * kHd + 4 * lane);
#pragma unroll
    for (int h = 0; h < kMaxRep; ++h) {
      if (h >= rep) break;
      float d = q4[h][0] * kv.x + q4[h][1] * kv.y + q4[h][2] * kv.z + q4[h][3] * kv.w;
      d = wave_sum(d);
      if (lane == 0) sc[h][tt] = d * A.scale;
    }
  }
  __syncthreads();
  // 4. per-head max and exp-sum over the chunk (wave h -> head h)
  for (int h = wid; h < rep; h += 4) {
    float mx = -INFINITY;
    for (int tt = lane; tt < len; tt += 64) mx = fmaxf(mx, sc[h][tt]);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    float l = 0.f;
    for (int tt = lane; tt < len; tt += 64) {
      const float p = expf(sc[h][tt] - mx);
      sc[h][tt] = p;
      l += p;
    }
    l = wave_sum(l);
    if (lane == 0) { hm[h] = mx; hl[h] = l; }
  }
  __syncthreads();
  // 5. o = sum_t p_t V_t
  float acc[kMaxRep][4];
#pragma unroll
  for (int h = 0; h < kMaxRep; ++h)
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[h][i] = 0.f;
  for (int tt = wid; tt < len; tt += 4) {
    const int t = t0 + tt;
    const float4 vv = (t == pos) ? *reinterpret_cast<const float4*>(&vn[4 * lane])
                                 : *reinterpret_cast<const float4*>(Vc + (size_t)t * kHd + 4 * lane);
#pragma unroll
    for (int h = 0; h < kMaxRep; ++h) {
      if (h >= rep) break;
      const float p = sc[h][tt];
      acc[h][0] += p * vv.x; acc[h][1] += p * vv.y; acc[h][2] += p * vv.z; acc[h][3] += p * vv.w;
    }
  }
#pragma unroll
  for (int h = 0; h < kMaxRep; ++h)
    *reinterpret_cast<float4*>(&ored[wid][h][4 * lane]) = make_float4(acc[h][0], acc[h][1], acc[h][2], acc[h][3]);
  __syncthreads();
  float o[kMaxRep];
#pragma unroll
  for (int h = 0; h < kMaxRep; ++h) o[h] = (ored[0][h][tid] + ored[1][h][tid]) + (ored[2][h][tid] + ored[3][h][tid]);

  const int grpi = b * a.nkv + g;
  const size_t gate0 = (size_t)b * a.ld_qg;
  if (nact == 1) {
#pragma unroll
    for (int h = 0; h < kMaxRep; ++h) {
      if (h >= rep) break;
      const int hq = g * rep + h;
      const float gv = ld1(a.qg, a.qg_f, gate0 + (size_t)hq * 2 * kHd + kHd + tid);
      a.out[(size_t)b * a.ld_out + (size_t)hq * kHd + tid] = (o[h] / hl[h]) * sigmoid_f(gv);
    }
    return;
  }
  float* pml = A.part_ml + ((size_t)grpi * A.nchunk + c) * 2 * kMaxRep;
  float* po = A.part_o + ((size_t)grpi * A.nchunk + c) * kMaxRep * kHd;
#pragma unroll
  for (int h = 0; h < kMaxRep; ++h) if (h < rep) st_agent(&po[h * kHd + tid], o[h]);
  if (tid < rep) { st_agent(&pml[tid], hm[tid]); st_agent(&pml[kMaxRep + tid], hl[tid]); }
  if (!arrive_last(&A.counters[grpi], (uint32_t)nact, &flag)) return;
  const float* mlg = A.part_ml + (size_t)grpi * A.nchunk * 2 * kMaxRep;
  const float* og = A.part_o + (size_t)grpi * A.nchunk * kMaxRep * kHd;
  // Merge: wave h turns the chunk maxima / sums of head h into weights w_c = exp(m_c - M)
  // (kept in LDS, reusing ored) and the total L; then every thread merges dim `tid` of all heads
  // in chunk order, 16 chunks of loads in flight.
  float* wts = &ored[0][0][0];  // [kMaxRep][kMaxChunks]
  for (int h = wid; h < rep; h += 4) {
    float M = -INFINITY;
    for (int cc = lane; cc < nact; cc += 64) M = fmaxf(M, ld_agent(&mlg[(size_t)cc * 2 * kMaxRep + h]));
#pragma unroll
    for (int o2 = 32; o2 > 0; o2 >>= 1) M = fmaxf(M, __shfl_xor(M, o2, 64));
    float L = 0.f;
    for (int cc = lane; cc < nact; cc += 64) {
      const float w = expf(ld_agent(&mlg[(size_t)cc * 2 * kMaxRep + h]) - M);
      wts[h * kMaxChunks + cc] = w;
      L += ld_agent(&mlg[(size_t)cc * 2 * kMaxRep + kMaxRep + h]) * w;
    }
    L = wave_sum(L);
    if (lane == 0) hl[h] = L;
  }
  __syncthreads();
  float O[kMaxRep] = {0.f, 0.f, 0.f, 0.f};
  for (int c0 = 0; c0 < nact; c0 += 16) {
    float ov[kMaxRep][16];
#pragma unroll
    for (int h = 0; h < kMaxRep; ++h)
#pragma unroll
      for (int j = 0; j < 16; ++j)
        ov[h][j] = (h < rep && c0 + j < nact) ? ld_agent(&og[((size_t)(c0 + j) * kMaxRep + h) * kHd + tid]) : 0.f;
#pragma unroll
    for (int h = 0; h < kMaxRep; ++h)
#pragma unroll
      for (int j = 0; j < 16; ++j)
        if (h < rep && c0 + j < nact) O[h] += ov[h][j] * wts[h * kMaxChunks + c0 + j];
  }
#pragma unroll
  for (int h = 0; h < kMaxRep; ++h) {
    if (h >= rep) break;
    const int hq = g * rep + h;
    const float gv = ld1(a.qg, a.qg_f, gate0 + (size_t)hq * 2 * kHd + kHd + tid);
    a.out[(size_t)b * a.ld_out + (size_t)hq * kHd + tid] = (O[h] / hl[h]) * sigmoid_f(gv);
  }
}

int pick_chunk(int32_t B, int32_t nkv, int32_t tmax) {
  const long long work = (long long)B * nkv * tmax;
  int ch = 16;
  while (ch < kMaxChunk && work / ch > 512) ch *= 2;
  return ch;
}

struct AttnLayout {
  int chunk, nchunk;
  size_t cnt_bytes, ml_bytes, o_bytes;
};

AttnLayout attn_layout(int32_t B, int32_t nkv, int32_t hd, int32_t tmax) {
  AttnLayout L;
  L.chunk = pick_chunk(B, nkv, tmax);
  L.nchunk = (tmax + L.chunk - 1) / L.chunk;
  const size_t groups = (size_t)B * nkv;
  L.cnt_bytes = kCounterBytes;
  L.ml_bytes = (groups * L.nchunk * 2 * kMaxRep * 4 + 255) & ~(size_t)255;
  L.o_bytes = (groups * L.nchunk * kMaxRep * (size_t)hd * 4 + 255) & ~(size_t)255;
  return L;
}

}  // namespace

size_t attn_ws_bytes(int32_t B, int32_t nh, int32_t nkv, int32_t hd, int32_t tmax) {
  (void)nh;
  AttnLayout L = attn_layout(B, nkv, hd, tmax);
  return L.cnt_bytes + L.ml_bytes + L.o_bytes;
}

int attn_launch(const AttnCall& c, void* ws, size_t ws_bytes, hipStream_t st) {
  if (!ws || ws_bytes < kCounterBytes) return fail(Q35_E_WS, "attention: workspace too small");
  return attn_launch_split(c, ws_counters(ws), ws_scratch(ws), ws_bytes - kCounterBytes, st);
}

int attn_launch_split(const AttnCall& c, uint32_t* counters, char* scratch, size_t scratch_bytes, hipStream_t st) {
  if ((!c.qg && !c.qg_f) || (!c.k && !c.k_f) || (!c.v && !c.v_f) || !c.qnw || !c.knw || !c.rcos || !c.rsin || !c.kc || !c.vc || !c.pos || !c.out)
    return fail(Q35_E_ARG, "attention: null pointer");
  if (c.hd != kHd) return fail(Q35_E_SHAPE, "attention: head_dim must be 256");
  if (c.nkv < 1 || c.nh % c.nkv != 0 || c.nh / c.nkv > kMaxRep)
    return fail(Q35_E_SHAPE, "attention: heads must be a multiple of kv heads, ratio <= 4");
  if (c.rot <= 0 || c.rot > c.hd || (c.rot % 2) != 0) return fail(Q35_E_SHAPE, "attention: bad rotary dim");
  if (c.B < 1 || c.tmax < 1) return fail(Q35_E_SHAPE, "attention: B and tmax must be >= 1");
  if (c.B * c.nkv > kMaxCounters) return fail(Q35_E_SHAPE, "attention: B*kv_heads too large");
  if ((size_t)c.B * c.nkv * c.tmax * c.hd > (size_t)1 << 40) return fail(Q35_E_SHAPE, "attention: cache too large");
  AttnLayout L = attn_layout(c.B, c.nkv, c.hd, c.tmax);
  if (!counters || !scratch || scratch_bytes < L.ml_bytes + L.o_bytes) return fail(Q35_E_WS, "attention: workspace too small");
  if (L.nchunk > kMaxChunks) return fail(Q35_E_SHAPE, "attention: tmax too large for one merge");
  AttnArgs A;
  A.c = c;
  A.scale = (float)(1.0 / sqrt((double)c.hd));
  A.chunk = L.chunk; A.nchunk = L.nchunk;
  A.counters = counters;
  A.part_ml = reinterpret_cast<float*>(scratch);
  A.part_o = reinterpret_cast<float*>(scratch + L.ml_bytes);
  const int grid = c.B * c.nkv * L.nchunk;
  hipLaunchKernelGGL(attn_decode_kernel, dim3(grid), dim3(kThreads), 0, st, A);
  Q35_HIP_TRY(hipGetLastError());
  return Q35_OK;
}

}  // namespace q35
