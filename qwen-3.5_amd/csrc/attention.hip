// Gated GQA attention for one decode token (text_modules.rs:842-944): per-head q/k RMSNorm
// (1+w), partial RoPE on the first rot dims (rotate_half, :739-774), K/V append at the
// current position, softmax(q K^T / sqrt(d)) V over the cache with GQA (q head h reads kv
// head h / (nh/nkv), repeat_kv :776-792) and the sigmoid output gate (:936).
//
// Split-T ("flash decoding") in two kernels:
//  * chunk kernel, block (b, kv head g, chunk c) over `chunk` cached tokens for the rep = nh/nkv
//    query heads of g, so each K/V row is read once for all of them.  Wave w takes tokens
//    w, w+4, ...; a lane owns 4 of the 256 dims (one float4 of every row, 1 KB per wave per row).
//    Every K and V row of a batch of 2 tokens per wave is requested before the first is used,
//    and the next batch's rows before the current batch is computed, so a chunk costs one memory
//    round trip rather than one per token.  Scores feed an online softmax (running max, sum and
//    P.V per head in registers); the 4 waves are combined through LDS.  A block whose chunk is
//    the only one writes the gated output; otherwise it publishes (max, sum, o[rep][256]).
//  * merge kernel, block (b, query head h, 64-dim slice): chunk weights 2^(m_c - M) in LDS (the
//    maxima are kept in log2 units), 4 threads per dim each summing a quarter of the chunks (16
//    loads in flight), then the gate.
// The grids cover tmax, so a captured graph stays valid as the position advances; blocks past
// the current length exit at once.  A position outside [0, tmax) is reported through the
// workspace's error word and its row is left untouched.
#include "q35_internal.h"

namespace q35 {

namespace {

constexpr int kThreads = 256;
constexpr int kNW = kThreads / 64;
constexpr int kHd = 256;
constexpr int kMaxRep = 4;
constexpr int kMinChunk = 16;
constexpr int kMaxChunk = 256;     // tokens per block
constexpr int kMaxChunks = 1024;   // chunks per (b, kv head): the merge keeps their weights in LDS
#ifndef Q35_ATT_BATCH
#define Q35_ATT_BATCH 2
#endif
constexpr int kBatch = Q35_ATT_BATCH;  // tokens per wave per load batch

struct AttnArgs {
  AttnCall c;
  float scale;
  int32_t chunk, nchunk;
  uint32_t* counters;  // counters[kWsErrWord]: the sticky error word
  float* part_ml;      // [B*nkv][nchunk][2][kMaxRep]
  float* part_o;       // [B*nkv][nchunk][kMaxRep][hd]
};

Q35_DEV float4 ld4(const float* f, const fx_t* x, size_t i) {
  if (x) return make_float4(from_fx(x[i]), from_fx(x[i + 1]), from_fx(x[i + 2]), from_fx(x[i + 3]));
  return *reinterpret_cast<const float4*>(f + i);
}
Q35_DEV float ld1(const float* f, const fx_t* x, size_t i) { return x ? from_fx(x[i]) : f[i]; }
Q35_DEV float4 ldf4(const float* p) {
  const uint4 u = ldg16(p);
  return make_float4(__uint_as_float(u.x), __uint_as_float(u.y), __uint_as_float(u.z), __uint_as_float(u.w));
}

Q35_DEV bool pos_ok(const AttnArgs& A, int b, int* pos) {
  *pos = A.c.pos[b];
  return *pos >= 0 && *pos < A.c.tmax;
}

__global__ __launch_bounds__(kThreads) void attn_chunk_kernel(const AttnArgs A) {
  const AttnCall& a = A.c;
  __shared__ __align__(16) float qn[kMaxRep][kHd];
  __shared__ __align__(16) float kn[kHd];
  __shared__ __align__(16) float vn[kHd];
  __shared__ float rtmp[kMaxRep + 1][kHd];
  __shared__ __align__(16) float wo[kNW][kMaxRep][kHd];
  __shared__ float wm[kNW][kMaxRep], wl[kNW][kMaxRep];

  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int c = blockIdx.x % A.nchunk;
  const int g = (blockIdx.x / A.nchunk) % a.nkv;
  const int b = blockIdx.x / (A.nchunk * a.nkv);
  const int rep = a.nh / a.nkv;
  int pos;
  if (!pos_ok(A, b, &pos)) {  // no cache row or rotary row exists for it: report, touch nothing
    if (tid == 0 && c == 0 && g == 0) ws_raise(A.counters, kWsErrPos);
    return;
  }
  const int T = pos + 1;
  const int nact = (T + A.chunk - 1) / A.chunk;
  if (c >= nact) return;
  const int t0 = c * A.chunk;
  const int len = min(A.chunk, T - t0);
  const bool has_new = (c == nact - 1);
  const size_t cache_off = (((size_t)b * a.nkv + g) * a.tmax) * kHd;
  const float* Kc = a.kc + cache_off;
  const float* Vc = a.vc + cache_off;
  // rows of wave wid: t0 + wid + 4 i, i < nw_tok; rows at or past pos (the new token) are not read
  const int nw_tok = (len - wid + kNW - 1) / kNW;
  // two register buffers of kBatch rows each (fixed indices: the batch loop below is unrolled by 2)
  float4 k0b[kBatch], v0b[kBatch], k1b[kBatch], v1b[kBatch];
  auto load_batch = [&](int bi, float4 (&kb)[kBatch], float4 (&vb)[kBatch]) {
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int t = t0 + wid + kNW * (bi * kBatch + u);
      const int tr = max(0, min(t, pos - 1));  // clamped into the cache; masked when used
      kb[u] = ldf4(Kc + (size_t)tr * kHd + 4 * lane);
      vb[u] = ldf4(Vc + (size_t)tr * kHd + 4 * lane);
    }
  };
  const int nbatch = (nw_tok + kBatch - 1) / kBatch;
  if (nbatch > 0) load_batch(0, k0b, v0b);

  // q heads (wave w -> head g*rep + w), plus k/v of the new token in the chunk holding it
  for (int w = wid; w < rep + (has_new ? 2 : 0); w += kNW) {
    const int d = 4 * lane;
    if (w < rep) {
      const int hq = g * rep + w;
      const float4 v = ld4(a.qg, a.qg_f, (size_t)b * a.ld_qg + (size_t)hq * 2 * kHd + d);
      const float r = rsqrt_f(wave_sum(v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w) / (float)kHd + a.eps);
      qn[w][d + 0] = (v.x * r) * (1.0f + a.qnw[d + 0]);
      qn[w][d + 1] = (v.y * r) * (1.0f + a.qnw[d + 1]);
      qn[w][d + 2] = (v.z * r) * (1.0f + a.qnw[d + 2]);
      qn[w][d + 3] = (v.w * r) * (1.0f + a.qnw[d + 3]);
    } else if (w == rep) {
      const float4 v = ld4(a.k, a.k_f, (size_t)b * a.ld_kv + (size_t)g * kHd + d);
      const float r = rsqrt_f(wave_sum(v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w) / (float)kHd + a.eps);
      kn[d + 0] = (v.x * r) * (1.0f + a.knw[d + 0]);
      kn[d + 1] = (v.y * r) * (1.0f + a.knw[d + 1]);
      kn[d + 2] = (v.z * r) * (1.0f + a.knw[d + 2]);
      kn[d + 3] = (v.w * r) * (1.0f + a.knw[d + 3]);
    } else {
      *reinterpret_cast<float4*>(&vn[d]) = ld4(a.v, a.v_f, (size_t)b * a.ld_kv + (size_t)g * kHd + d);
    }
  }
  __syncthreads();
  // RoPE on dims [0, rot): x' = x*cos + rotate_half(x)*sin (computed into rtmp, then copied)
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
  if (has_new) {  // append (post-RoPE k, raw v) at row `pos`
    a.kc[cache_off + (size_t)pos * kHd + tid] = kn[tid];
    a.vc[cache_off + (size_t)pos * kHd + tid] = vn[tid];
  }

  float q4[kMaxRep][4];
#pragma unroll
  for (int h = 0; h < kMaxRep; ++h)
#pragma unroll
    for (int i = 0; i < 4; ++i) q4[h][i] = (h < rep) ? qn[h][4 * lane + i] : 0.f;
  const float4 kn4 = *reinterpret_cast<const float4*>(&kn[4 * lane]);
  const float4 vn4 = *reinterpret_cast<const float4*>(&vn[4 * lane]);
  // online softmax per head: running max m, sum l, and acc = sum p v (this lane's 4 dims)
  float m[kMaxRep], l[kMaxRep], acc[kMaxRep][4];
#pragma unroll
  for (int h = 0; h < kMaxRep; ++h) {
    m[h] = -INFINITY;
    l[h] = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[h][i] = 0.f;
  }
  // Scores are kept in log2 units (scale * log2 e folded in) so that every exponential is one
  // hardware exp2; the running max is updated once per batch of kBatch tokens.
  const float sl2 = A.scale * 1.44269504088896341f;
  auto compute = [&](int bi, const float4 (&kb)[kBatch], const float4 (&vb)[kBatch]) {
    const int nb = min(kBatch, nw_tok - bi * kBatch);  // tokens of this batch (uniform in the wave)
#pragma unroll
    for (int h = 0; h < kMaxRep; ++h) {
      if (h >= rep) break;
      float s[kBatch];
      float bm = -INFINITY;
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const int t = t0 + wid + kNW * (bi * kBatch + u);
        const float4 kv = (t == pos) ? kn4 : kb[u];
        s[u] = (u < nb) ? wave_sum(q4[h][0] * kv.x + q4[h][1] * kv.y + q4[h][2] * kv.z + q4[h][3] * kv.w) * sl2
                        : -INFINITY;
        bm = fmaxf(bm, s[u]);
      }
      const float mn = fmaxf(m[h], bm);
      const float al = __builtin_amdgcn_exp2f(m[h] - mn);  // 0 while m is -inf
      l[h] *= al;
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[h][e] *= al;
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const int t = t0 + wid + kNW * (bi * kBatch + u);
        const float4 vv = (t == pos) ? vn4 : vb[u];
        const float p = __builtin_amdgcn_exp2f(s[u] - mn);  // 0 for the masked slots
        l[h] += p;
        acc[h][0] += p * vv.x;
        acc[h][1] += p * vv.y;
        acc[h][2] += p * vv.z;
        acc[h][3] += p * vv.w;
      }
      m[h] = mn;
    }
  };
  // the next batch's rows are requested before the current batch is computed
  for (int bi = 0; bi < nbatch; bi += 2) {
    if (bi + 1 < nbatch) load_batch(bi + 1, k1b, v1b);
    compute(bi, k0b, v0b);
    if (bi + 1 >= nbatch) break;
    if (bi + 2 < nbatch) load_batch(bi + 2, k0b, v0b);
    compute(bi + 1, k1b, v1b);
  }
  // combine the 4 waves (a wave with no token has m = -inf, weight 0)
#pragma unroll
  for (int h = 0; h < kMaxRep; ++h) {
    if (h >= rep) break;
    *reinterpret_cast<float4*>(&wo[wid][h][4 * lane]) = make_float4(acc[h][0], acc[h][1], acc[h][2], acc[h][3]);
    if (lane == 0) { wm[wid][h] = m[h]; wl[wid][h] = l[h]; }
  }
  __syncthreads();
  const int grpi = b * a.nkv + g;
  float* pml = A.part_ml + ((size_t)grpi * A.nchunk + c) * 2 * kMaxRep;
  float* po = A.part_o + ((size_t)grpi * A.nchunk + c) * kMaxRep * kHd;
#pragma unroll
  for (int h = 0; h < kMaxRep; ++h) {
    if (h >= rep) break;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kNW; ++w) M = fmaxf(M, wm[w][h]);
    float L = 0.f, o = 0.f;
#pragma unroll
    for (int w = 0; w < kNW; ++w) {
      const float e = (wm[w][h] == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(wm[w][h] - M);
      L += wl[w][h] * e;
      o += wo[w][h][tid] * e;
    }
    if (nact == 1) {  // the only chunk: finish here
      const int hq = g * rep + h;
      const float gv = ld1(a.qg, a.qg_f, (size_t)b * a.ld_qg + (size_t)hq * 2 * kHd + kHd + tid);
      a.out[(size_t)b * a.ld_out + (size_t)hq * kHd + tid] = (o / L) * sigmoid_f(gv);
    } else {
      po[h * kHd + tid] = o;
      if (tid == 0) { pml[h] = M; pml[kMaxRep + h] = L; }
    }
  }
}

// Block (b, query head hq, 64-dim slice ds): merges the chunk partials of that slice.
__global__ __launch_bounds__(kThreads) void attn_merge_kernel(const AttnArgs A) {
  const AttnCall& a = A.c;
  __shared__ float wts[kMaxChunks];
  __shared__ float red[kNW][64];
  __shared__ float shm[kNW], shl[kNW];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int nds = kHd / 64;
  const int ds = blockIdx.x % nds;
  const int hq = (blockIdx.x / nds) % a.nh;
  const int b = blockIdx.x / (nds * a.nh);
  const int rep = a.nh / a.nkv, g = hq / rep, hr = hq % rep;
  int pos;
  if (!pos_ok(A, b, &pos)) return;  // reported by the chunk kernel
  const int nact = (pos + A.chunk) / A.chunk;
  if (nact <= 1) return;  // the chunk kernel wrote the output
  const int grpi = b * a.nkv + g;
  const float* ml = A.part_ml + (size_t)grpi * A.nchunk * 2 * kMaxRep;
  const float* og = A.part_o + (size_t)grpi * A.nchunk * kMaxRep * kHd;
  // chunk maxima -> M, weights w_c = exp(m_c - M) (LDS) and L = sum l_c w_c
  float mx = -INFINITY;
  for (int cc = tid; cc < nact; cc += kThreads) mx = fmaxf(mx, ml[(size_t)cc * 2 * kMaxRep + hr]);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
  if (lane == 0) shm[wid] = mx;
  __syncthreads();
  const float M = fmaxf(fmaxf(shm[0], shm[1]), fmaxf(shm[2], shm[3]));
  float ls = 0.f;
  for (int cc = tid; cc < nact; cc += kThreads) {
    const float w = __builtin_amdgcn_exp2f(ml[(size_t)cc * 2 * kMaxRep + hr] - M);  // maxima in log2 units
    wts[cc] = w;
    ls += ml[(size_t)cc * 2 * kMaxRep + kMaxRep + hr] * w;
  }
  ls = wave_sum(ls);
  if (lane == 0) shl[wid] = ls;
  __syncthreads();
  const float L = (shl[0] + shl[1]) + (shl[2] + shl[3]);
  // thread (part = wid, dim = lane): chunks part, part + 4, ... , 16 loads in flight
  const int d = ds * 64 + lane;
  const float* src = og + (size_t)hr * kHd + d;
  float o = 0.f;
  for (int c0 = wid; c0 < nact; c0 += kNW * 16) {
    float v[16], w[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int cc = min(c0 + kNW * j, nact - 1);  // clamped; masked below
      v[j] = src[(size_t)cc * kMaxRep * kHd];
      w[j] = wts[cc];
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) o += (c0 + kNW * j < nact) ? v[j] * w[j] : 0.f;
  }
  red[wid][lane] = o;
  __syncthreads();
  if (tid < 64) {
    const float s = (red[0][tid] + red[1][tid]) + (red[2][tid] + red[3][tid]);
    const float gv = ld1(a.qg, a.qg_f, (size_t)b * a.ld_qg + (size_t)hq * 2 * kHd + kHd + d);
    a.out[(size_t)b * a.ld_out + (size_t)hq * kHd + d] = (s / L) * sigmoid_f(gv);
  }
}

// Tokens per chunk: about 512 chunk blocks over the (b, kv head, tmax) work, 16 .. 256 tokens.
int pick_chunk(int32_t B, int32_t nkv, int32_t tmax) {
  const long long work = (long long)B * nkv * tmax;
  long long ch = (work + 511) / 512;
  ch = (ch + kMinChunk - 1) / kMinChunk * kMinChunk;
  if (ch < kMinChunk) ch = kMinChunk;
  if (ch > kMaxChunk) ch = kMaxChunk;
  return (int)ch;
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
  hipLaunchKernelGGL(attn_chunk_kernel, dim3(c.B * c.nkv * L.nchunk), dim3(kThreads), 0, st, A);
  Q35_HIP_TRY(hipGetLastError());
  if (L.nchunk > 1) {
    hipLaunchKernelGGL(attn_merge_kernel, dim3(c.B * c.nh * (kHd / 64)), dim3(kThreads), 0, st, A);
    Q35_HIP_TRY(hipGetLastError());
  }
  return Q35_OK;
}

}  // namespace q35
