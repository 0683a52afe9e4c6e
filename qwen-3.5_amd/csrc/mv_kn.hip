// Q8F matvec for the reference's projection layout (KN: W[K][N] int8, scale[K][N/64] f32,
// blocks of 64 along N — kernels.rs:53-92,103-165), memory-bound on HBM.
//
// Decomposition: a 256-thread block owns a 256-column tile and a chunk of K rows.  Each lane
// reads 16 consecutive int8 columns of a row with one 16-byte load (16 lanes cover 256 B of a
// row, 16 rows per block step), dequantises in registers with the row's block scale folded
// into x[k] and accumulates 16 columns in f32.  Rows are reduced through LDS, then the K
// chunks of a tile ("splits") are combined by the last block to finish (fixed split order, so
// results are bit-reproducible run to run).  The first weight loads are issued before the
// prologue so their latency overlaps the prologue's reduction over x.
//
// Prologues fold the element-wise producer of x into the kernel: plain, RMSNorm (1+w),
// gated RMSNorm with SiLU(z), SwiGLU, and embedding-lookup + RMSNorm.  Epilogues: store, or
// add into the residual stream.  An optional f32 gate projection (GatedDeltaNet in_proj_b /
// in_proj_a, kernels.rs:174-247) rides in the same launch on extra blocks.
#include "q35_internal.h"

namespace q35 {

namespace {

constexpr int kThreads = 256;
constexpr int kTile = 256;        // columns per tile
constexpr int kRowsPerStep = 16;  // 256 threads / 16 lanes per row
constexpr int kKchMax = 512;      // max rows per block
constexpr int kU = 4;             // rows in flight per lane per step
constexpr int kMaxGroups = 16;    // PRO_GATED groups touched by one block

struct MvArgs {
  MvSeg seg[4];
  int32_t tile0[5];
  int32_t nseg, ntiles, nsplit, kchunk, naux, achunk;
  int32_t K, M;
  int32_t pro, epi;
  const float* x; int32_t ldx;
  const float* x2; int32_t ldx2;
  const float* pw;
  int32_t group, swiglu_off;
  float eps;
  const int8_t* emb_q; const float* emb_s; const int32_t* token; float* h_out;
  const int32_t* prompt; const int32_t* plen; const int32_t* pos;
  const float* aux_wb; const float* aux_wa; const float* aux_alog; const float* aux_dtb;
  int32_t aux_nh; float* aux_out; int32_t aux_ldo;
  uint32_t* counters;  // [ntiles + 1]
  float* partials;     // [ntiles][nsplit][M][256]
  float* aux_part;     // [naux][M][2*aux_nh]
};

// Fills xs[m][0..klen) with the prologue-transformed input rows k0..k0+klen.
template <int MR>
__device__ void mv_prologue(const MvArgs& a, int k0, int klen, float* xs, float* sh, float* grp) {
  const int tid = threadIdx.x;
  float rstat[MR];
#pragma unroll
  for (int m = 0; m < MR; ++m) rstat[m] = 0.f;
  int32_t tok = 0;
  if (a.pro == PRO_EMBED_RMS) {
    tok = *a.token;
    if (a.prompt) {
      const int32_t p = *a.pos;
      if (p < *a.plen) tok = a.prompt[p];
    }
  }
  const int nbK = a.K >> 6;

  if (a.pro == PRO_RMS || a.pro == PRO_EMBED_RMS) {
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      if (m >= a.M) break;
      float ss = 0.f;
      for (int k = tid; k < a.K; k += kThreads) {
        float v;
        if (a.pro == PRO_RMS) v = a.x[(size_t)m * a.ldx + k];
        else v = (float)a.emb_q[(size_t)tok * a.K + k] * a.emb_s[(size_t)tok * nbK + (k >> 6)];
        ss += v * v;
      }
      ss = block_sum256(ss, sh);
      rstat[m] = 1.0f / sqrtf(ss / (float)a.K + a.eps);
    }
  }
  int g0 = 0;
  if (a.pro == PRO_GATED) {
    const int G = a.group;
    g0 = k0 / G;
    const int g1 = (k0 + klen - 1) / G;
    const int lane = tid & 63, wid = tid >> 6;
    for (int gi = g0 + wid; gi <= g1; gi += 4) {
      for (int m = 0; m < a.M; ++m) {
        float ss = 0.f;
        for (int i = lane; i < G; i += 64) {
          float v = a.x[(size_t)m * a.ldx + (size_t)gi * G + i];
          ss += v * v;
        }
        ss = wave_sum(ss);
        if (lane == 0) grp[m * kMaxGroups + (gi - g0)] = 1.0f / sqrtf(ss / (float)G + a.eps);
      }
    }
    __syncthreads();
  }
  for (int i = tid; i < klen; i += kThreads) {
    const int k = k0 + i;
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      float v = 0.f;
      if (m < a.M) {
        switch (a.pro) {
          case PRO_PLAIN: v = a.x[(size_t)m * a.ldx + k]; break;
          case PRO_RMS: v = (a.x[(size_t)m * a.ldx + k] * rstat[m]) * (1.0f + a.pw[k]); break;
          case PRO_EMBED_RMS: {
            float e = (float)a.emb_q[(size_t)tok * a.K + k] * a.emb_s[(size_t)tok * nbK + (k >> 6)];
            v = (e * rstat[m]) * (1.0f + a.pw[k]);
          } break;
          case PRO_GATED: {
            const int G = a.group;
            const float r = grp[m * kMaxGroups + (k / G - g0)];
            const float o = a.x[(size_t)m * a.ldx + k];
            const float z = a.x2[(size_t)m * a.ldx2 + k];
            v = (a.pw[k % G] * (o * r)) * silu_f(z);
          } break;
          case PRO_SWIGLU: {
            const float g = a.x[(size_t)m * a.ldx + k];
            const float u = a.x[(size_t)m * a.ldx + a.swiglu_off + k];
            v = u * silu_f(g);
          } break;
        }
      }
      xs[m * kKchMax + i] = v;
    }
  }
  if (a.pro == PRO_EMBED_RMS && blockIdx.x == 0) {
    for (int k = tid; k < a.K; k += kThreads)
      a.h_out[k] = (float)a.emb_q[(size_t)tok * a.K + k] * a.emb_s[(size_t)tok * nbK + (k >> 6)];
  }
  __syncthreads();
}

template <int MR>
__device__ void mv_aux_block(const MvArgs& a, int ab, float* xs, float* red, float* sh, float* grp, int* flag) {
  const int tid = threadIdx.x;
  const int k0 = ab * a.achunk;
  const int klen = min(a.achunk, a.K - k0);
  mv_prologue<MR>(a, k0, klen, xs, sh, grp);
  const int nh = a.aux_nh, nout = 2 * nh, subs = kThreads / nout;
  const int o = tid % nout, sub = tid / nout;
  const int h = o % nh;
  const float* W = (o < nh) ? a.aux_wb : a.aux_wa;
  for (int m = 0; m < a.M; ++m) {
    float acc = 0.f;
    for (int i = sub; i < klen; i += subs) acc += xs[m * kKchMax + i] * W[(size_t)(k0 + i) * nh + h];
    red[sub * nout + o] = acc;
    __syncthreads();
    if (tid < nout) {
      float s = 0.f;
      for (int j = 0; j < subs; ++j) s += red[j * nout + tid];
      a.aux_part[((size_t)ab * a.M + m) * nout + tid] = s;
    }
    __syncthreads();
  }
  if (!arrive_last(&a.counters[a.ntiles], (uint32_t)a.naux, flag)) return;
  if (tid < nout) {
    for (int m = 0; m < a.M; ++m) {
      float s = 0.f;
      for (int j = 0; j < a.naux; ++j) s += a.aux_part[((size_t)j * a.M + m) * nout + tid];
      float out;
      if (tid < nh) {
        out = 1.0f / (1.0f + expf(-s));
      } else {
        const float xg = s + a.aux_dtb[h];
        const float pre = logf(expf(xg) + 1.0f);
        const float sp = pre > 20.0f ? xg : pre;
        out = -expf(a.aux_alog[h]) * sp;
      }
      a.aux_out[(size_t)m * a.aux_ldo + tid] = out;
    }
  }
}

template <int MR>
__global__ __launch_bounds__(kThreads) void mv_kn_kernel(const MvArgs a) {
  __shared__ __align__(16) float xs[MR * kKchMax];
  __shared__ __align__(16) float red[kRowsPerStep * kTile];
  __shared__ float sh[4];
  __shared__ float grp[MR * kMaxGroups];
  __shared__ int flag;

  const int tid = threadIdx.x;
  const int nmain = a.ntiles * a.nsplit;
  if ((int)blockIdx.x >= nmain) {
    mv_aux_block<MR>(a, (int)blockIdx.x - nmain, xs, red, sh, grp, &flag);
    return;
  }
  const int tile = blockIdx.x / a.nsplit;
  const int split = blockIdx.x - tile * a.nsplit;
  int s = 0;
  while (s + 1 < a.nseg && tile >= a.tile0[s + 1]) ++s;
  const MvSeg seg = a.seg[s];
  const int n0 = (tile - a.tile0[s]) * kTile;
  const int k0 = split * a.kchunk;
  const int klen = min(a.kchunk, a.K - k0);

  const int cg = tid & 15, rr = tid >> 4;
  const int ncol = n0 + cg * 16;
  const bool colok = ncol < seg.N;
  const size_t N = (size_t)seg.N;
  const int nb = seg.N >> 6;
  const int8_t* wbase = seg.w + (size_t)k0 * N + (colok ? ncol : 0);
  const float* sbase = seg.s + (size_t)k0 * nb + (colok ? (ncol >> 6) : 0);

  uint4 wv[kU];
  float sv[kU];
#pragma unroll
  for (int u = 0; u < kU; ++u) {
    const int r = rr + kRowsPerStep * u;
    const bool ok = colok && r < klen;
    wv[u] = ok ? *reinterpret_cast<const uint4*>(wbase + (size_t)r * N) : make_uint4(0, 0, 0, 0);
    sv[u] = ok ? sbase[(size_t)r * nb] : 0.f;
  }

  mv_prologue<MR>(a, k0, klen, xs, sh, grp);

  float acc[MR][16];
#pragma unroll
  for (int m = 0; m < MR; ++m)
#pragma unroll
    for (int j = 0; j < 16; ++j) acc[m][j] = 0.f;

  for (int r0 = 0; r0 < klen; r0 += kRowsPerStep * kU) {
    uint4 wn[kU];
    float sn[kU];
    const bool more = r0 + kRowsPerStep * kU < klen;
    if (more) {
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        const int r = r0 + kRowsPerStep * kU + rr + kRowsPerStep * u;
        const bool ok = colok && r < klen;
        wn[u] = ok ? *reinterpret_cast<const uint4*>(wbase + (size_t)r * N) : make_uint4(0, 0, 0, 0);
        sn[u] = ok ? sbase[(size_t)r * nb] : 0.f;
      }
    }
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int r = r0 + rr + kRowsPerStep * u;
      float f[16];
      unpack16(wv[u], f);
#pragma unroll
      for (int m = 0; m < MR; ++m) {
        const float c = (r < klen) ? xs[m * kKchMax + r] * sv[u] : 0.f;
#pragma unroll
        for (int j = 0; j < 16; ++j) acc[m][j] += f[j] * c;
      }
    }
    if (more) {
#pragma unroll
      for (int u = 0; u < kU; ++u) { wv[u] = wn[u]; sv[u] = sn[u]; }
    }
  }

  // reduce the 16 row groups of the block: column tid of the tile
  float colsum[MR];
#pragma unroll
  for (int m = 0; m < MR; ++m) {
    float4* dst = reinterpret_cast<float4*>(&red[rr * kTile + cg * 16]);
#pragma unroll
    for (int q = 0; q < 4; ++q)
      dst[q] = make_float4(acc[m][q * 4 + 0], acc[m][q * 4 + 1], acc[m][q * 4 + 2], acc[m][q * 4 + 3]);
    __syncthreads();
    float v = 0.f;
#pragma unroll
    for (int i = 0; i < kRowsPerStep; ++i) v += red[i * kTile + tid];
    colsum[m] = v;
    __syncthreads();
  }

  const int n = n0 + tid;
  const bool nok = n < seg.N;
  if (a.nsplit > 1) {
#pragma unroll
    for (int m = 0; m < MR; ++m)
      if (m < a.M) a.partials[(((size_t)tile * a.nsplit + split) * a.M + m) * kTile + tid] = colsum[m];
    if (!arrive_last(&a.counters[tile], (uint32_t)a.nsplit, &flag)) return;
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      if (m >= a.M) break;
      float t = 0.f;
      for (int sp = 0; sp < a.nsplit; ++sp)
        t += a.partials[(((size_t)tile * a.nsplit + sp) * a.M + m) * kTile + tid];
      colsum[m] = t;
    }
  }
  if (nok) {
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      if (m >= a.M) break;
      float* yp = seg.y + (size_t)m * seg.ldy + n;
      if (a.epi == EPI_RESID) *yp = *yp + colsum[m];
      else *yp = colsum[m];
    }
  }
}

struct MvPlan {
  int ntiles = 0, nsplit = 1, kchunk = 0, naux = 0, achunk = 0;
  int tile0[5] = {0, 0, 0, 0, 0};
  size_t counters_bytes = 0, part_bytes = 0, aux_bytes = 0;
};

MvPlan make_plan(const MvCall& c) {
  MvPlan p;
  int t = 0;
  for (int s = 0; s < c.nseg; ++s) {
    p.tile0[s] = t;
    t += (c.seg[s].N + kTile - 1) / kTile;
  }
  p.tile0[c.nseg] = t;
  p.ntiles = t;
  if (p.ntiles > 0) {
    const int target = 640;  // blocks per launch: ~2.5 per CU on 256 CUs
    int nsplit = (target + p.ntiles - 1) / p.ntiles;
    const int maxsplit = (c.K + 31) / 32;
    if (nsplit > maxsplit) nsplit = maxsplit;
    if (nsplit < 1) nsplit = 1;
    int kch = (c.K + nsplit - 1) / nsplit;
    kch = (kch + 15) & ~15;
    if (kch > kKchMax) kch = kKchMax;
    p.kchunk = kch;
    p.nsplit = (c.K + kch - 1) / kch;
  }
  if (c.aux_nh > 0) {
    p.achunk = 256;
    p.naux = (c.K + p.achunk - 1) / p.achunk;
  }
  p.counters_bytes = kCounterBytes;
  p.part_bytes = p.nsplit > 1 ? align256((size_t)p.ntiles * p.nsplit * c.M * kTile * sizeof(float)) : 0;
  p.aux_bytes = p.naux > 0 ? align256((size_t)p.naux * c.M * 2 * c.aux_nh * sizeof(float)) : 0;
  return p;
}

}  // namespace

size_t mv_kn_ws_bytes(const MvCall& c) {
  MvPlan p = make_plan(c);
  return p.counters_bytes + p.part_bytes + p.aux_bytes;
}

int mv_kn_launch(const MvCall& c, void* ws, size_t ws_bytes, hipStream_t st) {
  if (c.K <= 0 || c.M < 1 || c.M > 8) return fail(Q35_E_SHAPE, "mv_kn: K must be > 0 and M in [1,8]");
  if (c.nseg < 0 || c.nseg > 4) return fail(Q35_E_ARG, "mv_kn: 0..4 segments");
  for (int s = 0; s < c.nseg; ++s) {
    const MvSeg& g = c.seg[s];
    if (!g.w || !g.s || !g.y) return fail(Q35_E_ARG, "mv_kn: null segment pointer");
    if (g.N <= 0 || (g.N % 64) != 0) return fail(Q35_E_SHAPE, "mv_kn: N must be a positive multiple of 64");
    if ((reinterpret_cast<uintptr_t>(g.w) & 15) != 0) return fail(Q35_E_ALIGN, "mv_kn: weights not 16-byte aligned");
  }
  if (c.nseg == 0 && c.aux_nh == 0) return fail(Q35_E_ARG, "mv_kn: nothing to compute");
  if (c.aux_nh > 0) {
    if (!c.aux_wb || !c.aux_wa || !c.aux_alog || !c.aux_dtb || !c.aux_out) return fail(Q35_E_ARG, "mv_kn: null gate-projection pointer");
    if (2 * c.aux_nh > kThreads || (kThreads % (2 * c.aux_nh)) != 0)
      return fail(Q35_E_SHAPE, "gate projection: 2*n_heads must divide 256");
  }
  if (c.pro == PRO_GATED) {
    if (c.group <= 0 || (c.K % c.group) != 0) return fail(Q35_E_SHAPE, "mv_kn: gated-norm group must divide K");
    if (kKchMax / c.group + 2 > kMaxGroups) return fail(Q35_E_SHAPE, "mv_kn: gated-norm group too small");
    if (!c.x2 || !c.pw) return fail(Q35_E_ARG, "mv_kn: gated-norm needs z and weight");
  }
  if ((c.pro == PRO_RMS || c.pro == PRO_EMBED_RMS) && !c.pw) return fail(Q35_E_ARG, "mv_kn: RMSNorm needs weight");
  if (c.pro == PRO_EMBED_RMS && (c.M != 1 || !c.emb_q || !c.emb_s || !c.token || !c.h_out))
    return fail(Q35_E_ARG, "mv_kn: embedding prologue needs M==1, table, token, h_out");
  if (c.pro != PRO_EMBED_RMS && !c.x) return fail(Q35_E_ARG, "mv_kn: null x");
  MvPlan p = make_plan(c);
  const size_t need = p.counters_bytes + p.part_bytes + p.aux_bytes;
  if (!ws || ws_bytes < need) return fail(Q35_E_WS, "mv_kn: workspace too small");
  if (c.aux_nh > 0 && p.achunk > kKchMax) return fail(Q35_E_SHAPE, "mv_kn: aux chunk");
  if (p.ntiles + 1 > kMaxCounters) return fail(Q35_E_SHAPE, "mv_kn: too many column tiles");

  MvArgs a;
  for (int s = 0; s < 4; ++s) a.seg[s] = (s < c.nseg) ? c.seg[s] : MvSeg{nullptr, nullptr, nullptr, 0, 0};
  for (int s = 0; s < 5; ++s) a.tile0[s] = p.tile0[s];
  a.nseg = c.nseg; a.ntiles = p.ntiles; a.nsplit = p.nsplit; a.kchunk = p.kchunk;
  a.naux = p.naux; a.achunk = p.achunk;
  a.K = c.K; a.M = c.M; a.pro = c.pro; a.epi = c.epi;
  a.x = c.x; a.ldx = c.ldx; a.x2 = c.x2; a.ldx2 = c.ldx2; a.pw = c.pw; a.group = c.group; a.swiglu_off = c.swiglu_off;
  a.eps = c.eps;
  a.emb_q = c.emb_q; a.emb_s = c.emb_s; a.token = c.token; a.h_out = c.h_out;
  a.prompt = c.prompt; a.plen = c.plen; a.pos = c.pos;
  if (c.prompt && (!c.plen || !c.pos)) return fail(Q35_E_ARG, "mv_kn: device prompt needs plen and pos");
  a.aux_wb = c.aux_wb; a.aux_wa = c.aux_wa; a.aux_alog = c.aux_alog; a.aux_dtb = c.aux_dtb;
  a.aux_nh = c.aux_nh; a.aux_out = c.aux_out; a.aux_ldo = c.aux_ldo;
  char* base = static_cast<char*>(ws);
  a.counters = reinterpret_cast<uint32_t*>(base);
  a.partials = reinterpret_cast<float*>(base + p.counters_bytes);
  a.aux_part = reinterpret_cast<float*>(base + p.counters_bytes + p.part_bytes);

  const int nblocks = p.ntiles * p.nsplit + p.naux;
  const dim3 grid(nblocks), block(kThreads);
  if (c.M == 1) hipLaunchKernelGGL(mv_kn_kernel<1>, grid, block, 0, st, a);
  else if (c.M == 2) hipLaunchKernelGGL(mv_kn_kernel<2>, grid, block, 0, st, a);
  else if (c.M <= 4) hipLaunchKernelGGL(mv_kn_kernel<4>, grid, block, 0, st, a);
  else hipLaunchKernelGGL(mv_kn_kernel<8>, grid, block, 0, st, a);
  Q35_HIP_TRY(hipGetLastError());
  return Q35_OK;
}

size_t gate_proj_ws_bytes(int32_t B, int32_t in_dim, int32_t nh) {
  MvCall c;
  c.K = in_dim; c.M = B < 8 ? B : 8; c.aux_nh = nh;
  return mv_kn_ws_bytes(c);
}

int gate_proj_launch(const float* x, int32_t B, int32_t in_dim, const float* wb, const float* wa,
                     const float* alog, const float* dtb, int32_t nh, float* out, void* ws,
                     size_t ws_bytes, hipStream_t st) {
  for (int b0 = 0; b0 < B; b0 += 8) {
    MvCall c;
    c.K = in_dim; c.M = (B - b0) < 8 ? (B - b0) : 8;
    c.pro = PRO_PLAIN; c.x = x + (size_t)b0 * in_dim; c.ldx = in_dim;
    c.aux_wb = wb; c.aux_wa = wa; c.aux_alog = alog; c.aux_dtb = dtb; c.aux_nh = nh;
    c.aux_out = out + (size_t)b0 * 2 * nh; c.aux_ldo = 2 * nh;
    int rc = mv_kn_launch(c, ws, ws_bytes, st);
    if (rc != Q35_OK) return rc;
  }
  return Q35_OK;
}

}  // namespace q35
