// Q8F matvec for the reference's projection layout (KN: W[K][N] int8, scale[K][N/64] f32,
// blocks of 64 along N — kernels.rs:53-92,103-165), memory-bound on HBM.
//
// Decomposition: a 256-thread block owns a 256-column tile and a chunk of at most 256 K rows.
// Each lane reads 16 consecutive int8 columns of a row with one 16-byte load (16 lanes cover
// 256 B of a row, 16 rows per block step); for M == 1 all 16 row steps of the block are
// requested before the prologue runs, so the whole 64 KB chunk is in flight at once.  Values
// are dequantised in registers with the row's block scale folded into x[k] and accumulated
// over 16 columns in f32; the 16 row groups are reduced through LDS; the block's column sums
// are then added to the output with 64-bit fixed-point atomics (see fx_add), which combine
// the K chunks ("splits") of a tile without any cross-block wait and deterministically.
//
// Prologues fold the element-wise producer of x into the kernel: plain, RMSNorm (1+w),
// gated RMSNorm with SiLU(z), SwiGLU, and embedding-lookup + RMSNorm; inputs may be f32 or a
// fixed-point accumulator left by the previous kernel.  The output accumulator is either zero
// (a plain projection) or the residual stream itself (residual add for free).  Optional side
// tasks ride along: the f32 gate projection of GatedDeltaNet (in_proj_b / in_proj_a,
// kernels.rs:174-247) on extra blocks, zeroing an accumulator for a later kernel, and
// advancing the causal-conv state after the DeltaNet step has consumed it.
#include "q35_internal.h"

namespace q35 {

namespace {

constexpr int kThreads = 256;
constexpr int kTile = 256;        // columns per tile
constexpr int kRowsPerStep = 16;  // 256 threads / 16 lanes per row
constexpr int kKchMax = 256;      // max rows per block
// rows each lane keeps in flight: all 16 row steps of a block for M == 1, fewer when the
// M accumulator sets need the registers
template <int MR> constexpr int kRowsInFlight = MR == 1 ? 16 : (MR == 2 ? 8 : 4);
constexpr int kMaxGroups = 16;    // PRO_GATED groups touched by one block
#ifndef Q35_MV_TARGET
#define Q35_MV_TARGET 256
#endif
#ifndef Q35_MV_MIN_ROWS
#define Q35_MV_MIN_ROWS 32
#endif
constexpr int kTargetBlocks = Q35_MV_TARGET;  // blocks per launch (256 CUs)
constexpr int kMinRows = Q35_MV_MIN_ROWS;      // fewest K rows per block
constexpr int kAuxRows = 256;                  // K rows per gate-projection block
constexpr int kRmsPerThread = 32;              // RMSNorm prologues: K <= 256 * 32

struct MvArgs {
  MvSeg seg[4];
  int32_t tile0[5];
  int32_t nseg, ntiles, nsplit, kchunk, naux;
  int32_t K, M, pro;
  const float* x; const fx_t* xf; int32_t ldx;
  const float* x2; const fx_t* x2f; int32_t ldx2;
  const float* pw;
  int32_t group, swiglu_off;
  float eps;
  const int8_t* emb_q; const float* emb_s; const int32_t* token; fx_t* h_out;
  const int32_t* prompt; const int32_t* plen; const int32_t* pos;
  const float* aux_wb; const float* aux_wa; int32_t aux_nh; fx_t* aux_acc; int32_t aux_ldo;
  fx_t* zero_ptr; int64_t zero_n;
  float* cs_state; const fx_t* cs_x; int32_t cs_ch, cs_ldx, cs_B;
  float* y_out; int32_t ldy; uint32_t* tile_ctr;
  uint32_t* err;
};

Q35_DEV float in1(const MvArgs& a, int m, int k) {
  const size_t i = (size_t)m * a.ldx + k;
  return a.xf ? from_fx(a.xf[i]) : a.x[i];
}
Q35_DEV float in2(const MvArgs& a, int m, int k) {
  const size_t i = (size_t)m * a.ldx2 + k;
  return a.x2f ? from_fx(a.x2f[i]) : a.x2[i];
}

// Side tasks, spread over every block of the launch.
__device__ void mv_side_tasks(const MvArgs& a) {
  const int64_t gt = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  const int64_t gs = (int64_t)gridDim.x * kThreads;
  for (int64_t i = gt; i < a.zero_n; i += gs) a.zero_ptr[i] = 0;
  if (a.cs_state) {
    const int64_t n = (int64_t)a.cs_B * a.cs_ch;
    for (int64_t i = gt; i < n; i += gs) {  // conv state [B][ch][3] <- [s1, s2, x]
      const int64_t b = i / a.cs_ch, c = i % a.cs_ch;
      float* st = a.cs_state + i * 3;
      const float s1 = st[1], s2 = st[2];
      st[0] = s1; st[1] = s2; st[2] = from_fx(a.cs_x[b * a.cs_ldx + c]);
    }
  }
}

// Fills xs[m][0..klen) with the prologue-transformed input rows k0..k0+klen.
template <int MR>
__device__ void mv_prologue(const MvArgs& a, int k0, int klen, float* xs, float* sh, float* grp) {
  const int tid = threadIdx.x;
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
    // thread t holds x[t + 256 j]: all loads of the row are issued at once, then the same
    // registers feed the block's slice of xs (one round trip to memory for the prologue)
    // (a runtime row loop: unrolled over MR rows with an early exit, the multi-row kernels kept
    // the rows' registers in private memory)
    for (int m = 0; m < (MR == 1 ? 1 : a.M); ++m) {
      float v[kRmsPerThread];
#pragma unroll
      for (int j = 0; j < kRmsPerThread; ++j) {
        const int k = tid + kThreads * j;
        float e = 0.f;
        if (k < a.K) {
          if (a.pro == PRO_RMS) e = in1(a, m, k);
          else e = (float)a.emb_q[(size_t)tok * a.K + k] * a.emb_s[(size_t)tok * nbK + (k >> 6)];
        }
        v[j] = e;
      }
      float ss = 0.f;
#pragma unroll
      for (int j = 0; j < kRmsPerThread; ++j) ss += v[j] * v[j];
      ss = block_sum256(ss, sh);
      const float r = rsqrt_f(ss / (float)a.K + a.eps);
#pragma unroll
      for (int j = 0; j < kRmsPerThread; ++j) {
        const int k = tid + kThreads * j;
        if (k >= k0 && k < k0 + klen) xs[m * kKchMax + (k - k0)] = (v[j] * r) * (1.0f + a.pw[k]);
      }
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
          const float v = in1(a, m, gi * G + i);
          ss += v * v;
        }
        ss = wave_sum(ss);
        if (lane == 0) grp[m * kMaxGroups + (gi - g0)] = rsqrt_f(ss / (float)G + a.eps);
      }
    }
    __syncthreads();
  }
  const bool filled = (a.pro == PRO_RMS || a.pro == PRO_EMBED_RMS);
  for (int i = tid; i < klen; i += kThreads) {
    const int k = k0 + i;
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      if (filled && m < a.M) continue;  // written from the statistics registers above
      float v = 0.f;
      if (m < a.M) {
        switch (a.pro) {
          case PRO_PLAIN: v = in1(a, m, k); break;
          case PRO_GATED: {
            const int G = a.group;
            const float r = grp[m * kMaxGroups + (k / G - g0)];
            v = (a.pw[k % G] * (in1(a, m, k) * r)) * silu_f(in2(a, m, k));
          } break;
          case PRO_SWIGLU: v = in1(a, m, a.swiglu_off + k) * silu_f(in1(a, m, k)); break;
        }
      }
      xs[m * kKchMax + i] = v;
    }
  }
  if (a.pro == PRO_EMBED_RMS && blockIdx.x == 0) {
    for (int k = tid; k < a.K; k += kThreads)
      a.h_out[k] = to_fx((float)a.emb_q[(size_t)tok * a.K + k] * a.emb_s[(size_t)tok * nbK + (k >> 6)]);
  }
  __syncthreads();
}

// Gate projection block: raw sums x.W_b[:, h], x.W_a[:, h] over this block's K rows, added to
// aux_acc; the DeltaNet step applies sigmoid / -exp(A_log)*softplus(. + dt_bias).
template <int MR>
__device__ void mv_aux_block(const MvArgs& a, int ab, float* xs, float* red, float* sh, float* grp) {
  const int tid = threadIdx.x;
  const int k0 = ab * kAuxRows;
  const int klen = min(kAuxRows, a.K - k0);
  // thread t owns head column h = t % nh and rows rg, rg + groups, ...; a row of W_b / W_a is
  // nh contiguous floats, so nh neighbouring threads read it together.  The first 16 rows of
  // both matrices are requested before the prologue.
  const int nh = a.aux_nh, groups = kThreads / nh;
  const int h = tid % nh, rg = tid / nh;
  const int nrow = (klen + groups - 1) / groups;
  constexpr int J = MR >= 4 ? 8 : 16;
  float wb[J], wa[J];
  auto load = [&](int j0) {
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int r = rg + groups * (j0 + j);
      const bool ok = (j0 + j) < nrow && r < klen;
      wb[j] = ok ? a.aux_wb[(size_t)(k0 + r) * nh + h] : 0.f;
      wa[j] = ok ? a.aux_wa[(size_t)(k0 + r) * nh + h] : 0.f;
    }
  };
  load(0);
  mv_prologue<MR>(a, k0, klen, xs, sh, grp);
  float accb[MR], acca[MR];
#pragma unroll
  for (int m = 0; m < MR; ++m) { accb[m] = 0.f; acca[m] = 0.f; }
  for (int j0 = 0; j0 < nrow; j0 += J) {
    if (j0 > 0) load(j0);
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int r = rg + groups * (j0 + j);
      if ((j0 + j) < nrow && r < klen) {
#pragma unroll
        for (int m = 0; m < MR; ++m) {
          const float xv = xs[m * kKchMax + r];
          accb[m] += xv * wb[j];
          acca[m] += xv * wa[j];
        }
      }
    }
  }
  const int nout = 2 * nh;
#pragma unroll
  for (int m = 0; m < MR; ++m) {
    if (m < a.M) {  // uniform: every thread takes the same branch
      red[rg * nout + h] = accb[m];
      red[rg * nout + nh + h] = acca[m];
      __syncthreads();
      if (tid < nout) {
        float s = 0.f;
        for (int g = 0; g < groups; ++g) s += red[g * nout + tid];
        fx_add_chk(&a.aux_acc[(size_t)m * a.aux_ldo + tid], s, a.err);
      }
      __syncthreads();
    }
  }
}

template <int MR>
__global__ __launch_bounds__(kThreads) void mv_kn_kernel(const MvArgs a) {
  __shared__ __align__(16) float xs[MR * kKchMax];
  __shared__ __align__(16) float red[kRowsPerStep * kTile];
  __shared__ float sh[4];
  __shared__ float grp[MR * kMaxGroups];
  __shared__ int last_flag;

  const int tid = threadIdx.x;
  const int nmain = a.ntiles * a.nsplit;
  if ((int)blockIdx.x >= nmain) {
    mv_side_tasks(a);
    mv_aux_block<MR>(a, (int)blockIdx.x - nmain, xs, red, sh, grp);
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
  // row strides: N bytes / N/64 scales (row-major), or 256 / 4 inside a tile (tiled layout,
  // where the block's K chunk of its tile is one contiguous run)
  const size_t N = seg.tiled ? (size_t)kTile : (size_t)seg.N;
  const int nb = seg.tiled ? kTile / 64 : (seg.N >> 6);
  const int tl = tile - a.tile0[s];
  const int8_t* wbase = seg.tiled ? seg.w + ((size_t)tl * a.K + k0) * kTile + cg * 16
                                  : seg.w + (size_t)k0 * N + (colok ? ncol : 0);
  const float* sbase = seg.tiled ? seg.s + ((size_t)tl * a.K + k0) * (kTile / 64) + (cg >> 2)
                                 : seg.s + (size_t)k0 * nb + (colok ? (ncol >> 6) : 0);

  // All of a block's rows (up to 16 per lane for M == 1) are requested before the prologue,
  // so the whole weight chunk is in flight while x is being prepared.
  constexpr int U = kRowsInFlight<MR>;
  // (M == 1 keeps every row in flight in uint4 registers; the multi-row kernels use native
  // vectors, which the compiler keeps in registers across the loop)
  using WV = std::conditional_t<MR == 1, uint4, q35_u32x4>;
  WV wv[U];
  float sv[U];
  auto load_batch = [&](int r0) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int r = r0 + rr + kRowsPerStep * u;
      const bool ok = colok && r < klen;
      if constexpr (MR == 1) wv[u] = ok ? ldg16_nt(wbase + (size_t)r * N) : make_uint4(0, 0, 0, 0);
      else wv[u] = ok ? ldg16v_nt(wbase + (size_t)r * N) : q35_u32x4{0u, 0u, 0u, 0u};
      sv[u] = ok ? ldg_nt(sbase + (size_t)r * nb) : 0.f;
    }
  };
  load_batch(0);

  mv_side_tasks(a);
  mv_prologue<MR>(a, k0, klen, xs, sh, grp);

  float acc[MR][16];
#pragma unroll
  for (int m = 0; m < MR; ++m)
#pragma unroll
    for (int j = 0; j < 16; ++j) acc[m][j] = 0.f;

  for (int r0 = 0; r0 < klen; r0 += kRowsPerStep * U) {
    if (r0 > 0) load_batch(r0);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int r = r0 + rr + kRowsPerStep * u;
      if (r0 + kRowsPerStep * u >= klen) break;
      float f[16];
      if constexpr (MR == 1) unpack16(wv[u], f);
      else unpack16v(wv[u], f);
#pragma unroll
      for (int m = 0; m < MR; ++m) {
        const float c = (r < klen) ? xs[m * kKchMax + r] * sv[u] : 0.f;
#pragma unroll
        for (int j = 0; j < 16; ++j) acc[m][j] += f[j] * c;
      }
    }
  }

  // reduce the 16 row groups of the block (column tid of the tile), add to the output
  const int n = n0 + tid;
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
    if (m < a.M && n < seg.N) fx_add_chk(&seg.acc[(size_t)m * seg.ldacc + n], v, a.err);
    __syncthreads();
  }
  // f32 output: the last block of the tile to finish (its adds and every earlier block's are
  // complete once the counter says so) converts the tile's sums and re-zeroes them
  if (!a.y_out) return;
  if (!arrive_last(&a.tile_ctr[tile], (uint32_t)a.nsplit, &last_flag)) return;
  if (n < seg.N) {
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      if (m >= a.M) break;
      fx_t* p = &seg.acc[(size_t)m * seg.ldacc + n];
      a.y_out[(size_t)m * a.ldy + n] = from_fx(ld_agent(p));
      st_agent(p, (fx_t)0);
    }
  }
}

struct MvPlan {
  int ntiles = 0, nsplit = 1, kchunk = 0, naux = 0;
  int tile0[5] = {0, 0, 0, 0, 0};
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
    int nsplit = (kTargetBlocks + p.ntiles - 1) / p.ntiles;
    const int maxsplit = (c.K + kMinRows - 1) / kMinRows;
    if (nsplit > maxsplit) nsplit = maxsplit;
    const int minsplit = (c.K + kKchMax - 1) / kKchMax;
    if (nsplit < minsplit) nsplit = minsplit;
    if (nsplit < 1) nsplit = 1;
    int kch = (c.K + nsplit - 1) / nsplit;
    kch = (kch + 15) & ~15;
    if (kch > kKchMax) kch = kKchMax;
    p.kchunk = kch;
    p.nsplit = (c.K + kch - 1) / kch;
  }
  if (c.aux_nh > 0) p.naux = (c.K + kAuxRows - 1) / kAuxRows;
  return p;
}

__global__ __launch_bounds__(kThreads) void fx_to_f32_kernel(fx_t* acc, int64_t n, float* y, int zero_after) {
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads) {
    y[i] = from_fx(acc[i]);
    if (zero_after) acc[i] = 0;
  }
}

__global__ __launch_bounds__(kThreads) void fx_zero_kernel(fx_t* acc, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads)
    acc[i] = 0;
}

int grid_for(int64_t n) {
  int64_t g = (n + kThreads - 1) / kThreads;
  if (g > 1024) g = 1024;
  return g < 1 ? 1 : (int)g;
}

}  // namespace

int mv_kn_launch(const MvCall& c, hipStream_t st) {
  if (c.K <= 0 || c.M < 1 || c.M > 8) return fail(Q35_E_SHAPE, "mv_kn: K must be > 0 and M in [1,8]");
  if (c.nseg < 0 || c.nseg > 4) return fail(Q35_E_ARG, "mv_kn: 0..4 segments");
  for (int s = 0; s < c.nseg; ++s) {
    const MvSeg& g = c.seg[s];
    if (!g.w || !g.s || !g.acc) return fail(Q35_E_ARG, "mv_kn: null segment pointer");
    if (g.N <= 0 || (g.N % 64) != 0) return fail(Q35_E_SHAPE, "mv_kn: N must be a positive multiple of 64");
    if ((reinterpret_cast<uintptr_t>(g.w) & 15) != 0) return fail(Q35_E_ALIGN, "mv_kn: weights not 16-byte aligned");
  }
  if (c.nseg == 0 && c.aux_nh == 0) return fail(Q35_E_ARG, "mv_kn: nothing to compute");
  if (!c.err) return fail(Q35_E_ARG, "mv_kn: null error word");
  if (c.aux_nh > 0) {
    if (!c.aux_wb || !c.aux_wa || !c.aux_acc) return fail(Q35_E_ARG, "mv_kn: null gate-projection pointer");
    if (2 * c.aux_nh > kThreads || (kThreads % (2 * c.aux_nh)) != 0)
      return fail(Q35_E_SHAPE, "gate projection: 2*n_heads must divide 256");
  }
  if (c.pro == PRO_GATED) {
    if (c.group <= 0 || (c.K % c.group) != 0) return fail(Q35_E_SHAPE, "mv_kn: gated-norm group must divide K");
    if (kKchMax / c.group + 2 > kMaxGroups) return fail(Q35_E_SHAPE, "mv_kn: gated-norm group too small");
    if ((!c.x2 && !c.x2f) || !c.pw) return fail(Q35_E_ARG, "mv_kn: gated-norm needs z and weight");
  }
  if ((c.pro == PRO_RMS || c.pro == PRO_EMBED_RMS) && !c.pw) return fail(Q35_E_ARG, "mv_kn: RMSNorm needs weight");
  if ((c.pro == PRO_RMS || c.pro == PRO_EMBED_RMS) && c.K > kThreads * kRmsPerThread)
    return fail(Q35_E_SHAPE, "mv_kn: RMSNorm prologue needs K <= 8192");
  if (c.pro == PRO_EMBED_RMS && (c.M != 1 || !c.emb_q || !c.emb_s || !c.token || !c.h_out))
    return fail(Q35_E_ARG, "mv_kn: embedding prologue needs M==1, table, token, h_out");
  if (c.pro == PRO_EMBED_RMS && c.prompt && (!c.plen || !c.pos))
    return fail(Q35_E_ARG, "mv_kn: device prompt needs plen and pos");
  if (c.pro != PRO_EMBED_RMS && !c.x && !c.xf) return fail(Q35_E_ARG, "mv_kn: null x");
  if (c.zero_n > 0 && !c.zero_ptr) return fail(Q35_E_ARG, "mv_kn: null zero_ptr");
  if (c.cs_state && (!c.cs_x || c.cs_ch <= 0 || c.cs_B <= 0)) return fail(Q35_E_ARG, "mv_kn: bad conv-shift task");
  MvPlan p = make_plan(c);

  MvArgs a;
  for (int s = 0; s < 4; ++s) a.seg[s] = (s < c.nseg) ? c.seg[s] : MvSeg{nullptr, nullptr, nullptr, 0, 0};
  for (int s = 0; s < 5; ++s) a.tile0[s] = p.tile0[s];
  a.nseg = c.nseg; a.ntiles = p.ntiles; a.nsplit = p.nsplit; a.kchunk = p.kchunk; a.naux = p.naux;
  a.K = c.K; a.M = c.M; a.pro = c.pro;
  a.x = c.x; a.xf = c.xf; a.ldx = c.ldx; a.x2 = c.x2; a.x2f = c.x2f; a.ldx2 = c.ldx2;
  a.pw = c.pw; a.group = c.group; a.swiglu_off = c.swiglu_off; a.eps = c.eps;
  a.emb_q = c.emb_q; a.emb_s = c.emb_s; a.token = c.token; a.h_out = c.h_out;
  a.prompt = c.prompt; a.plen = c.plen; a.pos = c.pos;
  a.aux_wb = c.aux_wb; a.aux_wa = c.aux_wa; a.aux_nh = c.aux_nh; a.aux_acc = c.aux_acc; a.aux_ldo = c.aux_ldo;
  a.zero_ptr = c.zero_ptr; a.zero_n = c.zero_n;
  a.cs_state = c.cs_state; a.cs_x = c.cs_x; a.cs_ch = c.cs_ch; a.cs_ldx = c.cs_ldx; a.cs_B = c.cs_B;
  a.y_out = c.y_out; a.ldy = c.ldy; a.tile_ctr = c.tile_ctr;
  a.err = c.err;
  if (c.y_out && (c.nseg != 1 || c.aux_nh > 0 || !c.tile_ctr || p.ntiles > kMaxCounters))
    return fail(Q35_E_ARG, "mv_kn: f32 output needs one segment, no gate blocks and a counter per tile");

  const int nblocks = p.ntiles * p.nsplit + p.naux;
  const dim3 grid(nblocks), block(kThreads);
  if (c.M == 1) hipLaunchKernelGGL(mv_kn_kernel<1>, grid, block, 0, st, a);
  else if (c.M == 2) hipLaunchKernelGGL(mv_kn_kernel<2>, grid, block, 0, st, a);
  else if (c.M <= 4) hipLaunchKernelGGL(mv_kn_kernel<4>, grid, block, 0, st, a);
  else hipLaunchKernelGGL(mv_kn_kernel<8>, grid, block, 0, st, a);
  Q35_HIP_TRY(hipGetLastError());
  return Q35_OK;
}

int fx_to_f32_launch(fx_t* acc, int64_t n, float* y, bool zero_after, hipStream_t st) {
  if (n <= 0) return Q35_OK;
  hipLaunchKernelGGL(fx_to_f32_kernel, dim3(grid_for(n)), dim3(kThreads), 0, st, acc, n, y, zero_after ? 1 : 0);
  Q35_HIP_TRY(hipGetLastError());
  return Q35_OK;
}

int fx_zero_launch(fx_t* acc, int64_t n, hipStream_t st) {
  if (n <= 0) return Q35_OK;
  hipLaunchKernelGGL(fx_zero_kernel, dim3(grid_for(n)), dim3(kThreads), 0, st, acc, n);
  Q35_HIP_TRY(hipGetLastError());
  return Q35_OK;
}

}  // namespace q35
