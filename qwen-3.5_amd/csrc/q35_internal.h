// Internal declarations shared by the HIP kernels, the launchers and the C ABI.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>
#include <string>
#include "../../include/q35.h"

namespace q35 {

// ------------------------------------------------------------------ error plumbing
void set_error(const std::string& msg);
int fail(int code, const std::string& msg);

#define Q35_HIP_TRY(expr)                                                              \
  do {                                                                                 \
    hipError_t e_ = (expr);                                                            \
    if (e_ != hipSuccess)                                                              \
      return ::q35::fail(Q35_E_HIP, std::string(#expr) + ": " + hipGetErrorString(e_)); \
  } while (0)

// ------------------------------------------------------------------ device helpers
#define Q35_DEV __device__ __forceinline__

Q35_DEV float silu_f(float v) { return v * (1.0f / (1.0f + expf(-v))); }
Q35_DEV float sigmoid_f(float v) { return 1.0f / (1.0f + expf(-v)); }

Q35_DEV float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Sum over a 256-thread block; `sh` needs 4 floats of LDS.  All threads get the result.
Q35_DEV float block_sum256(float v, float* sh) {
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) sh[wid] = v;
  __syncthreads();
  return (sh[0] + sh[1]) + (sh[2] + sh[3]);
}

// 16 signed bytes -> 16 floats
Q35_DEV void unpack16(const uint4 w, float* f) {
  const uint32_t d[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int q = 0; q < 4; ++q) {
#pragma unroll
    for (int j = 0; j < 4; ++j) f[q * 4 + j] = (float)(int8_t)(d[q] >> (8 * j));
  }
}

// Split-K / split-T "last block finishes" protocol.  Every block of a group publishes its
// partial, then increments the group's counter; the block that brings it to `expected`
// reads all partials (in a fixed order, so results are deterministic) and resets the counter
// to zero so the next launch (or graph replay) starts clean.  Returns true in that block.
Q35_DEV bool arrive_last(uint32_t* counter, uint32_t expected, int* sh_flag) {
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t prev = atomicAdd(counter, 1u);
    const bool last = (prev + 1u == expected);
    if (last) *counter = 0u;
    *sh_flag = last ? 1 : 0;
  }
  __syncthreads();
  const bool last = *sh_flag != 0;
  if (last) __threadfence();
  return last;
}

// Workspace layout shared by every kernel: the first kCounterBytes hold completion
// counters (zero between launches; each kernel leaves them zero), scratch follows.  Kernels on
// one stream run one after another, so they can all reuse the same workspace.
constexpr size_t kCounterBytes = 65536;
constexpr int kMaxCounters = (int)(kCounterBytes / 4);
inline uint32_t* ws_counters(void* ws) { return static_cast<uint32_t*>(ws); }
inline char* ws_scratch(void* ws) { return static_cast<char*>(ws) + kCounterBytes; }
inline size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

// ------------------------------------------------------------------ Q8F KN matvec (split-K)
enum { PRO_PLAIN = 0, PRO_RMS = 1, PRO_GATED = 2, PRO_SWIGLU = 3, PRO_EMBED_RMS = 4 };
enum { EPI_STORE = 0, EPI_RESID = 1 };

struct MvSeg {
  const int8_t* w;  // [K][N]
  const float* s;   // [K][N/64]
  float* y;         // y[m*ldy + n]; for EPI_RESID the residual stream updated in place
  int32_t N;
  int32_t ldy;
};

struct MvCall {
  MvSeg seg[4];
  int32_t nseg = 0;
  int32_t K = 0, M = 1;
  int32_t pro = PRO_PLAIN, epi = EPI_STORE;
  const float* x = nullptr;   // prologue input x[m*ldx + k]
  int32_t ldx = 0;
  const float* x2 = nullptr;  // PRO_GATED: z[m*ldx2 + k]
  int32_t ldx2 = 0;
  const float* pw = nullptr;  // PRO_RMS: norm weight (applied as 1+w); PRO_GATED: weight [group]
  int32_t group = 0;          // PRO_GATED group size
  int32_t swiglu_off = 0;     // PRO_SWIGLU: x = in[off+k] * silu(in[k])
  float eps = 1e-6f;
  // PRO_EMBED_RMS (M == 1): residual = dequant(embed[tok]); block 0 stores it to h_out.
  // tok = prompt[*pos] while *pos < *plen (prompt fed from device memory), else *token.
  const int8_t* emb_q = nullptr;
  const float* emb_s = nullptr;
  const int32_t* token = nullptr;
  const int32_t* prompt = nullptr;
  const int32_t* plen = nullptr;
  const int32_t* pos = nullptr;
  float* h_out = nullptr;
  // optional f32 gate projection riding in the same launch (GatedDeltaNet in_proj_b/in_proj_a)
  const float* aux_wb = nullptr;
  const float* aux_wa = nullptr;
  const float* aux_alog = nullptr;
  const float* aux_dtb = nullptr;
  int32_t aux_nh = 0;
  float* aux_out = nullptr;  // [M][2*aux_nh] = [beta | g]
  int32_t aux_ldo = 0;
};

size_t mv_kn_ws_bytes(const MvCall& c);
int mv_kn_launch(const MvCall& c, void* ws, size_t ws_bytes, hipStream_t st);

// ------------------------------------------------------------------ Q8F NK matvec / lm_head
struct NkCall {
  const int8_t* q;  // [N][K]
  const float* s;   // [N][K/64]
  int32_t N = 0, K = 0, M = 1;
  const float* x = nullptr;
  int32_t ldx = 0;
  float* y = nullptr;  // y[m*ldy + n] (may be null when only the argmax is wanted)
  int32_t ldy = 0;
  int32_t pro = PRO_PLAIN;  // PRO_PLAIN or PRO_RMS
  const float* pw = nullptr;
  float eps = 1e-6f;
  int32_t* argmax_out = nullptr;  // M == 1: index of the max logit
  int32_t* pos_inc = nullptr;     // optional device counter incremented once by the last block
  int32_t* hist = nullptr;        // optional: hist[*pos_inc] = argmax before the increment
};
size_t nk_ws_bytes(const NkCall& c);
int nk_launch(const NkCall& c, void* ws, size_t ws_bytes, hipStream_t st);

// standalone argmax over a device vector
size_t argmax_ws_bytes(int64_t n);
int argmax_launch(const float* v, int64_t n, int32_t* out, void* ws, size_t ws_bytes, hipStream_t st);

// embedding lookup
int embed_launch(const int8_t* q, const float* s, int32_t V, int32_t D, const int32_t* ids, int32_t n,
                 float* out, hipStream_t st);

// ------------------------------------------------------------------ Gated DeltaNet step
struct GdnCall {
  const float* qkv; int32_t ld_qkv;  // pre-conv mixed qkv [B][conv_dim]
  const float* bg;  int32_t ld_bg;   // [B][2*nh] = [beta | g]
  float* conv_state;                 // [B][conv_dim][conv_k-1]
  const float* conv_w;               // [conv_dim][conv_k]
  float* S;                          // [B][nh][dk][dv]
  float* o;         int32_t ld_o;    // [B][nh*dv] raw core output (before the gated norm)
  int32_t B, nh, dk, dv, conv_k;
};
size_t gdn_step_ws_bytes(int32_t B, int32_t nh);
int gdn_step_launch(const GdnCall& c, void* ws, size_t ws_bytes, hipStream_t st);

// Gate projection alone (kernels.rs gate_proj): uses the matvec kernel's aux path.
int gate_proj_launch(const float* x, int32_t B, int32_t in_dim, const float* wb, const float* wa,
                     const float* alog, const float* dtb, int32_t nh, float* out, void* ws,
                     size_t ws_bytes, hipStream_t st);
size_t gate_proj_ws_bytes(int32_t B, int32_t in_dim, int32_t nh);
// Gate projection without workspace: one block per batch row.
int gate_proj_simple_launch(const float* x, int32_t B, int32_t in_dim, const float* wb, const float* wa,
                            const float* alog, const float* dtb, int32_t nh, float* out, hipStream_t st);

// Gated-RMSNorm alone is folded into the out_proj prologue (PRO_GATED).

// ------------------------------------------------------------------ attention decode
struct AttnCall {
  const float* qg; int32_t ld_qg;   // [B][nh*2*hd], per head [query | gate]
  const float* k; const float* v;   // new token's k / v rows: k[b*ld_kv + g*hd + i]
  int32_t ld_kv;
  const float* qnw; const float* knw; float eps;
  const float* rcos; const float* rsin; int32_t rot;
  float* kc; float* vc; int32_t tmax;  // [B][nkv][tmax][hd]
  const int32_t* pos;                  // [B]
  float* out; int32_t ld_out;          // [B][nh*hd]
  int32_t B, nh, nkv, hd;
};
size_t attn_ws_bytes(int32_t B, int32_t nh, int32_t nkv, int32_t hd, int32_t tmax);
int attn_launch(const AttnCall& c, void* ws, size_t ws_bytes, hipStream_t st);

}  // namespace q35
