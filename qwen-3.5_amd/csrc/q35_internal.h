// Internal declarations shared by the HIP kernels, the launchers and the C ABI.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>
#include <string>
#include <type_traits>
#include "../../include/q35.h"
#include "fx_range.h"

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

// Native 4 x u32 / 4 x f32 vectors.  Register arrays that stay live across a runtime loop must
// use these: arrays of HIP's uint4 / float4 structs there are left in private memory (scratch).
typedef unsigned int q35_u32x4 __attribute__((ext_vector_type(4)));
typedef float q35_f32x4 __attribute__((ext_vector_type(4)));

// 1/x and 1/sqrt(x) as the single hardware instructions (v_rcp_f32, v_rsq_f32; about 1 ulp):
// the IEEE-rounded divide and square root are ~10-instruction dependent sequences each, and these
// sit on the latency chain of every norm and gate.  Arguments here are positive and normal.
Q35_DEV float rcp_f(float x) { return __builtin_amdgcn_rcpf(x); }
Q35_DEV float rsqrt_f(float x) { return __builtin_amdgcn_rsqf(x); }
// e^-v for the logistic function as 2^(-v log2 e) with the hardware exp2 (v_exp_f32): rounding the
// product gives a relative error of about |v| 2^-24, which a logistic gate does not compound
// (the DeltaNet decay, applied step after step, keeps the library expf).  Large |v| saturate
// correctly: 1 + inf -> rcp 0, 1 + 0 -> 1.
Q35_DEV float exp_neg_hw(float v) { return __builtin_amdgcn_exp2f(-v * 1.44269504088896341f); }
Q35_DEV float silu_f(float v) { return v * rcp_f(1.0f + exp_neg_hw(v)); }
Q35_DEV float sigmoid_f(float v) { return rcp_f(1.0f + exp_neg_hw(v)); }

// x from lane (l + N) mod 16 of the same 16-lane row (DPP row_ror: a VALU operand modifier, no
// trip through the LDS crossbar as a lane shuffle takes)
template <int N>
Q35_DEV float row_ror(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x120 + N, 0xf, 0xf, false));
}

// Sum over the 64 lanes of a wave, the same value in every lane: rotations by 8, 4, 2, 1 within
// each 16-lane row leave every lane with its row's sum; the four row sums are then read from
// lanes 0, 16, 32 and 48.  Every lane of the wave must be active.
Q35_DEV float wave_sum(float v) {
  v += row_ror<8>(v);
  v += row_ror<4>(v);
  v += row_ror<2>(v);
  v += row_ror<1>(v);
  const int b = __float_as_int(v);
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(b, 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(b, 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(b, 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(b, 48));
  return (r0 + r1) + (r2 + r3);
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
Q35_DEV void unpack16v(const q35_u32x4 w, float* f) {
#pragma unroll
  for (int q = 0; q < 4; ++q) {
#pragma unroll
    for (int j = 0; j < 4; ++j) f[q * 4 + j] = (float)(int8_t)(w[q] >> (8 * j));
  }
}
Q35_DEV void unpack16(const uint4 w, float* f) {
  const uint32_t d[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int q = 0; q < 4; ++q) {
#pragma unroll
    for (int j = 0; j < 4; ++j) f[q * 4 + j] = (float)(int8_t)(d[q] >> (8 * j));
  }
}

// Split-K accumulation in 64-bit fixed point (value * 2^32, two's complement).  Every block
// adds its partial sums with a fire-and-forget atomic; integer addition is associative, so the
// total is identical whatever order the blocks arrive in (bit-reproducible), and the only
// rounding is one f32 -> 2^-32 grid step per partial (|error| <= 2^-33 each).  The consumer
// (a later kernel) converts the total back to f32.  Valid for |value| < 2^31: contributions go
// through fx_add_chk, which drops one that is not (fx_addable) and reports it.
typedef long long fx_t;
Q35_DEV fx_t to_fx(float v) { return __float2ll_rn(v * 4294967296.0f); }
Q35_DEV float from_fx(fx_t a) { return (float)((double)a * (1.0 / 4294967296.0)); }

// Every buffer the kernels touch through these helpers is device memory (global address
// space).  Pointers that reach a kernel through a table in memory are generic to the compiler,
// and generic accesses become FLAT instructions, which count against the LDS counter too: a
// workgroup barrier (which waits for LDS) would then also wait for every weight load in flight.
// The casts keep them `global_*`.
#define Q35_GLOBAL __attribute__((address_space(1)))
template <class T>
Q35_DEV T ldg(const T* p) { return *(const Q35_GLOBAL T*)p; }
template <class T>
Q35_DEV void stg(T* p, T v) { *(Q35_GLOBAL T*)p = v; }
// 16-byte global load (p 16-byte aligned)
Q35_DEV uint4 ldg16(const void* p) {
  const q35_u32x4 v = *(const Q35_GLOBAL q35_u32x4*)p;
  return make_uint4(v.x, v.y, v.z, v.w);
}
// The same with the non-temporal hint, for the weight stream: each weight is read once per
// decode step and the stream is far larger than the caches, so it should not evict what is
// reused (the kernel's code, norm weights, the small shared activations).
Q35_DEV uint4 ldg16_nt(const void* p) {
  const q35_u32x4 v = __builtin_nontemporal_load((const Q35_GLOBAL q35_u32x4*)p);
  return make_uint4(v.x, v.y, v.z, v.w);
}
template <class T>
Q35_DEV T ldg_nt(const T* p) { return __builtin_nontemporal_load((const Q35_GLOBAL T*)p); }
// The same as a native vector (for register arrays that stay live across a runtime loop)
Q35_DEV q35_u32x4 ldg16v_nt(const void* p) { return __builtin_nontemporal_load((const Q35_GLOBAL q35_u32x4*)p); }

// ---- f32-equivalent products on the f16 matrix cores (v_mfma_f32_16x16x32_f16): 8-bit weights
// are exact in f16; an f32 input y is carried as hi + lo halves.
typedef _Float16 q35_h2 __attribute__((ext_vector_type(2)));
typedef _Float16 q35_h8 __attribute__((ext_vector_type(8)));
typedef __fp16 q35_hf2 __attribute__((ext_vector_type(2)));
// Two weights u0, u1 (bytes sel of dw, u = q + 128) -> f16 pair (q0, q1), exact.
Q35_DEV q35_h2 u8_pair(uint32_t dw, uint32_t sel) {
  const uint32_t v = __builtin_amdgcn_perm(0x64646464u, dw, sel);  // halves 0x6400 | u
  return __builtin_bit_cast(q35_h2, v) - q35_h2{(_Float16)1152.0f, (_Float16)1152.0f};
}
// The 8 weights of bytes 0..3 of da and 0..3 of db as an f16 MFMA operand.
Q35_DEV q35_h8 a8_from(uint32_t da, uint32_t db) {
  const q35_h2 p0 = u8_pair(da, 0x04010400u), p1 = u8_pair(da, 0x04030402u);
  const q35_h2 p2 = u8_pair(db, 0x04010400u), p3 = u8_pair(db, 0x04030402u);
  return q35_h8{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
}
// 2^(14 - E) and its inverse for a row whose largest |value| is amax < 2^E (E from the float's
// exponent field; rows of zeros get 1)
Q35_DEV void split_scale(float amax, float& f, float& inv) {
  const int bits = __float_as_int(amax);
  const int E = amax > 0.f ? ((bits >> 23) & 0xff) - 126 : 14;
  const int e = min(max(14 - E, -126), 126);  // (both 2^e and 2^-e normal)
  f = __int_as_float((127 + e) << 23);
  inv = __int_as_float((127 - e) << 23);
}
// y -> (hi, lo) f16 halves (packed conversions, rounding toward zero), y = hi + lo to about 22
// bits: y - hi is exact in f32, and lo keeps its leading 11 bits
Q35_DEV void split2(float y0, float y1, uint32_t& hi, uint32_t& lo) {
  const q35_hf2 h = __builtin_amdgcn_cvt_pkrtz(y0, y1);
  const q35_hf2 l = __builtin_amdgcn_cvt_pkrtz(y0 - (float)h[0], y1 - (float)h[1]);
  hi = __builtin_bit_cast(uint32_t, h);
  lo = __builtin_bit_cast(uint32_t, l);
}


Q35_DEV void fx_add(fx_t* p, float v) {
  __hip_atomic_fetch_add((Q35_GLOBAL unsigned long long*)p, (unsigned long long)to_fx(v), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
}
// fx_add of a value that is checked first: a non-finite one, or one whose magnitude would
// overflow the fixed point, is not added; it ORs kWsErrRange into the error word *err instead
// (where the reference's f32 sums would carry the NaN / Inf on, text_modules.rs:1080,1084).
Q35_DEV void fx_add_chk(fx_t* p, float v, uint32_t* err);

// Cross-block partial results are written and read with agent-scope relaxed atomics: on
// gfx950 these are `global_store ... sc1` / `global_load ... sc1`, i.e. coherent at the device
// level (write-through / miss in the per-XCD L2) without the whole-L2 writeback and
// invalidate (`buffer_wbl2` / `buffer_inv`) that a device-scope fence costs on every block.
Q35_DEV void st_agent(float* p, float v) { __hip_atomic_store((Q35_GLOBAL float*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
Q35_DEV void st_agent(int32_t* p, int32_t v) {
  __hip_atomic_store((Q35_GLOBAL int32_t*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
Q35_DEV float ld_agent(const float* p) {
  return __hip_atomic_load((Q35_GLOBAL float*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
Q35_DEV int32_t ld_agent(const int32_t* p) {
  return __hip_atomic_load((Q35_GLOBAL int32_t*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

Q35_DEV fx_t ld_agent(const fx_t* p) {
  return __hip_atomic_load((Q35_GLOBAL fx_t*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
Q35_DEV void st_agent(fx_t* p, fx_t v) { __hip_atomic_store((Q35_GLOBAL fx_t*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
Q35_DEV uint32_t ld_agent(const uint32_t* p) {
  return __hip_atomic_load((Q35_GLOBAL uint32_t*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Greedy argmax order of the reference (kernels.rs:298-371).  Its first kernel lets unit
// p < c = n/8 scan p, p + c, ..., p + 7c keeping the first strict maximum; its second has
// thread t < 256 scan the unit results t, t + 256, ... and thread 0 scan the 256 thread
// results, each keeping the first strict maximum.  Among exactly equal maxima the winner is
// therefore the index i = k c + p minimising (p mod 256, p div 256, k), which is not always the
// lowest index (i = 256 beats i = 1; i = c beats i = 1).  The key below encodes that tuple in 32
// bits; an argmax is "larger value, or equal value and smaller key", a total order on indices,
// so any reduction tree (lanes, waves, blocks) returns the reference's winner.  The last n mod 8
// values, which the reference never reads, rank after all others on ties; the out-of-range
// index (the INT_MAX sentinel of an empty partial) ranks last.  NaN never wins here.
struct ArgOrder {
  uint32_t n, c, s, n8;  // n values; c = n / 8; s = ceil(c / 256); n8 = 8 c
};
inline ArgOrder make_arg_order(int64_t n) {
  ArgOrder o;
  o.n = (uint32_t)n;
  o.c = (uint32_t)(n / 8);
  o.s = (o.c + 255u) / 256u;
  o.n8 = 8u * o.c;
  return o;
}
Q35_DEV uint32_t arg_key(const ArgOrder& o, int i) {
  if (i < 0 || (uint32_t)i >= o.n) return 0xffffffffu;
  const uint32_t u = (uint32_t)i;
  if (u >= o.n8) return (o.s << 11) + (u - o.n8);
  const uint32_t k = u / o.c, p = u - k * o.c;
  return ((((p & 255u) * o.s) + (p >> 8)) << 3) + k;
}
Q35_DEV bool argmax_better(float v, int i, float bv, int bi, const ArgOrder& o) {
  return v > bv || (v == bv && arg_key(o, i) < arg_key(o, bi));
}
Q35_DEV void wave_argmax(float& v, int& i, const ArgOrder& o) {
#pragma unroll
  for (int s = 32; s > 0; s >>= 1) {
    const float ov = __shfl_xor(v, s, 64);
    const int oi = __shfl_xor(i, s, 64);
    if (argmax_better(ov, oi, v, i, o)) { v = ov; i = oi; }
  }
}

// f(std::integral_constant<int, i>) for i = 0 .. N-1 at compile time: register arrays indexed
// through it see constant indices from the start (a #pragma unroll loop only gets them after
// unrolling, which is too late for arrays that live across a runtime loop: those stay in memory).
template <int N, class F>
Q35_DEV void static_for(F&& f) {
  if constexpr (N > 0) {
    static_for<N - 1>(f);
    f(std::integral_constant<int, N - 1>{});
  }
}

// Transposed butterfly over R per-lane row partials: on return every lane holds the full sum of
// row (lane / (64 / R)).  Stage S (32, 16, ...) halves the rows a lane keeps: lanes with bit S
// set keep the upper half and receive their partner's copy of it, the others the lower half;
// then the 64/R lanes sharing a row finish the sum: log2(R) + log2(64/R) exchanges for R rows.
// Written as compile-time recursion so every index into p is a constant (no private memory).
template <int R, int CNT, int S>
Q35_DEV void fold_stage(float (&p)[R], int lane) {
  if constexpr (CNT > 1) {
    constexpr int half = CNT / 2;
    const bool hi = (lane & S) != 0;
#pragma unroll
    for (int i = 0; i < half; ++i) {
      const float snd = hi ? p[i] : p[i + half];
      const float keep = hi ? p[i + half] : p[i];
      p[i] = keep + __shfl_xor(snd, S, 64);
    }
    fold_stage<R, half, S / 2>(p, lane);
  }
}
template <int R>
Q35_DEV float fold_rows(float (&p)[R], int lane) {
  static_assert(R >= 1 && R <= 64 && (R & (R - 1)) == 0, "R must be a power of two <= 64");
  fold_stage<R, R, 32>(p, lane);
  float v = p[0];
#pragma unroll
  for (int s = 32 / R; s > 0; s >>= 1) v += __shfl_xor(v, s, 64);
  return v;
}

// sum_{i<n} p[i*stride] in index order.  Loads are issued kSumBatch at a time so their latency
// overlaps (a loop that adds each value as it arrives would wait for every load in turn).
#ifndef Q35_SUM_BATCH
#define Q35_SUM_BATCH 32
#endif
constexpr int kSumBatch = Q35_SUM_BATCH;
Q35_DEV float sum_agent(const float* p, int n, size_t stride) {
  float t = 0.f;
  for (int i = 0; i < n; i += kSumBatch) {
    float v[kSumBatch];
#pragma unroll
    for (int j = 0; j < kSumBatch; ++j) v[j] = (i + j < n) ? ld_agent(p + (size_t)(i + j) * stride) : 0.f;
#pragma unroll
    for (int j = 0; j < kSumBatch; ++j) t += v[j];
  }
  return t;
}

// Split-K / split-T "last block finishes" protocol.  Every block of a group publishes its
// partial with st_agent, then increments the group's counter; the block that brings it to
// `expected` reads all partials with ld_agent (in a fixed order, so results are
// deterministic) and resets the counter to zero so the next launch (or graph replay) starts
// clean.  Ordering: s_waitcnt 0 makes every wave's earlier memory operations (the sc1 partial
// stores included) complete before the barrier, and the counter RMW is issued after it; the
// reader's sc1 loads are issued after the RMW result is known.  Returns true in that block.
Q35_DEV bool arrive_last(uint32_t* counter, uint32_t expected, int* sh_flag) {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t prev = __hip_atomic_fetch_add((Q35_GLOBAL uint32_t*)counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const bool last = (prev + 1u == expected);
    if (last) __hip_atomic_store((Q35_GLOBAL uint32_t*)counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *sh_flag = last ? 1 : 0;
  }
  __syncthreads();
  return *sh_flag != 0;
}

// Workspace layout shared by every kernel: the first kCounterBytes hold completion
// counters (zero between launches; each kernel leaves them zero), scratch follows.  Kernels on
// one stream run one after another, so they can all reuse the same workspace.
constexpr size_t kCounterBytes = 65536;
// The last counter word is the workspace's sticky error word: kernels that validate
// device-resident arguments (positions) OR a Q35_WS_ERR_* bit into it instead of touching memory
// out of range; q35_workspace_status reads and clears it.
constexpr int kWsErrWord = (int)(kCounterBytes / 4) - 1;
constexpr int kMaxCounters = kWsErrWord;
inline uint32_t* ws_counters(void* ws) { return static_cast<uint32_t*>(ws); }
enum : uint32_t {
  kWsErrPos = 1u,    // an attention position outside [0, tmax)
  kWsErrRange = 2u,  // a value for a fixed-point accumulator was not finite or |v| >= 2^31 (dropped)
};
Q35_DEV void ws_raise(uint32_t* counters, uint32_t bit) {
  __hip_atomic_fetch_or((Q35_GLOBAL uint32_t*)&counters[kWsErrWord], bit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
Q35_DEV void fx_add_chk(fx_t* p, float v, uint32_t* err) {
  if (fx_addable(v)) fx_add(p, v);
  else __hip_atomic_fetch_or((Q35_GLOBAL uint32_t*)err, kWsErrRange, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
inline char* ws_scratch(void* ws) { return static_cast<char*>(ws) + kCounterBytes; }
inline size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

// arrive_last for a whole grid of many blocks: blocks arrive on a counter per group of 64
// (counters[1 + blockIdx/64]); the last block of each group arrives on counters[0].  Keeps
// the same-address atomic chain at <= 64 instead of gridDim.x.  Uses 1 + ceil(grid/64)
// counters.
Q35_DEV bool arrive_last_grid(uint32_t* counters, int* sh_flag) {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t G = 64;
    const uint32_t grp = blockIdx.x / G;
    const uint32_t ngrp = (gridDim.x + G - 1) / G;
    const uint32_t in_grp = (gridDim.x - grp * G) < G ? (gridDim.x - grp * G) : G;
    bool last = false;
    const uint32_t p1 = __hip_atomic_fetch_add((Q35_GLOBAL uint32_t*)&counters[1 + grp], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (p1 + 1u == in_grp) {
      __hip_atomic_store((Q35_GLOBAL uint32_t*)&counters[1 + grp], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const uint32_t p0 = __hip_atomic_fetch_add((Q35_GLOBAL uint32_t*)&counters[0], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (p0 + 1u == ngrp) {
        __hip_atomic_store((Q35_GLOBAL uint32_t*)&counters[0], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last = true;
      }
    }
    *sh_flag = last ? 1 : 0;
  }
  __syncthreads();
  return *sh_flag != 0;
}

// ------------------------------------------------------------------ Q8F KN matvec (split-K)
enum { PRO_PLAIN = 0, PRO_RMS = 1, PRO_GATED = 2, PRO_SWIGLU = 3, PRO_EMBED_RMS = 4, PRO_ATTN = 5, PRO_GDN = 6 };
struct MvSeg {
  const int8_t* w;  // [K][N]
  const float* s;   // [K][N/64]
  fx_t* acc;        // acc[m*ldacc + n] += y: a zeroed accumulator, or the residual stream
  int32_t N;
  int32_t ldacc;
  int32_t tiled = 0;  // 1: w, s in the Q35_KN_TILED layout (w[t][K][256], s[t][K][4])
};

struct MvCall {
  MvSeg seg[4];
  int32_t nseg = 0;
  int32_t K = 0, M = 1;
  int32_t pro = PRO_PLAIN;
  // prologue input in[m][k]: f32 x[m*ldx + k], or the fixed-point accumulator xf when set
  const float* x = nullptr;
  const fx_t* xf = nullptr;
  int32_t ldx = 0;
  const float* x2 = nullptr;  // PRO_GATED: z (f32 or fixed point x2f), row stride ldx2
  const fx_t* x2f = nullptr;
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
  fx_t* h_out = nullptr;
  // optional f32 gate projection on extra blocks (GatedDeltaNet in_proj_b / in_proj_a): raw
  // sums [x.W_b | x.W_a] added to aux_acc[m*aux_ldo + 0 .. 2*aux_nh)
  const float* aux_wb = nullptr;
  const float* aux_wa = nullptr;
  int32_t aux_nh = 0;
  fx_t* aux_acc = nullptr;
  int32_t aux_ldo = 0;
  // side task: zero zero_ptr[0 .. zero_n) for a later kernel
  fx_t* zero_ptr = nullptr;
  int64_t zero_n = 0;
  // side task: causal-conv state shift, state[b][c] <- [s1, s2, x[b*cs_ldx + c]] for c < cs_ch
  float* cs_state = nullptr;
  const fx_t* cs_x = nullptr;
  int32_t cs_ch = 0, cs_ldx = 0, cs_B = 0;
  // optional f32 output y[m*ldy + n] of a one-segment call: the last block of each tile converts
  // the tile's fixed-point sums and re-zeroes them (tile_ctr: one zeroed counter per tile)
  float* y_out = nullptr;
  int32_t ldy = 0;
  uint32_t* tile_ctr = nullptr;
  // the error word that receives kWsErrRange (required): a workspace's counters[kWsErrWord]
  uint32_t* err = nullptr;
};

int mv_kn_launch(const MvCall& c, hipStream_t st);
// y[m][n] = x[m][:] . dequant(W)[:, n] for the Q35_KN_PANEL layout (one launch, M <= 8)
int mvp_launch(const int8_t* q, const float* s, int32_t K, int32_t N, const float* x, int32_t ldx, int32_t M,
               float* y, int32_t ldy, hipStream_t st);
// y[i] = f32(acc[i]) (optionally re-zeroing acc); acc[i] = 0
int fx_to_f32_launch(fx_t* acc, int64_t n, float* y, bool zero_after, hipStream_t st);
int fx_zero_launch(fx_t* acc, int64_t n, hipStream_t st);

// ------------------------------------------------------------------ Q8F GEMM (prompt projections)
// Y[m][n] (+)= X[m][:] . dequant(W)[:, n] on the fp32 matrix cores; up to kGemmMaxSeg weight
// matrices over the same X, each writing its own columns of Y.
constexpr int kGemmMaxSeg = 4;
struct GemmSeg {
  const int8_t* q;
  const float* s;
  float* y;        // y[m*ldy + n]
  int32_t N;       // columns (multiple of 64)
  int32_t layout;  // Q35_KN, Q35_KN_TILED, Q35_KN_MB (rows = K) or Q35_NK (rows = N)
  int32_t ldy;
  const float* smax = nullptr;  // Q35_KN_MB: device copy of max |scale| (mb_scale_max_launch), optional
};
struct GemmCall {
  GemmSeg seg[kGemmMaxSeg];
  int32_t nseg = 0;
  const float* x = nullptr;  // [M][ldx], 16-byte aligned rows
  int32_t ldx = 0, M = 0, K = 0;
  int32_t accumulate = 0;    // 1: y += result (each element owned by one block), 0: y = result
  // optional split-K partials [splits][M][sum of N]: the launcher may then split K when that is
  // estimated faster, and sums the splits in a fixed order in a second kernel
  float* part = nullptr;
  size_t part_floats = 0;
  // Q35_KN_MB launches (every segment MB): kGemmAuxFloats(M) floats for the row and scale maxima
  float* aux = nullptr;
  // Q35_KN_MB: max |x| of each row [M] when the producer of x has computed it (skips that pass)
  const float* amax = nullptr;
  // Q35_KN_MB, one segment: with defer_reduce set, a launch that splits K leaves the splits'
  // partial sums in part ([split][M][N]) instead of adding them into y; *ksplit_out (when given)
  // reports how many the caller must add (1: none, y was written), in split order and then y when
  // accumulating (rms_rows_launch does, before it normalises the rows)
  int32_t defer_reduce = 0;
  int32_t* ksplit_out = nullptr;
  // Q35_KN_MB, one segment whose 64-column blocks alternate gate and up (block 2 j: gate columns
  // 64 j .., block 2 j + 1: up columns 64 j ..): the launch writes act[m][64 j + c] =
  // up * silu(gate) (N / 2 columns) instead of y, and raises act_amax[m] (zero beforehand) to each
  // row's max |act|; K is not split
  float* act = nullptr;
  int32_t ld_act = 0;
  float* act_amax = nullptr;
};
// Scratch floats of an MB launch: row maxima [M] and scale partial maxima [64], 64-aligned.
inline size_t gemm_aux_floats(int M) { return ((size_t)M + 63) / 64 * 64 + 64; }
int gemm_launch(const GemmCall& c, hipStream_t st);
// Tile shape and K splits the launcher picks for c (BM x BN, ksplit).
int gemm_pick(const GemmCall& c, int* bm, int* bn, int* ksplit);
// Partial floats that let gemm_launch consider up to kGemmMaxSplit K splits for M rows of N columns.
constexpr int kGemmMaxSplit = 4;
inline size_t gemm_part_floats(int M, int64_t N) { return (size_t)kGemmMaxSplit * M * N; }

// ------------------------------------------------------------------ Q8F NK matvec / lm_head
struct NkCall {
  const int8_t* q;  // [N][K]
  const float* s;   // [N][K/64]
  int32_t N = 0, K = 0, M = 1;
  const float* x = nullptr;
  const fx_t* xf = nullptr;  // fixed-point input (the residual stream) instead of x
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
// Rows of x (1, 2, 4 or 8) one lm_head launch can stage in LDS for inner dimension K.
int nk_max_rows(int K);
int nk_launch(const NkCall& c, void* ws, size_t ws_bytes, hipStream_t st);

// standalone argmax over a device vector
size_t argmax_ws_bytes(int64_t n);
int argmax_launch(const float* v, int64_t n, int32_t* out, void* ws, size_t ws_bytes, hipStream_t st);

// embedding lookup
int embed_launch(const int8_t* q, const float* s, int32_t V, int32_t D, const int32_t* ids, int32_t n,
                 float* out, hipStream_t st);

// ------------------------------------------------------------------ Gated DeltaNet step
// The step reads the conv state but does not advance it (every value-column slice of a head
// reads the same q/k channels); the caller advances it afterwards (conv_shift_launch, or the
// cs_* side task of the next matvec).
struct GdnCall {
  // pre-conv mixed qkv [B][conv_dim]: f32 qkv, or the fixed-point accumulator qkv_f
  const float* qkv = nullptr; const fx_t* qkv_f = nullptr; int32_t ld_qkv = 0;
  // gates: activated [beta | g] bg (f32), or raw [x.W_b | x.W_a] ba_f (fixed point) plus
  // a_log / dt_bias, activated here as kernels.rs:228-244 does
  const float* bg = nullptr; const fx_t* ba_f = nullptr; int32_t ld_bg = 0;
  const float* a_log = nullptr; const float* dt_bias = nullptr;
  float* conv_state = nullptr;        // [B][conv_dim][conv_k-1]
  const float* conv_w = nullptr;      // [conv_dim][conv_k]
  float* S = nullptr;                 // [B][nh][dk][dv]
  float* o = nullptr; int32_t ld_o = 0;  // [B][nh*dv] raw core output (before the gated norm)
  int32_t B = 1, nh = 0, dk = 0, dv = 0, conv_k = 0;
  // optional zeroed counters [B*nh]: the kernel then advances the conv state itself (left zero)
  uint32_t* head_ctr = nullptr;
};
int gdn_step_launch(const GdnCall& c, hipStream_t st);
// state[b][c] <- [s1, s2, x[b][c]] for all conv_dim channels (f32 x)
int conv_shift_launch(float* state, const float* x, int32_t B, int32_t ch, hipStream_t st);

// Gate projection without workspace: one block per batch row.
// input_rule: softplus threshold on its input (the prompt path) instead of its result (decode).
int gate_proj_simple_launch(const float* x, int32_t B, int32_t in_dim, const float* wb, const float* wa,
                            const float* alog, const float* dtb, int32_t nh, float* out, hipStream_t st,
                            int32_t input_rule = 0);

// Gated-RMSNorm alone is folded into the out_proj prologue (PRO_GATED).

// ------------------------------------------------------------------ attention decode
// Inputs are f32, or (the *_f pointers, when set) the fixed-point accumulator of the q|k|v
// projection launch.
struct AttnCall {
  const float* qg = nullptr; const fx_t* qg_f = nullptr; int32_t ld_qg = 0;  // [B][nh*2*hd], per head [q | gate]
  const float* k = nullptr; const float* v = nullptr;   // new token's k / v rows: k[b*ld_kv + g*hd + i]
  const fx_t* k_f = nullptr; const fx_t* v_f = nullptr;
  int32_t ld_kv = 0;
  const float* qnw; const float* knw; float eps;
  const float* rcos; const float* rsin; int32_t rot;
  float* kc; float* vc; int32_t tmax;  // [B][nkv][tmax][hd]
  const int32_t* pos;                  // [B]
  float* out; int32_t ld_out;          // [B][nh*hd]
  int32_t B, nh, nkv, hd;
};
size_t attn_ws_bytes(int32_t B, int32_t nh, int32_t nkv, int32_t hd, int32_t tmax);
int attn_launch(const AttnCall& c, void* ws, size_t ws_bytes, hipStream_t st);
// same, with the completion counters and the chunk-partial scratch given separately
int attn_launch_split(const AttnCall& c, uint32_t* counters, char* scratch, size_t scratch_bytes, hipStream_t st);

// ------------------------------------------------------------------ batched projections (mvb.hip)
// Y[m][n] = X~[m][:] . dequant(W)[:, n] for up to 32 rows on the fp32 matrix cores, weights in
// the MB layout (mb_convert_launch).  X~ is x transformed by the prologue: plain, RMSNorm (with
// the rows' sums of squares `ss` from the producer), gated RMSNorm with SiLU(z) over groups of
// `group` values, or SwiGLU (up at column offset swiglu_off).  Outputs are stored, or added to y
// (residual rows) with each updated row's sum of squares added to ss_out (fixed point).
enum { MB_PRO_PLAIN = 0, MB_PRO_RMS = 1, MB_PRO_GATED = 2, MB_PRO_SWIGLU = 3 };
constexpr int kMbMaxSeg = 4;
struct MbSeg {
  const int8_t* q = nullptr;  // MB layout [N/64][K/16][64][16]
  const float* s = nullptr;   // [N/64][K]
  float* y = nullptr;         // y[m*ldy + n]
  int32_t N = 0, ldy = 0;
  // split factors [N/64] (mb_split_factor_launch, with the RMSNorm weights of the launch's
  // prologue): with them on every segment an RMS launch takes the direct path (no staging)
  const float* f = nullptr;
};
struct MbCall {
  MbSeg seg[kMbMaxSeg];
  int32_t nseg = 0;
  int32_t K = 0, M = 0;
  const float* x = nullptr; int32_t ldx = 0;
  int32_t pro = MB_PRO_PLAIN;
  const float* pw = nullptr; float eps = 1e-6f;
  const fx_t* ss = nullptr;
  const float* z = nullptr; int32_t ldz = 0, group = 0;
  int32_t swiglu_off = 0;
  int32_t add = 0; fx_t* ss_out = nullptr;
  // DeltaNet gate projection side task (raw x~ . in_proj_b | x~ . in_proj_a into aux_acc)
  const float* aux_wb = nullptr; const float* aux_wa = nullptr; int32_t aux_nh = 0;
  fx_t* aux_acc = nullptr; int32_t aux_ldo = 0;
  // split-K partials and one counter per 64-column block (zero between launches)
  float* part = nullptr; size_t part_floats = 0; uint32_t* ctr = nullptr; int32_t nctr = 0;
  float* words = nullptr; size_t word_floats = 0;  // counted split-K words (mb_word_floats), 8-byte aligned
  // defer_stride > 0 (no residual add, M <= 16): when the plan splits K in two, split s writes its
  // partial rows to seg.y + s * defer_stride and the launch ends without a hand-off;
  // *deferred_out tells.
  int64_t defer_stride = 0; int32_t* deferred_out = nullptr;
  // xsum = 2 (SwiGLU prologue, M <= 16): each input value is x[...] + x[... + xsstride], such partials
  int32_t xsum = 1; int64_t xsstride = 0;
  // the error word that receives kWsErrRange (required)
  uint32_t* err = nullptr;
  // the weights are in stream order (mb_stream_launch) rather than the MB order
  bool stream_order = false;
};
int mb_launch(const MbCall& c, hipStream_t st);
// Partial-sum floats a launch over ncb column blocks needs (0 without split-K).
size_t mb_part_floats(int ncb, int K, int M);
// Counted fixed-point split-K words of a launch of M rows over ncb column blocks (floats; a
// region of its own, zero before the first launch and left zero by every launch).
size_t mb_word_floats(int ncb, int M);
// ss[m] = fixed point of sum(x[m][k]^2, k < K) for M rows (the RMS prologue's row statistic)
int mb_row_ss_launch(const float* x, int32_t ldx, int32_t K, int32_t M, fx_t* ss, uint32_t* err, hipStream_t st);
// out[0] = max |s[i]| over n floats (one block).
int mb_scale_max_launch(const float* s, int64_t n, float* out, hipStream_t st);
// Split factors of an MB weight for RMS launches whose norm weights are norm_w.
int mb_split_factor_launch(const float* s_mb, int32_t K, int32_t N, const float* norm_w, float* f, hipStream_t st);
// MB weights in stream order: each 2 KB record (64 lanes x 32 bytes) as two 1 KB halves, lane l's
// first 16 bytes at 16 l and its second at 1024 + 16 l, so that each wave load instruction of the
// batched projections reads 1 KB contiguous (a pass that streams the weights once; the prompt
// GEMMs, which re-read them, keep the MB order).  nbytes: the MB copy's size (K * N).
int mb_stream_launch(const int8_t* q_mb, size_t nbytes, int8_t* q_stream, hipStream_t st);
// Tile-major projection weights (q[t][K][256], scale[t][K][4]; or, tiled = 0, row-major KN)
// -> MB layout.
int mb_convert_launch(const int8_t* q_tiled, const float* s_tiled, int32_t K, int32_t N, int8_t* q_mb, float* s_mb,
                      hipStream_t st, int tiled = 1);
// The lm_head's copy of the tied NK table q[V][K] in its load order (mb_lm_table_bytes bytes; K a
// multiple of 128).
size_t mb_lm_table_bytes(int32_t V, int32_t K);
int mb_lm_table_launch(const int8_t* q, int32_t V, int32_t K, int8_t* p, hipStream_t st);
// logits[m][n] = RMSNorm(h[m]) . dequant(E[n]) over the tied NK table (q: its copy in load order,
// mb_lm_table_launch; scales transposed, sT[K/64][V]), M <= 32 rows, K a multiple of 512 up to
// 2048; split16 holds 2 * M * K halves and invf M floats of scratch.
int mb_lm_head_launch(const int8_t* q, const float* sT, int32_t V, int32_t K, const float* h, int32_t ldh,
                      const float* norm_w, float eps, int32_t M, _Float16* split16, float* invf, float* y, int32_t ldy,
                      hipStream_t st);
// sT[kb][n] = s[n][kb] for the lm_head's scale table s[V][K/64].
int mb_scale_transpose_launch(const float* s, int32_t V, int32_t K, float* sT, hipStream_t st);

// ------------------------------------------------------------------ prompt (seq_len > 1) path
// *p = v on the stream (a kernel, so it can sit in a captured graph)
int store_i32_launch(int32_t* p, int32_t v, hipStream_t st);
// y[m] = RMSNorm(x[m]) * (1 + w) for M rows of K
// y = RMSNorm(x) (1 + w) per row; amax (optional): each row's max |y|.  part (optional, nsplit >
// 1): K-split partial sums of a deferred GEMM that accumulates into x: x = ((part_0 + part_1) + ...)
// + x is formed and written back to x first (split s, row m at part + s * sstride + m * ldp).
int rms_rows_launch(float* x, int ldx, int M, int K, const float* w, float eps, float* y, int ldy,
                    hipStream_t st, float* amax = nullptr, const float* part = nullptr, int nsplit = 1,
                    int64_t sstride = 0, int ldp = 0, float* clear = nullptr);
// [beta | g] rows of a prompt (x [T][ldx], softplus identity branch when its input exceeds 20)
int gate_prompt_launch(const float* x, int ldx, int T, int K, const float* wb, const float* wa, const float* alog,
                       const float* dtb, int nh, float* out, hipStream_t st);
// Gated DeltaNet over a prompt of T tokens (dk = dv = 128): causal conv continuing conv_state,
// chunked gated delta rule continuing S.  scr: nh * nchunk * kGdnScratchPerChunk floats.
constexpr int kGdnChunk = 64;
constexpr int kGdnScratchPerChunk = 4 * 64 * 128 + 64 * 64 + 64;
struct GdnPrefill {
  const float* raw = nullptr; int32_t ld_raw = 0;  // pre-conv q|k|v [T][conv_dim] (row stride ld_raw)
  const float* conv_state = nullptr;               // [conv_dim][3] before the prompt
  float* conv_state_out = nullptr;                 // written with the state after it (may alias)
  const float* conv_w = nullptr;                   // [conv_dim][4]
  const float* bg = nullptr; int32_t ld_bg = 0;    // [T][2 nh]: beta | g
  float* scr = nullptr;
  float* S = nullptr;                              // [nh][128][128], updated
  float* out = nullptr; int32_t ld_out = 0;        // [T][nh*128] core output (before the gated norm)
  int32_t T = 0, nh = 0, key_dim = 0, nchunk = 0;
  float qscale = 0.f;
};
int gdn_prefill_launch(const GdnPrefill& a, hipStream_t st);
// out[t][h*128 + i] = (w[i] * (o * rsqrt(mean(o^2) + eps))) * silu(z), per 128-wide head
int gated_norm_rows_launch(const float* o, int ldo, const float* z, int ldz, const float* w, int T, int nh, float eps,
                           float* out, int ldout, hipStream_t st, float* amax = nullptr);
// out[t][k] = gu[t][F + k] * silu(gu[t][k])
// Attention over a prompt of T tokens at positions p0..p0+T-1 (head_dim 256, one sequence).
constexpr int kHdP = 256;
struct AttnPrefill {
  const float* qg = nullptr; int32_t ld_qg = 0;  // q_proj rows, per head [query | gate]
  const float* k = nullptr; const float* v = nullptr; int32_t ld_kv = 0;
  const float* qnw = nullptr; const float* knw = nullptr; float eps = 1e-6f;
  const float* rcos = nullptr; const float* rsin = nullptr; int32_t rot = 0;
  float* kc = nullptr; float* vc = nullptr; int32_t tmax = 0;  // [nkv][tmax][256]
  int32_t p0 = 0, T = 0, nh = 0, nkv = 0;
  float* qbuf = nullptr;                        // scratch [T][nh][256]
  float* out = nullptr; int32_t ld_out = 0;     // [T][nh*256]
  float scale = 0.0625f;
};
int attn_prefill_launch(const AttnPrefill& a, hipStream_t st);

// ------------------------------------------------------------------ persistent decode step
// Per-layer pointers of the persistent decode-step kernel (Q8F projections in Q35_KN_TILED).
struct StepLayer {
  int32_t full;
  const float *in_norm, *post_norm;
  const int8_t *qkv_q, *z_q, *out_q;
  const float *qkv_s, *z_s, *out_s;
  const float *w_b, *w_a, *a_log, *dt_bias, *conv_w, *norm_w;
  float *conv_state, *rec;
  float *conv_alt, *rec_alt;  // second copies: odd steps of a launch read these and write the first
  const int8_t *q_q, *k_q, *v_q, *o_q;
  const float *q_s, *k_s, *v_s, *o_s;
  const float *q_norm, *k_norm;
  float *kc, *vc;
  const int8_t *gate_q, *up_q, *down_q;
  const float *gate_s, *up_s, *down_s;
};
// split-K plan of one matvec stage: item = (256-column tile, chunk of kch rows)
struct StepMv { int32_t kch, nchunk; };
enum { SMV_QKVZ = 0, SMV_OUT, SMV_QKV, SMV_O, SMV_GU, SMV_DOWN, SMV_COUNT };
struct StepArgs {
  const StepLayer* layers;
  int32_t n_layers;
  int32_t H, F, V, nh, dk, dv, conv_dim, key_dim, vdim, ah, kvh, hd, rot, tmax;
  float eps, qscale, ascale;
  StepMv mv[SMV_COUNT];
  const int8_t* emb_q; const float* emb_s; const float* final_norm;
  const float *rope_cos, *rope_sin;
  // Counted fixed-point accumulators (value * 2^32 plus one 2^56 per contribution; see step.hip),
  // one set per token parity: token t uses set t & 1, and the lm stage of token t clears the
  // other set for token t + 1.
  fx_t* h;              // [2][n_res][2 * H] residual stream, one copy per residual stage (n_res = 2 n_layers):
                        // value k at k + (k & ~15) (one 128-byte line per 256 bytes)
  int32_t n_res;
  fx_t* acc;            // [2][acc_par]: [n_layers][acc_stride] per layer: projections | gate|up | in_proj_b|a sums
  int64_t acc_stride;   // fx_t entries per layer
  int64_t acc_gu_off, acc_ba_off;  // offsets of the gate|up and the b|a sums inside a layer's entries
  int64_t acc_par;      // fx_t entries per parity set (n_layers * acc_stride)
  // Attention partials, tagged: (tag << 32) | f32 bits, tag = a number unique to the token and layer
  uint64_t *att_ml, *att_o;
  int32_t att_nmax;     // attention chunks per kv head
  float* logits;        // may be null
  uint64_t* argp;       // per-block argmax partials [2][grid] (token parity): tag (14 bits) | index (18 bits) | f32 value
  uint32_t* tokseq;     // tokens the kernel has run since the last model reset (selects the parity set)
  int32_t *token, *pos, *prompt, *plen, *hist;
  // Token stream (null: none): device address of pinned, coherent host memory [tmax]; a
  // non-null pointer selects the streamed build, whose block 0 stores each token there, with one
  // system-scope store, as it records it in hist
  int32_t* tok_host;
  ArgOrder ord;         // the reference's argmax order over the vocabulary
  // Stop ids (main.rs:108-110): a generated step (position >= plen) whose input token is one of
  // them is not run; the launch ends there (pos = that position, token = the stop id).
  int32_t stop_ids[4];
  int32_t n_stop;
  // Sticky error word (its own allocation, cleared only by a model reset): bit 0 is set when a
  // wait for another block's results times out, bit 1 when a value to be accumulated in fixed
  // point is not finite or too large (|v| >= 2^22).  Every launch that finds it set at entry
  // returns at once without touching any state, so one failure cannot be followed by launches
  // that compute on a broken state.
  uint32_t* err;
  int32_t ntok;
};
constexpr uint32_t kStepErrTimeout = 1u, kStepErrRange = 2u;
// Every block of the qkvz stage adds into the 2 x lin_heads gate accumulators; packed, they
// would share two cache lines and the atomics would serialise on them.
constexpr int kStepBaStride = 16;  // fx_t entries (128 bytes)
constexpr int kStepThreads = 512;
// Blocks of the persistent kernel that fit co-resident (one per CU); 0 if the kernel cannot run.
int step_grid(int hidden);
// Attention chunks per kv head for a grid (the merge keeps their weights in LDS).
int step_att_nmax(int grid, int kvh);
// Checks dims / tmax against the kernel's limits.
int step_validate(const q35_dims& d, int tmax, int grid);
// Plans the split-K of every matvec stage for `grid` blocks.
void step_plan(const q35_dims& d, int grid, StepMv* mv);
int step_launch(const StepArgs& a, int grid, hipStream_t st);

}  // namespace q35
