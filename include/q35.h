/*
 * q35.h — C ABI of the MI355X (gfx950) decode hot path for the Qwen3.5-2B-shaped hybrid
 * decoder (Gated DeltaNet + gated GQA attention, Q8F weights).
 *
 * Every entry point replaces one function of the reference engine (inventwithdean/Qwen-3.5);
 * the citation beside each declaration names the file:line it replaces.  The reference reaches
 * these through `#[backend_extension(Cube, Fusion)] trait CustomKernels` (src/kernels.rs:373-433)
 * and the `seq_len == 1` branches of src/text_modules.rs; here they are plain C functions.
 *
 * Conventions
 *   - All tensor arguments are DEVICE pointers (hipMalloc'd) unless the name ends in `_host`.
 *   - `stream` is a hipStream_t passed as void* (NULL = the default stream).  Calls are
 *     stream-ordered and asynchronous; no entry point synchronises the device.
 *   - The caller owns every buffer.  Entry points that need scratch take `ws`/`ws_bytes`; the
 *     required size comes from the matching *_ws_bytes() query.  A workspace must be zero-filled
 *     once before its first use and then serve one entry point with one set of sizes (B, tmax):
 *     every call leaves the parts that must start at zero (completion counters, fixed-point
 *     split-K accumulators) zero again, so later such calls on the same stream can reuse it.
 *     The layout depends on the entry point and its sizes (use one workspace per combination,
 *     or re-zero it), and calls running concurrently need distinct workspaces.
 *   - Return value: Q35_OK or a Q35_E_* code; q35_last_error() gives a message.  Nothing aborts.
 *   - Q8F: int8 two's complement values plus one f32 scale per block of 64 consecutive elements
 *     along the stored matrix's contiguous axis; dequant = f32(q) * scale (kernels.rs:34-43,84-88).
 */
#ifndef Q35_H
#define Q35_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  Q35_OK = 0,
  Q35_E_SHAPE = 1,   /* a dimension violates the kernel contract (multiple of 64, limits) */
  Q35_E_ALIGN = 2,   /* a pointer is not 16-byte aligned */
  Q35_E_HIP = 3,     /* a HIP runtime call failed */
  Q35_E_ARG = 4,     /* NULL pointer or invalid enum */
  Q35_E_WS = 5,      /* workspace smaller than the *_ws_bytes() requirement */
  Q35_E_NOMEM = 6,   /* device or host allocation failed (model creation only) */
  Q35_E_RANGE = 7,   /* a value bound for a fixed-point accumulator was not finite or out of
                        range (|v| >= 2^31; 2^22 in the persistent step kernel): it was dropped and
                        the results of the calls since the last check are invalid.  Where the
                        reference's f32 sums would carry a NaN / Inf on, the split-K fixed-point
                        sums cannot hold one, so the library reports it instead. */
};

/* Storage layouts of a Q8F matrix.
 *   Q35_KN: q is [rows=K(in)][cols=N(out)], scale is [K][N/64]  — Burn Linear weight of the
 *           reference projections, blocks along N (kernels.rs:56-57,75-76,87).
 *   Q35_NK: q is [rows=N(out)][cols=K(in)], scale is [N][K/64]  — the tied embedding table
 *           used as lm_head, blocks along K (kernels.rs:253-255,283).
 *   Q35_KN_TILED: the Q35_KN matrix (rows=K, cols=N) re-laid out by q35_q8f_pack_kn_tiled into
 *           256-column tiles stored one after another: q[t][K][256], scale[t][K][4] for
 *           t < ceil(N/256) (columns past N zero).  Same values, so results are identical to
 *           Q35_KN; every K-chunk of a tile is one contiguous run of HBM, which is how the
 *           matvec streams it.
 *   Q35_KN_PANEL: the Q35_KN matrix re-laid out by q35_q8f_pack_kn_panel into 16-column panels,
 *           q[N/16][K][16], with the scales transposed to scale[N/64][K].  Same values and byte
 *           count; each panel (16 outputs over all of K) is one contiguous run, so the standalone
 *           matvec computes it in one block with no cross-block reduction and no workspace.
 *           Accepted by q35_q8_gemv / q35_q8_gemv_partial_sum only.
 *   Q35_KN_MB: the Q35_KN matrix re-laid out on the device by q35_q8f_pack_mb for the f16
 *           matrix cores: per 64-column block cb and 32-row step ks a 2 KB record in which lane
 *           l = 16 g + c of a 64-lane wave finds the bytes q + 128 of rows 32 ks + 8 g + j
 *           (j < 8) of columns 64 cb + 16 t + c, t < 4 (its operands of four 16x16x32 MFMAs);
 *           scales transposed to scale[N/64][K].  Same values and byte count.  Accepted by
 *           q35_q8_gemm_ws only (K and N multiples of 128). */
enum { Q35_KN = 0, Q35_NK = 1, Q35_KN_TILED = 2, Q35_KN_PANEL = 3, Q35_KN_MB = 4 };

typedef struct {
  const int8_t* q;
  const float* scale;
  int32_t rows;
  int32_t cols;
  int32_t layout; /* Q35_KN, Q35_NK, Q35_KN_TILED, Q35_KN_PANEL or Q35_KN_MB */
} q35_q8f;

/* Shape constants of the decoder; mirrors the fields of TextConfig that the decode path
 * reads (src/text_config.rs:56-126).  q35_dims_qwen35_2b() returns the 2B values. */
typedef struct {
  int32_t hidden, ffn, vocab, n_layers, full_interval;
  int32_t lin_heads, lin_dk, lin_dv, conv_k;
  int32_t attn_heads, kv_heads, head_dim, rot_dim;
  float eps, theta;
} q35_dims;

const char* q35_last_error(void);
q35_dims q35_dims_qwen35_2b(void);

/* ---------------------------------------------------------------- tensor level (kernels.rs) */

/* y[M][N] = x[M][K] @ dequant(W).  W.layout selects KN (reference projections), its tiled or
 * panel re-layouts, or NK.  Full-K semantics (every input row is summed).  M in [1, 64]; K, N
 * multiples of 64.  One kernel launch per 8 rows of x (Q35_KN_PANEL needs no workspace: ws may
 * be NULL).  Replaces q8_gemv (src/kernels.rs:681-688, kernel :53-92). */
int q35_q8_gemv(const float* x, int32_t M, q35_q8f W, float* y, void* ws, size_t ws_bytes, void* stream);

/* Same contract; replaces q8_gemv_partial_sum (src/kernels.rs:690-700, impl :495-537, kernels
 * :103-165) whose split-K reduction is done here deterministically inside one launch. */
int q35_q8_gemv_partial_sum(const float* x, int32_t M, q35_q8f W, float* y, void* ws, size_t ws_bytes, void* stream);
size_t q35_q8_gemv_ws_bytes(int32_t M, q35_q8f W);

/* q35_q8_gemv without a workspace and without any allocation: no counterpart in the reference;
 * for callers that cannot allocate device memory (code under hipGraph capture, serving loops,
 * harnesses that forbid hipMalloc).  Same results as q35_q8_gemv (the same kernels).  The
 * Q35_KN / Q35_KN_TILED split-K scratch is a fixed 1 MiB + 64 KiB device array per GPU (held
 * until the process ends), so min(M, 8) * N must be <= 131072 (else Q35_E_SHAPE); the panel and
 * NK layouts need no scratch.  Every call on one GPU shares that GPU's array, which each call
 * leaves zeroed: calls that overlap on one GPU (different streams, concurrent graph replays)
 * race and must be serialised by the caller. */
int q35_q8_gemv_noalloc(const float* x, int32_t M, q35_q8f W, float* y, void* stream);

/* logits[M][V] = h[M][D] @ dequant(E)^T with E the NK [V][D] embedding table.
 * Replaces q8_lm_head (src/kernels.rs:724-731, kernel :251-291). */
int q35_q8_lm_head(const float* h, int32_t M, q35_q8f E, float* logits, void* stream);

/* out[n][D] = dequant(table[ids[i]]).  Replaces q8_embedding_lookup (src/kernels.rs:669-679,
 * kernel :15-45).  ids must lie in [0, V). */
int q35_q8_embedding_lookup(q35_q8f table, const int32_t* ids, int32_t n, float* out, void* stream);

/* out[b] = [beta(n_heads) | g(n_heads)] with beta = sigmoid(x.W_b), g = -exp(A_log) *
 * softplus(x.W_a + dt_bias) (softplus branch x when ln(1+e^x) > 20).  x [B][in_dim];
 * W_b, W_a f32 [in_dim][n_heads].  Replaces gate_proj (src/kernels.rs:702-722, kernel :174-247). */
int q35_gate_proj(const float* x, int32_t B, int32_t in_dim, const float* w_b, const float* w_a,
                  const float* a_log, const float* dt_bias, int32_t n_heads, float* out, void* stream);

/* out[0] = index of the largest logit.  Exact ties resolve as the reference's two-stage argmax
 * does: with c = n/8 and i = k*c + p, the winner minimises (p mod 256, p div 256, k) — the
 * first strict maximum of its scans.  The last n mod 8 values, which the reference never reads,
 * are read here and rank after all others on ties; NaN is never returned (all NaN -> 0).
 * Replaces argmax (src/kernels.rs:733-739, kernels :298-371). */
int q35_argmax(const float* logits, int64_t n, int32_t* out, void* ws, size_t ws_bytes, void* stream);
size_t q35_argmax_ws_bytes(int64_t n);

/* ---------------------------------------------------------------- layer level (text_modules.rs) */

/* Projection weights of the layer entry points: Q35_KN or Q35_KN_TILED (rows = in, cols = out). */
typedef struct {
  q35_q8f in_proj_qkv; /* KN [hidden][2*key_dim+value_dim] */
  q35_q8f in_proj_z;   /* KN [hidden][value_dim] */
  q35_q8f out_proj;    /* KN [value_dim][hidden] */
  const float* in_proj_b; /* f32 [hidden][lin_heads] */
  const float* in_proj_a; /* f32 [hidden][lin_heads] */
  const float* a_log;     /* [lin_heads] */
  const float* dt_bias;   /* [lin_heads] */
  const float* conv_w;    /* [conv_dim][conv_k] */
  const float* norm_w;    /* [lin_dv] */
} q35_gdn_weights;

typedef struct {
  q35_q8f q_proj; /* KN [hidden][attn_heads*head_dim*2], per head [query | gate] */
  q35_q8f k_proj; /* KN [hidden][kv_heads*head_dim] */
  q35_q8f v_proj; /* KN [hidden][kv_heads*head_dim] */
  q35_q8f o_proj; /* KN [attn_heads*head_dim][hidden] */
  const float* q_norm; /* [head_dim], applied as (1 + w) */
  const float* k_norm; /* [head_dim] */
} q35_attn_weights;

typedef struct {
  q35_q8f gate_proj, up_proj, down_proj; /* KN */
} q35_mlp_weights;

/* One decode token through GatedDeltaNet for B rows.  x: [B][hidden] (already input-normed);
 * conv_state: [B][conv_dim][conv_k-1]; rec_state: [B][lin_heads][lin_dk][lin_dv] (both updated
 * in place); out: [B][hidden].  Replaces GatedDeltaNet::forward's seq_len==1 branch with cached
 * states (src/text_modules.rs:484-667). */
int q35_gated_deltanet_decode(const q35_dims* d, const q35_gdn_weights* w, const float* x, int32_t B,
                              float* conv_state, float* rec_state, float* out,
                              void* ws, size_t ws_bytes, void* stream);

/* One decode token through gated GQA attention for B rows.  k_cache/v_cache:
 * [B][kv_heads][tmax][head_dim]; d_pos[b] = tokens already cached for row b (the new K/V are
 * written at that index, then attention runs over d_pos[b]+1 tokens); d_pos[b] must lie in
 * [0, tmax): a row whose position does not is skipped and reported by q35_workspace_status;
 * rope_cos/rope_sin:
 * [tmax][rot_dim] from q35_rope_tables.  Replaces Attention::forward's seq_len==1 branch
 * (src/text_modules.rs:842-944). */
int q35_attention_decode(const q35_dims* d, const q35_attn_weights* w, const float* x, int32_t B,
                         float* k_cache, float* v_cache, int32_t tmax, const int32_t* d_pos,
                         const float* rope_cos, const float* rope_sin, float* out,
                         void* ws, size_t ws_bytes, void* stream);

/* down(up(x) * silu(gate(x))) for B rows.  Replaces MLP::forward (src/text_modules.rs:1000-1011). */
int q35_mlp_decode(const q35_dims* d, const q35_mlp_weights* w, const float* x, int32_t B, float* out,
                   void* ws, size_t ws_bytes, void* stream);

/* The recurrent core of GatedDeltaNet for one token, B rows: causal conv update + SiLU on the
 * mixed q|k|v channels, l2norm(q)*dk^-1/2, l2norm(k), S = e^g S; S += k (x) (v - S^T k) beta;
 * out = S^T q.  mixed_qkv: [B][2*key_dim+value_dim] (pre-conv projection output); beta_g:
 * [B][2*lin_heads] = [beta | g] as q35_gate_proj produces; conv_state [B][conv_dim][3] and
 * rec_state [B][lin_heads][128][lin_dv] updated in place; core_out: [B][lin_heads*lin_dv] (before
 * the gated norm).  ws (optional): a zeroed workspace of at least 64 KiB lets one kernel also
 * advance the conv state (left zeroed for the next call); with ws NULL a second kernel does it.
 * Replaces causal_conv1d_update + burn_recurrent_gated_delta_rule (src/text_modules.rs:134-162,
 * :365-443) as called at :515-530, :627-652. */
int q35_gated_delta_rule_decode(const float* mixed_qkv, int32_t B, const float* beta_g, float* conv_state,
                                const float* conv_w, float* rec_state, float* core_out, int32_t lin_heads,
                                int32_t lin_dk, int32_t lin_dv, void* ws, size_t ws_bytes, void* stream);

/* The attention core for one token, B rows: q_norm/k_norm (1+w), RoPE, K/V append at d_pos[b],
 * softmax(q K^T/sqrt(256)) V with GQA, times sigmoid(gate).  q_gate: [B][attn_heads*2*head_dim]
 * (q_proj output, per head [query | gate]); k_new, v_new: [B][kv_heads*head_dim] (k_proj / v_proj
 * outputs, ld = kv_ld floats between rows); out: [B][attn_heads*head_dim].  Replaces the part of
 * Attention::forward between the projections (src/text_modules.rs:860-936). */
int q35_attention_core_decode(const q35_dims* d, const float* q_gate, const float* k_new, const float* v_new,
                              int32_t kv_ld, int32_t B, const float* q_norm, const float* k_norm, float* k_cache,
                              float* v_cache, int32_t tmax, const int32_t* d_pos, const float* rope_cos,
                              const float* rope_sin, float* out, void* ws, size_t ws_bytes, void* stream);

/* Workspace large enough for any of the layer calls above with these B / tmax. */
size_t q35_layer_ws_bytes(const q35_dims* d, int32_t B, int32_t tmax);

/* Device-side errors recorded in a layer workspace by earlier calls on `stream` (synchronises
 * it), then cleared.  Q35_E_SHAPE: an attention call met a position d_pos[b] outside [0, tmax);
 * that row's cache and output were left untouched.  Q35_E_RANGE: a projection or gate sum met a
 * non-finite value or one of magnitude >= 2^31 (an input row holding NaN / Inf or overflowing
 * values); it was dropped, so the outputs of the calls since the last check are invalid.  Both
 * bits may be set; Q35_E_SHAPE is reported first.  Also reads the q35_q8_gemv workspace.  No
 * reference counterpart (the reference panics on a bad position on the host, text_modules.rs, and
 * carries a NaN through its f32 sums); it exists because the positions live in device memory,
 * where the host cannot check them without a synchronisation, and because the fixed-point sums
 * cannot hold a NaN. */
int q35_workspace_status(void* ws, void* stream);

/* Host: cos/sin tables [tmax][rot_dim] of TextRotaryEmbedding::forward for positions 0..tmax-1
 * (src/text_modules.rs:30-43,73-81; the mRoPE recomposition :45-58 is the identity for text). */
int q35_rope_tables(const q35_dims* d, int32_t tmax, float* cos_host, float* sin_host);

/* ---------------------------------------------------------------- prompt path (seq_len > 1) */

/* y[M][N] (+)= x[M][K] @ dequant(W) on the fp32 matrix cores: each weight is dequantised to f32
 * (f32(q) * scale) and the products are summed in f32, as the reference's Linear::forward on a
 * QFloat weight does for a prompt (dequantise, f32 matmul: text_modules.rs:500-508, :578-595,
 * :638-647, :880-890, :1003-1005).  W: Q35_KN / Q35_KN_TILED (K = rows, N = cols) or Q35_NK
 * (N = rows, K = cols: the tied lm_head matmul of model.rs:130-138).  x rows ldx floats apart
 * (16-byte aligned), y rows ldy apart; accumulate = 1 adds into y (a residual add).  K, N
 * multiples of 64; any M >= 1. */
int q35_q8_gemm(const float* x, int32_t M, int32_t ldx, q35_q8f W, float* y, int32_t ldy, int32_t accumulate,
                void* stream);
/* The same with a workspace of q35_q8_gemm_ws_bytes(M, W) bytes: the launcher may then split K
 * over more blocks (for shapes with few output tiles, e.g. the 2048-wide out / o / down
 * projections) and add the splits' partial sums in a fixed order in a second kernel.  Results
 * differ from q35_q8_gemm only in f32 summation order.  ws = NULL behaves as q35_q8_gemm.
 * W in Q35_KN_MB (a workspace is then required) runs on the f16 matrix cores with f32-equivalent
 * products: the int8 values are exact in f16, each block scale multiplies x instead, and x * scale
 * is carried as two f16 halves hi + lo (~22 significant bits, with a power-of-two factor per row
 * of x chosen from the row's largest |x| and the matrix's largest scale) whose products with q
 * are exact in the f32 accumulator; results differ from the fp32 path by f32 rounding. */
size_t q35_q8_gemm_ws_bytes(int32_t M, q35_q8f W);
int q35_q8_gemm_ws(const float* x, int32_t M, int32_t ldx, q35_q8f W, float* y, int32_t ldy, int32_t accumulate,
                   void* ws, size_t ws_bytes, void* stream);

/* The batched decode's projection (the kernel behind q35_batch_*) on its own: y[m][n] (+)=
 * in[m][:] . dequant(W)[:, n] for M <= 32 rows on the f16 matrix cores (x * scale as f16 hi + lo,
 * about 22 significant bits; f32 accumulation), W in Q35_KN_MB (rows = K, cols = N, both multiples
 * of 128).  The prologue forms in[m] from the x row (ldx floats apart, 16-byte aligned):
 *   Q35_MB_PLAIN   in = x;
 *   Q35_MB_RMS     in = x * rsqrt(mean(x^2) + eps) * (1 + norm_w) (RMSNorm, text_modules.rs:801-809;
 *                  the row statistic is formed here, the matrix's split factors too);
 *   Q35_MB_GATED   in = RMSNormGated(x, z) over groups of `group` (a power of two, 16..128):
 *                  x * rsqrt(mean_group(x^2) + eps) * norm_w * silu(z) (text_modules.rs:91-101),
 *                  z rows ldz floats apart;
 *   Q35_MB_SWIGLU  in[k] = x[K + k] * silu(x[k]) (x rows hold gate then up, ldx >= 2 K;
 *                  text_modules.rs:1005).
 * accumulate = 1 adds into y (a residual add).  Needs q35_q8_gemv_mb_ws_bytes(M, W) bytes of
 * workspace; range errors are reported by q35_workspace_status.  No reference counterpart (the
 * reference decodes one sequence): it is exposed for callers that batch rows themselves and for
 * per-projection parity tests of the batched path. */
enum { Q35_MB_PLAIN = 0, Q35_MB_RMS = 1, Q35_MB_GATED = 2, Q35_MB_SWIGLU = 3 };
size_t q35_q8_gemv_mb_ws_bytes(int32_t M, q35_q8f W);
int q35_q8_gemv_mb(const float* x, int32_t M, int32_t ldx, int32_t prologue, const float* norm_w, const float* z,
                   int32_t ldz, int32_t group, float eps, q35_q8f W, float* y, int32_t ldy, int32_t accumulate,
                   void* ws, size_t ws_bytes, void* stream);

/* out[t] = [beta | g] for T prompt rows, as the prompt branch computes them
 * (text_modules.rs:578-595): beta = sigmoid(x.W_b), g = -exp(A_log) * softplus(x.W_a + dt_bias)
 * with softplus's identity branch taken when its INPUT exceeds 20 (decode, q35_gate_proj,
 * tests the result). */
int q35_gate_proj_prompt(const float* x, int32_t T, int32_t in_dim, const float* w_b, const float* w_a,
                         const float* a_log, const float* dt_bias, int32_t n_heads, float* out, void* stream);

/* The recurrent core of GatedDeltaNet over T prompt tokens of one sequence (dk = dv = 128):
 * causal conv1d + SiLU over the prompt continuing conv_state (causal_conv1d_fn with the cached
 * state prepended, text_modules.rs:164-182,531-554), l2norm(q)*dk^-1/2, l2norm(k), and the
 * chunked gated delta rule (chunks of 64) continuing rec_state (burn_chunk_gated_delta_rule,
 * :189-363, as called at :627-652).  mixed_qkv: [T][ld_qkv] pre-conv projection rows;
 * beta_g: [T][2*lin_heads] from q35_gate_proj_prompt; conv_state [conv_dim][3] and rec_state
 * [lin_heads][128][128] are updated in place to the state after the prompt; core_out:
 * [T][lin_heads*128] (before the gated norm).  ws: q35_gated_delta_rule_prefill_ws_bytes(T,
 * lin_heads) bytes of scratch (no zeroing needed). */
int q35_gated_delta_rule_prefill(const float* mixed_qkv, int32_t T, int32_t ld_qkv, const float* beta_g,
                                 float* conv_state, const float* conv_w, float* rec_state, float* core_out,
                                 int32_t lin_heads, int32_t lin_dk, int32_t lin_dv, void* ws, size_t ws_bytes,
                                 void* stream);
size_t q35_gated_delta_rule_prefill_ws_bytes(int32_t T, int32_t lin_heads);

/* The attention core for T prompt tokens of one sequence at positions p0..p0+T-1: q_norm/k_norm
 * (1+w), RoPE, K/V appended at rows p0..p0+T-1 of k_cache/v_cache [kv_heads][tmax][256],
 * causal GQA softmax(q K^T / 16) V over rows 0..p0+t (the mask of model.rs:59-61), times
 * sigmoid(gate).  q_gate: [T][ld_qg] q_proj rows (per head [query | gate]); k_new, v_new:
 * [T][kv_ld]; out: [T][attn_heads*256].  Replaces the prompt branch of Attention::forward
 * between the projections (text_modules.rs:860-936).  ws: q35_attention_prefill_ws_bytes. */
int q35_attention_core_prefill(const q35_dims* d, const float* q_gate, int32_t ld_qg, const float* k_new,
                               const float* v_new, int32_t kv_ld, int32_t T, int32_t p0, const float* q_norm,
                               const float* k_norm, float* k_cache, float* v_cache, int32_t tmax,
                               const float* rope_cos, const float* rope_sin, float* out, void* ws, size_t ws_bytes,
                               void* stream);
size_t q35_attention_prefill_ws_bytes(const q35_dims* d, int32_t T);

/* ---------------------------------------------------------------- model level (model.rs, main.rs) */

typedef struct q35_model q35_model;

/* Builds the decoder with seeded random-init weights, the reference's init rules
 * (LinearConfig::init / EmbeddingConfig::init drawn N(0, 0.02) here, RMSNorm w=0, gated-norm
 * w=1, dt_bias=1, A_log=ln U(0.01,16), text_modules.rs:698-700,820,111) and Q8F quantisation of
 * the tensors main.rs:159-222 quantises.  Allocates weights, caches for tmax tokens and the step
 * workspace.  Replaces TextForCausalLMConfig::init + load_file (main.rs:29-37). */
int q35_model_create_synthetic(const q35_dims* d, uint64_t seed, int32_t tmax, q35_model** out);

/* Builds the decoder from a Hugging Face safetensors checkpoint as the reference's loader does
 * (main.rs:160-222): keys `model.language_model.<path>` (or without the `model.` prefix, which
 * the reference strips), `.A_log` read as `.a_log`; Linear weights transposed from PyTorch's
 * [out][in] to [in][out] (PyTorchToBurnAdapter); F32 / F16 / BF16 values cast to f32
 * (FloatCastAdapter); embed_tokens, the MLP, attention and DeltaNet in/out projections quantised
 * to Q8F per block of 64 (main.rs:175-220), everything else (norms, in_proj_b / in_proj_a, conv1d,
 * A_log, dt_bias) kept f32.  A missing tensor, a shape that disagrees with d, or an unsupported
 * dtype is reported (Q35_E_ARG / Q35_E_SHAPE), naming the key.  Tensors the decoder does not
 * read (lm_head with tied embeddings, vision tower, ...) are ignored. */
int q35_model_create_from_safetensors(const q35_dims* d, const char* path, int32_t tmax, q35_model** out);
int q35_model_destroy(q35_model* m);

/* Zero every cache and set the position to 0 (the chat loop's /reset, main.rs:65-71).  Also
 * clears a persistent-kernel failure recorded by q35_model_check. */
int q35_model_reset(q35_model* m, void* stream);

/* Write the next input token (host value) into the model's device token slot. */
int q35_model_set_token(q35_model* m, int32_t token, void* stream);

/* How a decode step is launched (the `use_graph` / `mode` arguments below):
 *   Q35_LAUNCH_STREAM      the step's ~120 fused kernels launched one by one on the stream;
 *   Q35_LAUNCH_GRAPH       the same kernels as a hipGraph captured on first use on this stream;
 *   Q35_LAUNCH_PERSISTENT  one cooperative launch of the persistent step kernel (one block per
 *                          CU; stages hand data over through counted and tagged words, no grid
 *                          barrier) that runs any number of consecutive steps; fastest.  Needs
 *                          hidden <= 4096, DeltaNet heads of dk = dv = 128, attention head_dim
 *                          256, tmax <= 2048 * min(256, CUs / kv_heads) (262144 for the 2B shape
 *                          on 256 CUs) and the device to co-schedule the grid
 *                          (q35_model_persistent_info). */
enum { Q35_LAUNCH_STREAM = 0, Q35_LAUNCH_GRAPH = 1, Q35_LAUNCH_PERSISTENT = 2 };

/* One decode step: reads the device token slot, runs embedding -> layers -> norm -> lm_head ->
 * argmax, writes the argmax back into the token slot and advances the device position.
 * Replaces TextForCausalLM::forward (model.rs:113-129) + kernels::argmax (main.rs:131).
 * use_graph: a Q35_LAUNCH_* mode. */
int q35_model_step(q35_model* m, int32_t use_graph, void* stream);

/* n_steps consecutive decode steps (each one's argmax feeds the next, or the prompt id while the
 * position is inside the prompt given to q35_model_generate); asynchronous on the stream.  In
 * Q35_LAUNCH_PERSISTENT mode all steps are one kernel launch. */
int q35_model_decode(q35_model* m, int32_t n_steps, int32_t mode, void* stream);

/* Synchronises the stream and reports a failure of the launches since the last check:
 * Q35_E_HIP for a persistent-kernel wait that timed out (the kernel then exits early and its
 * results are invalid), Q35_E_RANGE for a non-finite or out-of-range value met by a fixed-point
 * accumulator in any launch mode.  Q35_OK otherwise.  A persistent-kernel failure is sticky: it
 * is kept in device memory that no launch clears, every later persistent launch returns at entry
 * without touching the model state, and q35_model_step / _decode / _generate refuse persistent
 * mode once a check has seen it, until q35_model_reset.  q35_model_generate / _generate_until /
 * _decode_until run this check themselves. */
int q35_model_check(q35_model* m, void* stream);

/* Grid of the persistent step kernel (blocks, one per CU); returns an error code and message
 * when the persistent mode is unavailable for this model or device. */
int q35_model_persistent_info(q35_model* m, int32_t* grid_out);

/* Greedy generation (main.rs:100-132 without tokenizer or stop tokens): feeds the n_prompt
 * prompt ids one decode step at a time, then runs n_new decode steps.  out_tokens_host receives
 * n_new+1 ids: the argmax after the last prompt token, then the argmax after each decode step.
 * readback_each=1 copies each token to the host and synchronises per step as main.rs:107
 * does (in persistent mode: one launch per decode step; otherwise the prompt and the n_new
 * steps are one launch each).  decode_seconds_host (optional) receives the wall time of the
 * n_new decode steps.  use_graph: a Q35_LAUNCH_* mode. */
int q35_model_generate(q35_model* m, const int32_t* prompt_host, int32_t n_prompt, int32_t n_new,
                       int32_t* out_tokens_host, int32_t use_graph, int32_t readback_each,
                       double* decode_seconds_host, void* stream);

/* Greedy generation with stop ids, as the chat loop of main.rs:100-132 runs it: the prompt is fed
 * (n_prompt ids), then up to max_new steps; before each step the current token (the argmax
 * after the previous position) is compared with the n_stop (<= Q35_MAX_STOP_IDS) stop ids
 * (<|im_end|> and eos, main.rs:105-110) and the loop ends at the first match, which is not
 * forwarded.  out_tokens_host (room for max_new + 1) receives the *n_out_host produced ids (each
 * forwarded), then the id that ended the loop: the stop id, or the unforwarded argmax after the
 * last produced id when max_new were produced.  Afterwards the position is
 * start + n_prompt + *n_out_host and the token slot holds that last id, so the caller can forward
 * <|im_end|> as main.rs:141-144 does (q35_model_set_token + q35_model_step).  In
 * Q35_LAUNCH_PERSISTENT mode the generated steps are one launch that ends itself at a stop id
 * (no host round trip per token); the other modes read each token back as main.rs:107 does. */
#define Q35_MAX_STOP_IDS 4
int q35_model_generate_until(q35_model* m, const int32_t* prompt_host, int32_t n_prompt, int32_t max_new,
                             const int32_t* stop_ids_host, int32_t n_stop, int32_t* out_tokens_host,
                             int32_t* n_out_host, int32_t use_graph, double* decode_seconds_host, void* stream);

/* The prompt path: feeds n_prompt ids (host) at the current position as one forward at
 * seq_len = n_prompt, as TextForCausalLM::forward does for a prompt (model.rs:27-84,130-138;
 * main.rs:88-95): every projection is a Q8F GEMM on the fp32 matrix cores (f32 dequant, f32
 * products and accumulation), the Gated DeltaNet layers run the causal conv over the prompt
 * (continuing the cached conv state) and the chunked gated delta rule (chunks of 64, continuing
 * the cached recurrent state; text_modules.rs:164-182,189-363), the attention layers causal
 * attention over the cache.  Only the last row goes through the final norm and the lm_head (the
 * only logits the greedy loop reads); its argmax is left in the token slot, so decoding
 * continues from there.  Asynchronous after the prompt upload; prompts longer than the internal
 * pass size (1024) run in consecutive passes.  OR Q35_PREFILL_GEMM into the mode argument of
 * q35_model_generate / q35_model_generate_until to feed their prompt this way. */
#define Q35_PREFILL_GEMM 0x100
int q35_model_prefill(q35_model* m, const int32_t* prompt_host, int32_t n_prompt, void* stream);

/* The decode half of q35_model_generate_until from the current position: the token slot (the
 * argmax after the last fed token) is the first current token; up to max_new steps, ending at
 * the first current token that is a stop id.  Same outputs.  For a chat loop that feeds a turn
 * with q35_model_prefill and then streams the reply in chunks (main.rs:100-132). */
int q35_model_decode_until(q35_model* m, int32_t max_new, const int32_t* stop_ids_host, int32_t n_stop,
                           int32_t* out_tokens_host, int32_t* n_out_host, int32_t use_graph,
                           double* decode_seconds_host, void* stream);

/* Streamed decode: up to max_steps steps as one persistent launch (Q35_LAUNCH_PERSISTENT only),
 * returning once the launch is enqueued.  The token each step produces — the argmax after
 * position q, q = position before the call .. + max_steps - 1, the same values as hist[q] — is
 * stored by the running kernel into slot q of q35_model_token_stream() as soon as the device
 * knows it; the call first sets those slots to -1, so a host thread reads each token by waiting
 * for its slot to become >= 0, while the device runs on (main.rs:100-107 prints each token as it
 * is made; here without a per-step synchronisation).  With stop ids (0..4, main.rs:105-110) the
 * launch ends before a step whose input token is one of them, so the last slot written holds that
 * stop id and the later ones stay -1: stop reading there.  Then call q35_model_stream_end before
 * any other call on the model.  The tokens are identical to q35_model_decode's (_decode_until's
 * with stop ids). */
int q35_model_decode_stream(q35_model* m, int32_t max_steps, const int32_t* stop_ids_host, int32_t n_stop,
                            void* stream);

/* Ends a streamed decode: synchronises, reports a failed launch as q35_model_check does, sets the
 * model's position to where the launch ended and writes the steps it ran to *n_steps_out
 * (optional). */
int q35_model_stream_end(q35_model* m, int32_t* n_steps_out, void* stream);

/* The model's host token stream: pinned, coherent host memory of tmax slots written by
 * q35_model_decode_stream launches (read them as volatile); valid until q35_model_destroy. */
const int32_t* q35_model_token_stream(q35_model* m);

/* Tokens consumed so far (the cache length that TextModel::forward derives positions from,
 * model.rs:37-43). */
int q35_model_position(q35_model* m, int32_t* pos_out);

/* Device pointer and byte size of a named model tensor, named as the reference's module
 * paths: "embed_tokens", "norm", "layers.{i}.input_layernorm", "layers.{i}.linear_attn.in_proj_qkv"
 * (".q" / ".scale" suffix for the Q8F parts; projections are held in the Q35_KN_TILED layout,
 * the embedding table in Q35_NK), "...conv_state", "...recurrent_state",
 * "layers.{i}.self_attn.k_cache", "logits", "token", "pos", ...  Used by tests and tools. */
int q35_model_tensor(q35_model* m, const char* name, void** dptr, size_t* bytes);

/* ---------------------------------------------------------------- batched decode */

/* B independent sequences decoded together with one model's weights (the reference decodes one
 * sequence; kernels.rs:447,683 squeeze to bs = 1).  Each sequence has its own conv / recurrent
 * states, KV cache of tmax rows (tmax <= the model's), position, prompt, token and history; one
 * step runs every projection once for up to 8 sequences (Q8F matvec row groups), the DeltaNet
 * and attention kernels over all B rows at their own positions, the lm_head rows, and a
 * per-sequence greedy argmax with the reference's tie order.  Q35_LAUNCH_STREAM launches the step's
 * kernels one by one, Q35_LAUNCH_GRAPH replays a captured hipGraph of them. */
typedef struct q35_batch q35_batch;
int q35_batch_create(q35_model* m, int32_t B, int32_t tmax, q35_batch** out);
int q35_batch_destroy(q35_batch* b);
/* Zero every sequence's caches and positions. */
int q35_batch_reset(q35_batch* b, void* stream);
/* One decode step of all B sequences (each row's next prompt id, else its last argmax). */
int q35_batch_step(q35_batch* b, int32_t mode, void* stream);
int q35_batch_decode(q35_batch* b, int32_t n_steps, int32_t mode, void* stream);
/* Greedy generation for B prompts (prompts_host: the B prompts one after another, lens_host[B]
 * their lengths) at each sequence's current position: out_tokens_host [B][n_new + 1] receives,
 * per sequence, the argmax after its last prompt id and after each of n_new steps, as
 * q35_model_generate does for one.  Prompts are fed through the decode step (every row steps
 * max(len) + n_new times; a row with a shorter prompt generates past n_new, so tmax must allow
 * that) or, with Q35_PREFILL_GEMM in mode, through the prompt path one sequence at a time and
 * then n_new batched steps.  decode_seconds_host (optional): wall time of the batched steps.
 * Returns Q35_E_RANGE when a norm statistic or gate sum of this or an earlier q35_batch_step /
 * _decode met a non-finite or out-of-range value (the batch state is then invalid until
 * q35_batch_reset). */
int q35_batch_generate(q35_batch* b, const int32_t* prompts_host, const int32_t* lens_host, int32_t n_new,
                       int32_t* out_tokens_host, int32_t mode, double* decode_seconds_host, void* stream);
/* Host copy of the B positions. */
int q35_batch_position(q35_batch* b, int32_t* pos_out_host);
/* Device pointer and bytes of a batch tensor ("layers.{i}.linear_attn.recurrent_state" [B][...],
 * "layers.{i}.self_attn.k_cache" [B][kv_heads][tmax][256], "logits" [B][V], "hist" [B][tmax],
 * "pos", "token", ...). */
int q35_batch_tensor(q35_batch* b, const char* name, void** dptr, size_t* bytes);

/* ---------------------------------------------------------------- host utilities */

/* Seeded N(0, sigma) f32 values: counter-based splitmix64 + Box-Muller in double; element i of
 * stream `stream` is independent of how the range is split, so any slice can be regenerated. */
int q35_synth_normal(uint64_t seed, uint64_t stream, int64_t offset, int64_t n, float sigma, float* out_host);
/* Seeded U(lo, hi) f32 values from the same generator. */
int q35_synth_uniform(uint64_t seed, uint64_t stream, int64_t offset, int64_t n, float lo, float hi, float* out_host);
/* Stream id the model builder uses for a named tensor (FNV-1a of the name). */
uint64_t q35_synth_stream_id(const char* name);
/* Q8F quantiser, blocks of 64 along cols: scale = max|w|/127 (f32), q = round-half-away(w/scale)
 * clamped to [-127,127]; all-zero block -> scale 0.  Replaces the Quantizer of main.rs:175-179. */
int q35_quantize_q8f(const float* w_host, int64_t rows, int64_t cols, int8_t* q_host, float* scale_host);
/* Host: element counts of the Q35_KN_TILED form of a K x N Q8F matrix (int8 values, f32 scales). */
int64_t q35_q8f_tiled_q_count(int32_t K, int32_t N);
int64_t q35_q8f_tiled_scale_count(int32_t K, int32_t N);
/* Host: re-lay a Q35_KN matrix (q [K][N], scale [K][N/64]) out as Q35_KN_TILED. */
int q35_q8f_pack_kn_tiled(const int8_t* q_host, const float* scale_host, int32_t K, int32_t N, int8_t* q_tiled_host,
                          float* scale_tiled_host);
/* Device: re-lay a Q35_KN or Q35_KN_TILED matrix W (device memory) out as Q35_KN_MB into q_mb
 * (K*N bytes) and scale_mb (K*N/64 floats), on `stream`.  K a multiple of 32, N of 64.  No
 * reference counterpart (a load-time layout, as q35_q8f_pack_kn_tiled). */
int q35_q8f_pack_mb(q35_q8f W, int8_t* q_mb, float* scale_mb, void* stream);
/* Host: re-lay a Q35_KN matrix out as Q35_KN_PANEL (q [N/16][K][16], scale [N/64][K]; the same
 * K*N bytes and K*N/64 scales). */
int q35_q8f_pack_kn_panel(const int8_t* q_host, const float* scale_host, int32_t K, int32_t N, int8_t* q_panel_host,
                          float* scale_panel_host);
/* Host: the f32 values q35_model_create_from_safetensors takes for decoder tensor `name` (the
 * builder's names, as q35_model_tensor lists them without the .q/.scale suffix) from the
 * checkpoint at `path`, in the builder's layout ([in][out] for Linear weights), before Q8F
 * quantisation.  n must be the tensor's element count.  For tests and tools. */
int q35_safetensors_tensor(const char* path, const q35_dims* d, const char* name, float* out_host, int64_t n);
/* Host copy of the f32 values the model builder draws for a named tensor (before
 * quantisation), so a host-side checker can rebuild the same model. */
int q35_synth_model_tensor(const q35_dims* d, uint64_t seed, const char* name, float* out_host, int64_t n);

#ifdef __cplusplus
}
#endif
#endif /* Q35_H */
