/*
 * oracle.h — CPU restatement of the reference decode path (TEST INFRASTRUCTURE).
 *
 * This library is the checker for the HIP implementation under qwen-3.5_amd/.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it;
 * the product never links or calls it.
 *
 * Conventions
 *   - Q8F tensors are int8 values plus one f32 scale per block of 64 consecutive
 *     elements along the contiguous (last) axis of the stored matrix.  For the
 *     reference projections the stored matrix is Burn's Linear weight [in=K][out=N]
 *     (blocks along N, kernels.rs:56-57,75-76,87); for the tied embedding / lm_head it is
 *     [V][D] (blocks along D, kernels.rs:253-255,283).
 *   - Dot products and norms accumulate in double and are rounded to f32 once; element-wise
 *     formulas are evaluated in f32 in the order the reference writes them.
 *
 * Pinning (tests/test_oracle_*.py): every function is checked against numpy float64
 * brute force on small shapes, plus known-answer cases and invariants listed next to it;
 * orc_gdn_decode / orc_attn_decode / orc_model_step are checked against the pinned pieces
 * composed in the reference's order.  The reference ships no golden vectors and cannot be
 * built here (Rust, no toolchain), so nothing is compared with a reference run.
 *
 * Parity unpinned (no check can fix these without running the reference's dependencies):
 *   - orc_quantize_q8f vs Burn 0.22.1's Quantizer (main.rs:175-179): the rule implemented is
 *     the stated one (scale = max|w|/127, q = round-half-away(w/scale) clamped to +-127, an
 *     all-zero block gives scale 0); Burn's exact rounding and clamp are not pinned.
 *   - orc_attention_core: the 1/sqrt(head_dim) score scale assumes Burn attention()'s default
 *     options (text_modules.rs:921-928); no softcap.
 *   - orc_conv_update: Burn conv1d orientation assumed to be cross-correlation with the oldest
 *     tap first (text_modules.rs:153).
 *   - f32 transcendentals (exp/log/sqrt/sin/cos) of Rust/ndarray to the last ulp: covered only
 *     by the tolerances of the parity tests.
 *   - The token after a prompt: the reference picks it with Burn's generic logits.argmax(2)
 *     (main.rs:92-95), not with kernels::argmax; no fixture pins Burn's tie rule.  orc_argmax
 *     (the reference kernel's order, kernels.rs:298-371) is used for that token too, and so is
 *     the product's prompt path; the two can differ only on exact ties of the maximum.
 */
#ifndef Q35_ORACLE_H
#define Q35_ORACLE_H
#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
  const int8_t* q;
  const float* s;
  int32_t rows, cols; /* stored shape; blocks of 64 along cols */
} orc_q8;

/* model shape constants (text_config.rs:56-126 for the 2B values) */
typedef struct {
  int32_t hidden;          /* 2048 */
  int32_t ffn;             /* 6144 */
  int32_t vocab;           /* 248320 */
  int32_t n_layers;        /* 24 */
  int32_t full_interval;   /* 4: layer i is full attention iff (i+1) % 4 == 0 */
  int32_t lin_heads;       /* 16 (key heads == value heads) */
  int32_t lin_dk;          /* 128 */
  int32_t lin_dv;          /* 128 */
  int32_t conv_k;          /* 4 */
  int32_t attn_heads;      /* 8 */
  int32_t kv_heads;        /* 2 */
  int32_t head_dim;        /* 256 */
  int32_t rot_dim;         /* 64 = head_dim * partial_rotary_factor 0.25 */
  float eps;               /* 1e-6 */
  float theta;             /* 1e7 */
} orc_cfg;

typedef struct {
  orc_q8 qkv, z, out;             /* KN: [H][2Dk*h+Dv*h], [H][Dv*h], [Dv*h][H] */
  const float *w_b, *w_a;         /* f32 [H][lin_heads] */
  const float *a_log, *dt_bias;   /* [lin_heads] */
  const float* conv_w;            /* [conv_dim][conv_k] */
  const float* norm_w;            /* [lin_dv] */
} orc_gdn_w;

typedef struct {
  orc_q8 q, k, v, o;              /* KN */
  const float *q_norm, *k_norm;   /* [head_dim] */
} orc_attn_w;

typedef struct {
  orc_q8 gate, up, down;          /* KN */
} orc_mlp_w;

typedef struct {
  orc_gdn_w gdn;                  /* used when the layer is linear attention */
  orc_attn_w attn;                /* used when the layer is full attention */
  orc_mlp_w mlp;
  const float *in_norm, *post_norm; /* [hidden] */
} orc_layer_w;

typedef struct {
  orc_q8 embed;                   /* [vocab][hidden], blocks along hidden */
  const orc_layer_w* layers;
  const float* final_norm;
} orc_model_w;

/* per-layer decode state; pointers for the unused layer kind may be NULL */
typedef struct {
  float** conv;     /* [layer] -> [conv_dim][conv_k-1] */
  float** rec;      /* [layer] -> [lin_heads][lin_dk][lin_dv] */
  float** kc;       /* [layer] -> [kv_heads][tmax][head_dim] */
  float** vc;       /* [layer] -> [kv_heads][tmax][head_dim] */
  int32_t tmax;
  int32_t pos;      /* tokens already in the cache */
} orc_cache;

/* ---- tensor-level ops (kernels.rs) ---- */
void orc_quantize_q8f(const float* w, int64_t rows, int64_t cols, int8_t* q, float* s);
void orc_q8_gemv_kn(const float* x, int M, orc_q8 W, float* y, int rowdrop);
void orc_q8_gemv_nk(const float* x, int M, orc_q8 W, float* y, double* y64);
void orc_embedding_lookup(orc_q8 table, const int32_t* ids, int n, float* out);
void orc_gate_proj(const float* x, int in_dim, const float* w_b, const float* w_a,
                   const float* a_log, const float* dt_bias, int n_heads, float* out);
/* CPU-baseline timing only: switch both Q8F matvecs to dequantize-the-matrix + f32 GEMV (f32
 * accumulation) instead of the double-accumulated checker; set the OpenMP thread count. */
void orc_set_f32_dequant(int on);
void orc_set_threads(int n);
int orc_get_threads(void);
int32_t orc_argmax(const float* v, int64_t n);
int32_t orc_argmax_reference_order(const float* v, int64_t n);
int orc_gemv_num_splits(int in_dim, int out_dim);

/* ---- module-level ops (text_modules.rs) ---- */
void orc_rmsnorm(const float* x, int n, const float* w, float eps, float* out);
void orc_rmsnorm_gated(const float* x, const float* z, int n, const float* w, float eps, float* out);
void orc_conv_update(const float* x, float* state, const float* w, int channels, int k, float* out);
void orc_l2norm(const float* x, int n, float eps, float* out);
void orc_gated_delta_step(const float* q, const float* k, const float* v, const float* g,
                          const float* beta, float* S, int heads, int dk, int dv, float* out);
void orc_gated_delta_chunked(const float* q, const float* k, const float* v, const float* g,
                             const float* beta, int T, int heads, int dk, int dv, int chunk,
                             float* S, float* out);
void orc_rope_cos_sin(int pos, int rot_dim, float theta, float* cos_out, float* sin_out);
void orc_apply_rope(float* x, int rot_dim, const float* cosv, const float* sinv);
void orc_attention_core(const float* q, const float* kc, const float* vc, int T, int tmax,
                        int n_heads, int kv_heads, int head_dim, float* out);

/* layer forwards on one token (batch folded into B independent rows) */
void orc_gdn_decode(const orc_cfg* c, const orc_gdn_w* w, const float* x, int B,
                    float* conv_state, float* rec_state, float* out);
void orc_attn_decode(const orc_cfg* c, const orc_attn_w* w, const float* x, int B,
                     float* kc, float* vc, int tmax, const int32_t* pos, float* out);
void orc_mlp_decode(const orc_cfg* c, const orc_mlp_w* w, const float* x, int B, float* out);

/* one token through the whole model: returns argmax id; logits optional (vocab f32);
 * margin optional (top1 - top2 in double) */
int32_t orc_model_step(const orc_cfg* c, const orc_model_w* m, orc_cache* cache, int32_t token,
                       float* logits, double* margin);

#ifdef __cplusplus
}
#endif
#endif
