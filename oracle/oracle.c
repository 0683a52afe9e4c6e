/*
 * oracle.c — CPU restatement of the reference decode path.  TEST INFRASTRUCTURE ONLY:
 * it is the checker for the HIP product (tests/, smoke(), bench.py cpu_baseline) and is
 * never linked into or called by the product.
 *
 * Each function names the reference lines it restates (paths relative to the reference
 * checkout of inventwithdean/Qwen-3.5).  Reductions accumulate in double and round to f32
 * once; element-wise formulas are f32 in the reference's order.  Pinning of each function
 * is listed in oracle.h and done by tests/test_oracle_*.py.
 */
#include "oracle.h"
#include <math.h>
#include <omp.h>
#include <stdlib.h>
#include <string.h>

static inline float silu_f(float v) { return v * (1.0f / (1.0f + expf(-v))); }
static inline float sigmoid_f(float v) { return 1.0f / (1.0f + expf(-v)); }

/* Q8F per-block-64 symmetric quantizer.  Reference: main.rs:175-179 (Burn Quantizer with
 * Calibration::MinMax, per_block([64]), Q8F).  Rule as fixed by the workload definition:
 * scale = max|w| / 127 in f32, q = round-half-away(w / scale) clamped to [-127, 127];
 * an all-zero block has scale 0 and q 0. */
void orc_quantize_q8f(const float* w, int64_t rows, int64_t cols, int8_t* q, float* s) {
  const int64_t nb = cols / 64;
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t b = 0; b < nb; ++b) {
      const float* src = w + r * cols + b * 64;
      float amax = 0.0f;
      for (int j = 0; j < 64; ++j) { float a = fabsf(src[j]); if (a > amax) amax = a; }
      float sc = amax / 127.0f;
      s[r * nb + b] = sc;
      int8_t* dst = q + r * cols + b * 64;
      for (int j = 0; j < 64; ++j) {
        float v = (sc == 0.0f) ? 0.0f : roundf(src[j] / sc);
        if (v > 127.0f) v = 127.0f;
        if (v < -127.0f) v = -127.0f;
        dst[j] = (int8_t)v;
      }
    }
  }
}

/* Split rule of the reference's decode matvec (kernels.rs:504). */
int orc_gemv_num_splits(int in_dim, int out_dim) {
  int s = 25000 / out_dim;
  int hi = in_dim / 80; if (hi < 1) hi = 1;
  if (s < 1) s = 1;
  if (s > hi) s = hi;
  return s;
}

/* ---- CPU-baseline timing path (not a checker): Burn's dequantize-then-f32-matmul --------
 * With orc_set_f32_dequant(1) the two Q8F matvecs below stop being the double-accumulated
 * checker and time the path the workload names for the CPU column: the whole int8 matrix is
 * dequantised to an f32 copy (Burn materialises it per call; here into one reused buffer, so no
 * page-fault cost is added), then an f32 GEMV with f32 accumulation, OpenMP over output columns.
 * orc_set_threads sets the OpenMP thread count. */
static int g_f32_dequant = 0;
static float* g_wbuf = NULL;
static size_t g_wcap = 0;
void orc_set_f32_dequant(int on) { g_f32_dequant = on; }
void orc_set_threads(int n) { omp_set_num_threads(n > 0 ? n : 1); }
int orc_get_threads(void) { return omp_get_max_threads(); }

static float* dequant_buf(size_t n) {
  if (n > g_wcap) {
    free(g_wbuf);
    g_wbuf = (float*)malloc(n * sizeof(float));
    g_wcap = g_wbuf ? n : 0;
  }
  return g_wbuf;
}

/* dequantize (rows x cols, blocks of 64 along cols) into an f32 matrix of the same shape */
static void dequant_f32(orc_q8 W, float* out) {
  const int R = W.rows, C = W.cols, nb = C / 64;
#pragma omp parallel for schedule(static)
  for (int r = 0; r < R; ++r)
    for (int c = 0; c < C; ++c) out[(size_t)r * C + c] = (float)W.q[(size_t)r * C + c] * W.s[(size_t)r * nb + c / 64];
}

static void gemv_kn_f32(const float* x, int M, orc_q8 W, float* y) {
  const int K = W.rows, N = W.cols;
  float* Wf = dequant_buf((size_t)K * N);
  dequant_f32(W, Wf);
  const int NT = 256, ntiles = (N + NT - 1) / NT;
#pragma omp parallel for collapse(2) schedule(static)
  for (int m = 0; m < M; ++m) {
    for (int t = 0; t < ntiles; ++t) {
      float acc[256];
      const int n0 = t * NT, n1 = n0 + NT < N ? n0 + NT : N;
      for (int n = n0; n < n1; ++n) acc[n - n0] = 0.0f;
      for (int k = 0; k < K; ++k) {
        const float xk = x[(size_t)m * K + k];
        const float* wr = Wf + (size_t)k * N;
        for (int n = n0; n < n1; ++n) acc[n - n0] += xk * wr[n];
      }
      for (int n = n0; n < n1; ++n) y[(size_t)m * N + n] = acc[n - n0];
    }
  }
}

static void gemv_nk_f32(const float* x, int M, orc_q8 W, float* y, double* y64) {
  const int N = W.rows, K = W.cols;
  float* Wf = dequant_buf((size_t)N * K);
  dequant_f32(W, Wf);
#pragma omp parallel for collapse(2) schedule(static)
  for (int m = 0; m < M; ++m) {
    for (int n = 0; n < N; ++n) {
      const float* wr = Wf + (size_t)n * K;
      const float* xm = x + (size_t)m * K;
      float acc = 0.0f;
      for (int k = 0; k < K; ++k) acc += xm[k] * wr[k];
      y[(size_t)m * N + n] = acc;
      if (y64) y64[(size_t)m * N + n] = acc;
    }
  }
}

/* y[m][n] = sum_k x[m][k] * q[k][n] * s[k][n/64]   (KN layout, blocks along N).
 * Reference: kernels.rs:53-92 (q8_gemv), :103-165 (q8_gemv_partial_sum + reduction), the
 * Burn Linear dequant+matmul of the seq_len>1 branches.  rowdrop=1 reproduces the rows the
 * partial-sum kernel actually reads (kernels.rs:119-133: each split sums 8*floor(chunk/8)
 * rows), which skips rows whenever K/splits is not a multiple of 8. */
void orc_q8_gemv_kn(const float* x, int M, orc_q8 W, float* y, int rowdrop) {
  if (g_f32_dequant && !rowdrop) { gemv_kn_f32(x, M, W, y); return; }
  const int K = W.rows, N = W.cols, nb = N / 64;
  unsigned char* keep = (unsigned char*)malloc((size_t)K);
  for (int k = 0; k < K; ++k) keep[k] = 1;
  if (rowdrop) {
    int splits = orc_gemv_num_splits(K, N);
    int chunk = K / splits;
    int used = 8 * (chunk / 8);
    for (int k = 0; k < K; ++k) keep[k] = 0;
    for (int sp = 0; sp < splits; ++sp)
      for (int r = 0; r < used; ++r) keep[sp * chunk + r] = 1;
  }
  const int NT = 256; /* column tile per OpenMP task */
  const int ntiles = (N + NT - 1) / NT;
#pragma omp parallel for collapse(2) schedule(static)
  for (int m = 0; m < M; ++m) {
    for (int t = 0; t < ntiles; ++t) {
      double acc[256];
      int n0 = t * NT, n1 = n0 + NT < N ? n0 + NT : N;
      for (int n = n0; n < n1; ++n) acc[n - n0] = 0.0;
      for (int k = 0; k < K; ++k) {
        if (!keep[k]) continue;
        const double xk = (double)x[(size_t)m * K + k];
        const int8_t* qr = W.q + (size_t)k * N;
        const float* sr = W.s + (size_t)k * nb;
        for (int n = n0; n < n1; ++n) acc[n - n0] += xk * ((double)qr[n] * (double)sr[n >> 6]);
      }
      for (int n = n0; n < n1; ++n) y[(size_t)m * N + n] = (float)acc[n - n0];
    }
  }
  free(keep);
}

/* y[m][n] = sum_k x[m][k] * q[n][k] * s[n][k/64]   (NK layout, blocks along K).
 * Reference: kernels.rs:251-291 (q8_lm_head over the tied embedding table) and the
 * prefill lm_head matmul model.rs:130-138.  y64 (optional) receives the double result. */
void orc_q8_gemv_nk(const float* x, int M, orc_q8 W, float* y, double* y64) {
  if (g_f32_dequant) { gemv_nk_f32(x, M, W, y, y64); return; }
  const int N = W.rows, K = W.cols, nb = K / 64;
#pragma omp parallel for collapse(2) schedule(static)
  for (int m = 0; m < M; ++m) {
    for (int n = 0; n < N; ++n) {
      const int8_t* qr = W.q + (size_t)n * K;
      const float* sr = W.s + (size_t)n * nb;
      const float* xm = x + (size_t)m * K;
      double acc = 0.0;
      for (int b = 0; b < nb; ++b) {
        double part = 0.0;
        for (int j = 0; j < 64; ++j) part += (double)qr[b * 64 + j] * (double)xm[b * 64 + j];
        acc += part * (double)sr[b];
      }
      y[(size_t)m * N + n] = (float)acc;
      if (y64) y64[(size_t)m * N + n] = acc;
    }
  }
}

/* out[i][d] = q[id_i][d] * s[id_i][d/64].  Reference: kernels.rs:15-45. */
void orc_embedding_lookup(orc_q8 table, const int32_t* ids, int n, float* out) {
  const int D = table.cols, nb = D / 64;
  for (int i = 0; i < n; ++i) {
    const int64_t id = ids[i];
    for (int d = 0; d < D; ++d)
      out[(size_t)i * D + d] = (float)table.q[id * D + d] * table.s[id * nb + d / 64];
  }
}

/* beta = sigmoid(x . W_b[:,h]);  g = -exp(A_log[h]) * softplus(x . W_a[:,h] + dt_bias[h]),
 * softplus taking the branch x_gate when ln(exp(x_gate)+1) > 20.
 * Reference: kernels.rs:174-247 (decode) — W_b, W_a stored [in_dim][n_heads] (Burn Linear).
 * out = [beta(n_heads) | g(n_heads)] like the reference's packed output. */
void orc_gate_proj(const float* x, int in_dim, const float* w_b, const float* w_a,
                   const float* a_log, const float* dt_bias, int n_heads, float* out) {
  for (int h = 0; h < n_heads; ++h) {
    double b = 0.0, a = 0.0;
    for (int k = 0; k < in_dim; ++k) {
      b += (double)x[k] * (double)w_b[(size_t)k * n_heads + h];
      a += (double)x[k] * (double)w_a[(size_t)k * n_heads + h];
    }
    float bf = (float)b, af = (float)a;
    out[h] = 1.0f / (1.0f + expf(-bf));
    float x_gate = af + dt_bias[h];
    float pre = logf(expf(x_gate) + 1.0f);
    float sp = pre > 20.0f ? x_gate : pre;
    out[n_heads + h] = -expf(a_log[h]) * sp;
  }
}

/* Tie key of index i under the reference's argmax (kernels.rs:298-371): with c = n/8 and
 * i = k*c + p, the reference's scans keep the first strict maximum in the order
 * (p mod 256, p div 256, k).  Indices >= 8c (never read by the reference) come after all of
 * them, in index order. */
static uint64_t argmax_key(int64_t i, int64_t n) {
  const int64_t c = n / 8, s = (c + 255) / 256;
  if (i >= 8 * c) return (uint64_t)(s * 2048 + (i - 8 * c));
  const int64_t k = i / c, p = i - k * c;
  return (uint64_t)((((p % 256) * s) + p / 256) * 8 + k);
}

/* Greedy token: the largest value; among exactly equal maxima the one the reference's two-stage
 * argmax returns (argmax_key), which for n a multiple of 8 with n/8 >= 256 is
 * orc_argmax_reference_order's result.  NaN values are never picked. */
int32_t orc_argmax(const float* v, int64_t n) {
  int64_t best = -1;
  for (int64_t i = 0; i < n; ++i) {
    if (v[i] != v[i]) continue;
    if (best < 0 || v[i] > v[best] || (v[i] == v[best] && argmax_key(i, n) < argmax_key(best, n))) best = i;
  }
  return (int32_t)(best < 0 ? 0 : best);
}

/* Exact two-stage order of kernels.rs:298-371: unit p scans p + k*(n/8), k<8, strict '>';
 * 256 threads stride over the n/8 partials, strict '>'; thread 0 scans the 256 results.
 * Requires n/8 >= 256.  Indices >= 8*(n/8) are never read, as in the reference. */
int32_t orc_argmax_reference_order(const float* v, int64_t n) {
  const int64_t chunk = n / 8;
  float* pm = (float*)malloc(sizeof(float) * chunk);
  int32_t* pi = (int32_t*)malloc(sizeof(int32_t) * chunk);
  for (int64_t p = 0; p < chunk; ++p) {
    float mx = v[p]; int64_t mi = p;
    for (int k = 1; k < 8; ++k) { int64_t i = k * chunk + p; if (v[i] > mx) { mx = v[i]; mi = i; } }
    pm[p] = mx; pi[p] = (int32_t)mi;
  }
  float tm[256]; int32_t ti[256];
  const int64_t scans = (chunk + 255) / 256;
  for (int t = 0; t < 256; ++t) {
    float mx = pm[t]; int32_t mi = pi[t];
    for (int64_t k = 1; k < scans; ++k) {
      int64_t idx = k * 256 + t;
      if (idx < chunk && pm[idx] > mx) { mx = pm[idx]; mi = pi[idx]; }
    }
    tm[t] = mx; ti[t] = mi;
  }
  float mx = tm[0]; int32_t mi = ti[0];
  for (int t = 1; t < 256; ++t) if (tm[t] > mx) { mx = tm[t]; mi = ti[t]; }
  free(pm); free(pi);
  return mi;
}

/* x * rsqrt(mean(x^2) + eps) * (1 + w).  Reference: text_modules.rs:800-808. */
void orc_rmsnorm(const float* x, int n, const float* w, float eps, float* out) {
  double ss = 0.0;
  for (int i = 0; i < n; ++i) ss += (double)x[i] * (double)x[i];
  float var = (float)(ss / n);
  float r = 1.0f / sqrtf(var + eps);
  for (int i = 0; i < n; ++i) out[i] = (x[i] * r) * (1.0f + w[i]);
}

/* (w * (x * rsqrt(mean(x^2)+eps))) * silu(z).  Reference: text_modules.rs:91-100. */
void orc_rmsnorm_gated(const float* x, const float* z, int n, const float* w, float eps, float* out) {
  double ss = 0.0;
  for (int i = 0; i < n; ++i) ss += (double)x[i] * (double)x[i];
  float var = (float)(ss / n);
  float r = 1.0f / sqrtf(var + eps);
  for (int i = 0; i < n; ++i) out[i] = (w[i] * (x[i] * r)) * silu_f(z[i]);
}

/* Depthwise causal conv over [state(k-1) | x] (cross-correlation, oldest tap first, no
 * bias) then SiLU; the state keeps the newest k-1 columns.  Reference: text_modules.rs:134-162.
 * state is [channels][k-1], w is [channels][k]. */
void orc_conv_update(const float* x, float* state, const float* w, int channels, int k, float* out) {
  for (int c = 0; c < channels; ++c) {
    float* st = state + (size_t)c * (k - 1);
    const float* wc = w + (size_t)c * k;
    double acc = 0.0;
    for (int j = 0; j < k - 1; ++j) acc += (double)wc[j] * (double)st[j];
    acc += (double)wc[k - 1] * (double)x[c];
    out[c] = silu_f((float)acc);
    for (int j = 0; j < k - 2; ++j) st[j] = st[j + 1];
    st[k - 2] = x[c];
  }
}

/* x * rsqrt(sum(x^2) + eps).  Reference: text_modules.rs:184-187. */
void orc_l2norm(const float* x, int n, float eps, float* out) {
  double ss = 0.0;
  for (int i = 0; i < n; ++i) ss += (double)x[i] * (double)x[i];
  float r = 1.0f / sqrtf((float)ss + eps);
  for (int i = 0; i < n; ++i) out[i] = x[i] * r;
}

/* One recurrent gated-delta step for `heads` heads (batch folded in by the caller).
 * q, k: [heads][dk] RAW (normalised here, q also scaled by dk^-1/2); v: [heads][dv];
 * g, beta: [heads]; S: [heads][dk][dv] updated in place; out: [heads][dv].
 * Reference: text_modules.rs:365-443 (burn_recurrent_gated_delta_rule) with l2norm :389-392. */
void orc_gated_delta_step(const float* q, const float* k, const float* v, const float* g,
                          const float* beta, float* S, int heads, int dk, int dv, float* out) {
  const float qscale = powf((float)dk, -0.5f);
  float* qh = (float*)malloc(sizeof(float) * dk);
  float* kh = (float*)malloc(sizeof(float) * dk);
  double* m = (double*)malloc(sizeof(double) * dv);
  for (int h = 0; h < heads; ++h) {
    orc_l2norm(q + (size_t)h * dk, dk, 1e-6f, qh);
    orc_l2norm(k + (size_t)h * dk, dk, 1e-6f, kh);
    for (int i = 0; i < dk; ++i) qh[i] = qh[i] * qscale;
    float* Sh = S + (size_t)h * dk * dv;
    const float decay = expf(g[h]);
    for (size_t e = 0; e < (size_t)dk * dv; ++e) Sh[e] = Sh[e] * decay;
    for (int j = 0; j < dv; ++j) m[j] = 0.0;
    for (int i = 0; i < dk; ++i)
      for (int j = 0; j < dv; ++j) m[j] += (double)Sh[(size_t)i * dv + j] * (double)kh[i];
    for (int j = 0; j < dv; ++j) {
      float delta = (v[(size_t)h * dv + j] - (float)m[j]) * beta[h];
      for (int i = 0; i < dk; ++i) Sh[(size_t)i * dv + j] = Sh[(size_t)i * dv + j] + kh[i] * delta;
    }
    for (int j = 0; j < dv; ++j) m[j] = 0.0;
    for (int i = 0; i < dk; ++i)
      for (int j = 0; j < dv; ++j) m[j] += (double)Sh[(size_t)i * dv + j] * (double)qh[i];
    for (int j = 0; j < dv; ++j) out[(size_t)h * dv + j] = (float)m[j];
  }
  free(qh); free(kh); free(m);
}

/* Chunked (WY-form) gated delta rule over T tokens.  Reference: text_modules.rs:190-363.
 * q,k: [T][heads][dk] RAW; v: [T][heads][dv]; g, beta: [T][heads]; S: [heads][dk][dv] in/out;
 * out: [T][heads][dv].  Evaluated in double. */
void orc_gated_delta_chunked(const float* q, const float* k, const float* v, const float* g,
                             const float* beta, int T, int heads, int dk, int dv, int C,
                             float* S, float* out) {
  const int Tp = ((T + C - 1) / C) * C;
  const double qscale = (double)powf((float)dk, -0.5f);
  double *Q = malloc(sizeof(double) * Tp * dk), *Kk = malloc(sizeof(double) * Tp * dk);
  double *V = malloc(sizeof(double) * Tp * dv), *G = malloc(sizeof(double) * Tp),
         *Bt = malloc(sizeof(double) * Tp);
  double *cum = malloc(sizeof(double) * C), *U = malloc(sizeof(double) * C * C),
         *A = malloc(sizeof(double) * C * C);
  double *vnew = malloc(sizeof(double) * C * dv), *kcd = malloc(sizeof(double) * C * dk),
         *nv = malloc(sizeof(double) * C * dv);
  double* Sd = malloc(sizeof(double) * dk * dv);
  float* tmp = malloc(sizeof(float) * (dk > dv ? dk : dv));
  for (int h = 0; h < heads; ++h) {
    for (int t = 0; t < Tp; ++t) {
      if (t < T) {
        orc_l2norm(q + ((size_t)t * heads + h) * dk, dk, 1e-6f, tmp);
        for (int i = 0; i < dk; ++i) Q[t * dk + i] = (double)tmp[i] * qscale;
        orc_l2norm(k + ((size_t)t * heads + h) * dk, dk, 1e-6f, tmp);
        for (int i = 0; i < dk; ++i) Kk[t * dk + i] = tmp[i];
        for (int j = 0; j < dv; ++j) V[t * dv + j] = v[((size_t)t * heads + h) * dv + j];
        G[t] = g[(size_t)t * heads + h];
        Bt[t] = beta[(size_t)t * heads + h];
      } else {
        for (int i = 0; i < dk; ++i) { Q[t * dk + i] = 0; Kk[t * dk + i] = 0; }
        for (int j = 0; j < dv; ++j) V[t * dv + j] = 0;
        G[t] = 0; Bt[t] = 0;
      }
    }
    float* Sh = S + (size_t)h * dk * dv;
    for (int e = 0; e < dk * dv; ++e) Sd[e] = Sh[e];
    for (int c0 = 0; c0 < Tp; c0 += C) {
      double acc = 0;
      for (int i = 0; i < C; ++i) { acc += G[c0 + i]; cum[i] = acc; }
      /* A[i][j] = (k_beta_i . k_j) * exp(cum_i - cum_j) for j < i (strictly lower) */
      for (int i = 0; i < C; ++i)
        for (int j = 0; j < C; ++j) {
          double d = 0;
          if (j < i) {
            for (int e = 0; e < dk; ++e) d += Kk[(c0 + i) * dk + e] * Bt[c0 + i] * Kk[(c0 + j) * dk + e];
            d *= exp(cum[i] - cum[j]);
          }
          U[i * C + j] = -d;
        }
      /* forward substitution: U[i, :i] += U[i, :i] @ U[:i, :i] (rows in increasing order) */
      for (int i = 1; i < C; ++i) {
        double row[512];
        for (int j = 0; j < i; ++j) row[j] = U[i * C + j];
        for (int j = 0; j < i; ++j) {
          double s2 = 0;
          for (int l = 0; l < i; ++l) s2 += row[l] * U[l * C + j];
          U[i * C + j] = row[j] + s2;
        }
      }
      for (int i = 0; i < C; ++i) U[i * C + i] += 1.0;
      /* new_values = U @ v_beta ; k_cumdecay = U @ (k_beta * exp(cum)) */
      for (int i = 0; i < C; ++i) {
        for (int j = 0; j < dv; ++j) {
          double s2 = 0;
          for (int l = 0; l < C; ++l) s2 += U[i * C + l] * V[(c0 + l) * dv + j] * Bt[c0 + l];
          nv[i * dv + j] = s2;
        }
        for (int e = 0; e < dk; ++e) {
          double s2 = 0;
          for (int l = 0; l < C; ++l) s2 += U[i * C + l] * Kk[(c0 + l) * dk + e] * Bt[c0 + l] * exp(cum[l]);
          kcd[i * dk + e] = s2;
        }
      }
      /* intra[i][j] = (q_i . k_j) * exp(cum_i - cum_j), j <= i */
      for (int i = 0; i < C; ++i)
        for (int j = 0; j < C; ++j) {
          double d = 0;
          if (j <= i) {
            for (int e = 0; e < dk; ++e) d += Q[(c0 + i) * dk + e] * Kk[(c0 + j) * dk + e];
            d *= exp(cum[i] - cum[j]);
          }
          A[i * C + j] = d;
        }
      /* v_new = new_values - k_cumdecay @ S */
      for (int i = 0; i < C; ++i)
        for (int j = 0; j < dv; ++j) {
          double s2 = 0;
          for (int e = 0; e < dk; ++e) s2 += kcd[i * dk + e] * Sd[e * dv + j];
          vnew[i * dv + j] = nv[i * dv + j] - s2;
        }
      /* out = (q * exp(cum)) @ S + intra @ v_new */
      for (int i = 0; i < C; ++i) {
        int t = c0 + i;
        for (int j = 0; j < dv; ++j) {
          double s2 = 0;
          for (int e = 0; e < dk; ++e) s2 += Q[t * dk + e] * exp(cum[i]) * Sd[e * dv + j];
          for (int l = 0; l < C; ++l) s2 += A[i * C + l] * vnew[l * dv + j];
          if (t < T) out[((size_t)t * heads + h) * dv + j] = (float)s2;
        }
      }
      /* S = S * exp(cum_last) + (k * exp(cum_last - cum))^T @ v_new */
      const double cl = cum[C - 1];
      for (int e = 0; e < dk; ++e)
        for (int j = 0; j < dv; ++j) {
          double s2 = Sd[e * dv + j] * exp(cl);
          for (int l = 0; l < C; ++l) s2 += Kk[(c0 + l) * dk + e] * exp(cl - cum[l]) * vnew[l * dv + j];
          Sd[e * dv + j] = s2;
        }
    }
    for (int e = 0; e < dk * dv; ++e) Sh[e] = (float)Sd[e];
  }
  free(Q); free(Kk); free(V); free(G); free(Bt); free(cum); free(U); free(A);
  free(vnew); free(kcd); free(nv); free(Sd); free(tmp);
}

/* cos/sin for one position, rot_dim entries (the 32 frequencies repeated twice).
 * inv_freq[i] = exp(2i * (-ln(theta)/rot_dim)) in f32; angle = f32(pos) * inv_freq.
 * Reference: text_modules.rs:30-43,73-81 (mRoPE recomposition :45-58 is the identity when
 * the three position rows are equal, as model.rs:51-56 builds them for text). */
void orc_rope_cos_sin(int pos, int rot_dim, float theta, float* cos_out, float* sin_out) {
  const float sf = -logf(theta) / (float)rot_dim;
  const int half = rot_dim / 2;
  for (int i = 0; i < half; ++i) {
    float inv = expf((float)(2 * i) * sf);
    float ang = (float)pos * inv;
    float c = cosf(ang), s = sinf(ang);
    cos_out[i] = c; cos_out[i + half] = c;
    sin_out[i] = s; sin_out[i + half] = s;
  }
}

/* x[0:rot] = x*cos + rotate_half(x)*sin; dims >= rot pass through.
 * Reference: text_modules.rs:739-774. */
void orc_apply_rope(float* x, int rot_dim, const float* cosv, const float* sinv) {
  const int half = rot_dim / 2;
  float tmp[512];
  for (int i = 0; i < rot_dim; ++i) tmp[i] = x[i];
  for (int i = 0; i < half; ++i) x[i] = tmp[i] * cosv[i] + (-tmp[i + half]) * sinv[i];
  for (int i = half; i < rot_dim; ++i) x[i] = tmp[i] * cosv[i] + tmp[i - half] * sinv[i];
}

/* softmax(q k^T / sqrt(d)) v over T cached tokens, GQA head h -> kv head h / (n_heads/kv_heads).
 * q: [n_heads][d]; kc, vc: [kv_heads][tmax][d]; out: [n_heads][d].
 * Reference: text_modules.rs:911-928 (repeat_kv :776-792, Burn attention default options). */
void orc_attention_core(const float* q, const float* kc, const float* vc, int T, int tmax,
                        int n_heads, int kv_heads, int d, float* out) {
  const int rep = n_heads / kv_heads;
  const double scale = 1.0 / sqrt((double)d);
  double* sc = (double*)malloc(sizeof(double) * T);
  for (int h = 0; h < n_heads; ++h) {
    const int g = h / rep;
    const float* K = kc + (size_t)g * tmax * d;
    const float* Vv = vc + (size_t)g * tmax * d;
    double mx = -INFINITY;
    for (int t = 0; t < T; ++t) {
      double dot = 0;
      for (int e = 0; e < d; ++e) dot += (double)q[(size_t)h * d + e] * (double)K[(size_t)t * d + e];
      sc[t] = dot * scale;
      if (sc[t] > mx) mx = sc[t];
    }
    double den = 0;
    for (int t = 0; t < T; ++t) { sc[t] = exp(sc[t] - mx); den += sc[t]; }
    for (int e = 0; e < d; ++e) {
      double acc = 0;
      for (int t = 0; t < T; ++t) acc += sc[t] * (double)Vv[(size_t)t * d + e];
      out[(size_t)h * d + e] = (float)(acc / den);
    }
  }
  free(sc);
}

/* GatedDeltaNet decode forward for B independent rows (x already input-normed).
 * Reference: text_modules.rs:484-667 (seq_len == 1 with cached states).
 * conv_state: [B][conv_dim][conv_k-1]; rec_state: [B][heads][dk][dv]; out: [B][hidden]. */
void orc_gdn_decode(const orc_cfg* c, const orc_gdn_w* w, const float* x, int B,
                    float* conv_state, float* rec_state, float* out) {
  const int H = c->hidden, nh = c->lin_heads, dk = c->lin_dk, dv = c->lin_dv;
  const int key_dim = nh * dk, val_dim = nh * dv, conv_dim = 2 * key_dim + val_dim;
  float* qkv = malloc(sizeof(float) * conv_dim);
  float* conv_out = malloc(sizeof(float) * conv_dim);
  float* z = malloc(sizeof(float) * val_dim);
  float* core = malloc(sizeof(float) * val_dim);
  float* normed = malloc(sizeof(float) * val_dim);
  float* bg = malloc(sizeof(float) * 2 * nh);
  for (int b = 0; b < B; ++b) {
    const float* xb = x + (size_t)b * H;
    orc_q8_gemv_kn(xb, 1, w->qkv, qkv, 0);                 /* :497-501 */
    orc_q8_gemv_kn(xb, 1, w->z, z, 0);                     /* :504-508 */
    orc_conv_update(qkv, conv_state + (size_t)b * conv_dim * (c->conv_k - 1), w->conv_w,
                    conv_dim, c->conv_k, conv_out);        /* :515-530 */
    orc_gate_proj(xb, H, w->w_b, w->w_a, w->a_log, w->dt_bias, nh, bg); /* :569-576 */
    orc_gated_delta_step(conv_out, conv_out + key_dim, conv_out + 2 * key_dim, bg + nh, bg,
                         rec_state + (size_t)b * nh * dk * dv, nh, dk, dv, core); /* :627-636 */
    for (int h = 0; h < nh; ++h)                           /* :654-660 */
      orc_rmsnorm_gated(core + (size_t)h * dv, z + (size_t)h * dv, dv, w->norm_w, c->eps,
                        normed + (size_t)h * dv);
    orc_q8_gemv_kn(normed, 1, w->out, out + (size_t)b * H, 0); /* :661-663 */
  }
  free(qkv); free(conv_out); free(z); free(core); free(normed); free(bg);
}

/* Gated GQA attention decode for B rows; pos[b] = tokens already cached for row b.
 * kc/vc: [B][kv_heads][tmax][head_dim].  Reference: text_modules.rs:842-944. */
void orc_attn_decode(const orc_cfg* c, const orc_attn_w* w, const float* x, int B,
                     float* kc, float* vc, int tmax, const int32_t* pos, float* out) {
  const int H = c->hidden, nh = c->attn_heads, nkv = c->kv_heads, d = c->head_dim;
  float* qg = malloc(sizeof(float) * nh * 2 * d);
  float* q = malloc(sizeof(float) * nh * d);
  float* gate = malloc(sizeof(float) * nh * d);
  float* k = malloc(sizeof(float) * nkv * d);
  float* v = malloc(sizeof(float) * nkv * d);
  float* att = malloc(sizeof(float) * nh * d);
  float cosv[512], sinv[512];
  for (int b = 0; b < B; ++b) {
    const float* xb = x + (size_t)b * H;
    orc_q8_gemv_kn(xb, 1, w->q, qg, 0);                      /* :855-859 */
    for (int h = 0; h < nh; ++h) {                           /* :860-875 per-head [q | gate] */
      orc_rmsnorm(qg + (size_t)h * 2 * d, d, w->q_norm, c->eps, q + (size_t)h * d);
      memcpy(gate + (size_t)h * d, qg + (size_t)h * 2 * d + d, sizeof(float) * d);
    }
    orc_q8_gemv_kn(xb, 1, w->k, k, 0);                       /* :876-883 */
    for (int h = 0; h < nkv; ++h) orc_rmsnorm(k + (size_t)h * d, d, w->k_norm, c->eps, k + (size_t)h * d);
    orc_q8_gemv_kn(xb, 1, w->v, v, 0);                       /* :885-893 */
    orc_rope_cos_sin(pos[b], c->rot_dim, c->theta, cosv, sinv); /* model.rs:51-57 */
    for (int h = 0; h < nh; ++h) orc_apply_rope(q + (size_t)h * d, c->rot_dim, cosv, sinv);
    for (int h = 0; h < nkv; ++h) orc_apply_rope(k + (size_t)h * d, c->rot_dim, cosv, sinv);
    float* kcb = kc + (size_t)b * nkv * tmax * d;           /* :899-909 KV append */
    float* vcb = vc + (size_t)b * nkv * tmax * d;
    for (int h = 0; h < nkv; ++h) {
      memcpy(kcb + ((size_t)h * tmax + pos[b]) * d, k + (size_t)h * d, sizeof(float) * d);
      memcpy(vcb + ((size_t)h * tmax + pos[b]) * d, v + (size_t)h * d, sizeof(float) * d);
    }
    orc_attention_core(q, kcb, vcb, pos[b] + 1, tmax, nh, nkv, d, att); /* :911-928 */
    for (int i = 0; i < nh * d; ++i) att[i] = att[i] * sigmoid_f(gate[i]); /* :936 */
    orc_q8_gemv_kn(att, 1, w->o, out + (size_t)b * H, 0);    /* :938-942 */
  }
  free(qg); free(q); free(gate); free(k); free(v); free(att);
}

/* down(up(x) * silu(gate(x))).  Reference: text_modules.rs:1000-1011. */
void orc_mlp_decode(const orc_cfg* c, const orc_mlp_w* w, const float* x, int B, float* out) {
  const int H = c->hidden, F = c->ffn;
  float* up = malloc(sizeof(float) * F);
  float* gt = malloc(sizeof(float) * F);
  for (int b = 0; b < B; ++b) {
    orc_q8_gemv_kn(x + (size_t)b * H, 1, w->up, up, 0);
    orc_q8_gemv_kn(x + (size_t)b * H, 1, w->gate, gt, 0);
    for (int i = 0; i < F; ++i) up[i] = up[i] * silu_f(gt[i]);
    orc_q8_gemv_kn(up, 1, w->down, out + (size_t)b * H, 0);
  }
  free(up); free(gt);
}

static int is_full_layer(const orc_cfg* c, int l) { return ((l + 1) % c->full_interval) == 0; }

/* One token through TextForCausalLM (model.rs:27-84,113-129) and the greedy pick
 * (main.rs:131): embedding -> 24 x DecoderLayer (text_modules.rs:1053-1085) -> final RMSNorm
 * -> tied lm_head -> argmax.  Advances cache->pos by one. */
int32_t orc_model_step(const orc_cfg* c, const orc_model_w* m, orc_cache* cache, int32_t token,
                       float* logits, double* margin) {
  const int H = c->hidden;
  float* h = malloc(sizeof(float) * H);
  float* xn = malloc(sizeof(float) * H);
  float* y = malloc(sizeof(float) * H);
  orc_embedding_lookup(m->embed, &token, 1, h);
  const int32_t pos = cache->pos;
  for (int l = 0; l < c->n_layers; ++l) {
    const orc_layer_w* L = &m->layers[l];
    orc_rmsnorm(h, H, L->in_norm, c->eps, xn);
    if (is_full_layer(c, l))
      orc_attn_decode(c, &L->attn, xn, 1, cache->kc[l], cache->vc[l], cache->tmax, &pos, y);
    else
      orc_gdn_decode(c, &L->gdn, xn, 1, cache->conv[l], cache->rec[l], y);
    for (int i = 0; i < H; ++i) h[i] = h[i] + y[i];
    orc_rmsnorm(h, H, L->post_norm, c->eps, xn);
    orc_mlp_decode(c, &L->mlp, xn, 1, y);
    for (int i = 0; i < H; ++i) h[i] = h[i] + y[i];
  }
  orc_rmsnorm(h, H, m->final_norm, c->eps, xn);
  float* lg = logits ? logits : malloc(sizeof(float) * c->vocab);
  double* lg64 = malloc(sizeof(double) * c->vocab);
  orc_q8_gemv_nk(xn, 1, m->embed, lg, lg64);
  int32_t best = orc_argmax(lg, c->vocab);
  if (margin) {
    double b1 = -INFINITY, b2 = -INFINITY;
    for (int i = 0; i < c->vocab; ++i) {
      if (lg64[i] > b1) { b2 = b1; b1 = lg64[i]; } else if (lg64[i] > b2) b2 = lg64[i];
    }
    *margin = b1 - b2;
  }
  cache->pos += 1;
  if (!logits) free(lg);
  free(lg64); free(h); free(xn); free(y);
  return best;
}
