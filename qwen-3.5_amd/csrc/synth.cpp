// Host utilities: the seeded synthetic-weight generator, the Q8F quantiser, and the table of
// model tensors (names, shapes, storage kind and init rule) shared by the model builder and
// by q35_synth_model_tensor.
#include "q35_host.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <thread>
#include <vector>

namespace q35 {

namespace {

inline uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
  return z ^ (z >> 31);
}
constexpr uint64_t kGolden = 0x9E3779B97F4A7C15ULL;
inline uint64_t stream_key(uint64_t seed, uint64_t stream) { return mix64(seed ^ mix64(stream + kGolden)); }
// uniform in (0, 1): 53 random bits, centred in their cell so 0 and 1 never occur
inline double u01(uint64_t key, uint64_t c) {
  const uint64_t b = mix64(key + (c + 1) * kGolden);
  return ((double)(b >> 11) + 0.5) * 0x1.0p-53;
}
constexpr double kTwoPi = 6.283185307179586476925286766559;

}  // namespace

void parallel_for(int64_t n, const std::function<void(int64_t, int64_t)>& fn) {
  unsigned hw = std::thread::hardware_concurrency();
  int nt = (int)std::min<unsigned>(hw ? hw : 1, 32);
  if (n < (int64_t)1 << 16 || nt <= 1) { fn(0, n); return; }
  std::vector<std::thread> th;
  const int64_t per = (n + nt - 1) / nt;
  for (int t = 0; t < nt; ++t) {
    const int64_t a = t * per, b = std::min<int64_t>(n, a + per);
    if (a >= b) break;
    th.emplace_back([&fn, a, b] { fn(a, b); });
  }
  for (auto& t : th) t.join();
}

// Element i of a stream: Box-Muller pair i/2 from uniforms (2p, 2p+1); cos for even i, sin for odd.
void fill_normal(uint64_t seed, uint64_t stream, int64_t offset, int64_t n, float sigma, float* out) {
  const uint64_t key = stream_key(seed, stream);
  parallel_for(n, [&](int64_t a, int64_t b) {
    for (int64_t j = a; j < b; ++j) {
      const int64_t i = offset + j;
      const int64_t p = i >> 1;
      const double r = std::sqrt(-2.0 * std::log(u01(key, 2 * (uint64_t)p)));
      const double th = kTwoPi * u01(key, 2 * (uint64_t)p + 1);
      const double z = (i & 1) ? r * std::sin(th) : r * std::cos(th);
      out[j] = (float)((double)sigma * z);
    }
  });
}

void fill_uniform(uint64_t seed, uint64_t stream, int64_t offset, int64_t n, float lo, float hi, float* out) {
  const uint64_t key = stream_key(seed, stream);
  parallel_for(n, [&](int64_t a, int64_t b) {
    for (int64_t j = a; j < b; ++j) {
      const double u = u01(key, (uint64_t)(offset + j));
      out[j] = (float)((double)lo + ((double)hi - (double)lo) * u);
    }
  });
}

uint64_t fnv1a(const char* s) {
  uint64_t h = 0xcbf29ce484222325ULL;
  for (; *s; ++s) { h ^= (unsigned char)*s; h *= 0x100000001b3ULL; }
  return h;
}

void quantize_q8f(const float* w, int64_t rows, int64_t cols, int8_t* q, float* s) {
  const int64_t nb = cols / 64;
  parallel_for(rows, [&](int64_t r0, int64_t r1) {
    for (int64_t r = r0; r < r1; ++r) {
      for (int64_t b = 0; b < nb; ++b) {
        const float* src = w + r * cols + b * 64;
        float amax = 0.0f;
        for (int j = 0; j < 64; ++j) amax = std::max(amax, std::fabs(src[j]));
        const float sc = amax / 127.0f;
        s[r * nb + b] = sc;
        int8_t* dst = q + r * cols + b * 64;
        for (int j = 0; j < 64; ++j) {
          float v = (sc == 0.0f) ? 0.0f : std::round(src[j] / sc);
          v = std::min(127.0f, std::max(-127.0f, v));
          dst[j] = (int8_t)v;
        }
      }
    }
  });
}

void pack_kn_tiled(const int8_t* q, const float* s, int64_t K, int64_t N, int8_t* qt, float* st) {
  const int64_t ntile = (N + 255) / 256, nb = N / 64;
  parallel_for(ntile * K, [&](int64_t i0, int64_t i1) {
    for (int64_t i = i0; i < i1; ++i) {
      const int64_t t = i / K, k = i % K;
      for (int64_t c = 0; c < 256; ++c) {
        const int64_t n = t * 256 + c;
        qt[i * 256 + c] = n < N ? q[k * N + n] : 0;
      }
      for (int64_t j = 0; j < 4; ++j) {
        const int64_t b = t * 4 + j;
        st[i * 4 + j] = b < nb ? s[k * nb + b] : 0.0f;
      }
    }
  });
}

std::vector<TensorSpec> model_specs(const q35_dims& d) {
  std::vector<TensorSpec> v;
  const int64_t H = d.hidden, F = d.ffn, V = d.vocab;
  const int64_t nh = d.lin_heads, key_dim = (int64_t)d.lin_heads * d.lin_dk, vdim = (int64_t)d.lin_heads * d.lin_dv;
  const int64_t conv_dim = 2 * key_dim + vdim;
  const int64_t ah = d.attn_heads, kvh = d.kv_heads, hd = d.head_dim;
  v.push_back({"embed_tokens", V, H, kQ8NK, kInitNormal});
  v.push_back({"norm", 1, H, kF32, kInitZeros});
  for (int l = 0; l < d.n_layers; ++l) {
    const std::string p = "layers." + std::to_string(l) + ".";
    v.push_back({p + "input_layernorm", 1, H, kF32, kInitZeros});
    v.push_back({p + "post_attention_layernorm", 1, H, kF32, kInitZeros});
    if (!is_full_layer(d, l)) {
      const std::string a = p + "linear_attn.";
      v.push_back({a + "in_proj_qkv", H, conv_dim, kQ8KN, kInitNormal});
      v.push_back({a + "in_proj_z", H, vdim, kQ8KN, kInitNormal});
      v.push_back({a + "out_proj", vdim, H, kQ8KN, kInitNormal});
      v.push_back({a + "in_proj_b", H, nh, kF32, kInitNormal});
      v.push_back({a + "in_proj_a", H, nh, kF32, kInitNormal});
      v.push_back({a + "a_log", 1, nh, kF32, kInitALog});
      v.push_back({a + "dt_bias", 1, nh, kF32, kInitOnes});
      v.push_back({a + "conv1d", conv_dim, d.conv_k, kF32, kInitNormal});
      v.push_back({a + "norm", 1, d.lin_dv, kF32, kInitOnes});
    } else {
      const std::string a = p + "self_attn.";
      v.push_back({a + "q_proj", H, ah * hd * 2, kQ8KN, kInitNormal});
      v.push_back({a + "k_proj", H, kvh * hd, kQ8KN, kInitNormal});
      v.push_back({a + "v_proj", H, kvh * hd, kQ8KN, kInitNormal});
      v.push_back({a + "o_proj", ah * hd, H, kQ8KN, kInitNormal});
      v.push_back({a + "q_norm", 1, hd, kF32, kInitZeros});
      v.push_back({a + "k_norm", 1, hd, kF32, kInitZeros});
    }
    v.push_back({p + "mlp.gate_proj", H, F, kQ8KN, kInitNormal});
    v.push_back({p + "mlp.up_proj", H, F, kQ8KN, kInitNormal});
    v.push_back({p + "mlp.down_proj", F, H, kQ8KN, kInitNormal});
  }
  return v;
}

void synth_values(const TensorSpec& t, uint64_t seed, float* out) {
  const int64_t n = t.rows * t.cols;
  const uint64_t sid = fnv1a(t.name.c_str());
  switch (t.init) {
    case kInitNormal: fill_normal(seed, sid, 0, n, 0.02f, out); break;
    case kInitZeros: std::memset(out, 0, sizeof(float) * n); break;
    case kInitOnes: for (int64_t i = 0; i < n; ++i) out[i] = 1.0f; break;
    case kInitALog:
      fill_uniform(seed, sid, 0, n, 0.01f, 16.0f, out);
      for (int64_t i = 0; i < n; ++i) out[i] = std::log(out[i]);
      break;
  }
}

}  // namespace q35

using namespace q35;

extern "C" {

int q35_synth_normal(uint64_t seed, uint64_t stream, int64_t offset, int64_t n, float sigma, float* out_host) {
  if (!out_host || n < 0 || offset < 0) return fail(Q35_E_ARG, "synth_normal: bad argument");
  fill_normal(seed, stream, offset, n, sigma, out_host);
  return Q35_OK;
}

int q35_synth_uniform(uint64_t seed, uint64_t stream, int64_t offset, int64_t n, float lo, float hi, float* out_host) {
  if (!out_host || n < 0 || offset < 0) return fail(Q35_E_ARG, "synth_uniform: bad argument");
  fill_uniform(seed, stream, offset, n, lo, hi, out_host);
  return Q35_OK;
}

uint64_t q35_synth_stream_id(const char* name) { return name ? fnv1a(name) : 0; }

int q35_quantize_q8f(const float* w_host, int64_t rows, int64_t cols, int8_t* q_host, float* scale_host) {
  if (!w_host || !q_host || !scale_host) return fail(Q35_E_ARG, "quantize: null pointer");
  if (rows < 1 || cols < 64 || (cols % 64) != 0) return fail(Q35_E_SHAPE, "quantize: cols must be a positive multiple of 64");
  quantize_q8f(w_host, rows, cols, q_host, scale_host);
  return Q35_OK;
}

int64_t q35_q8f_tiled_q_count(int32_t K, int32_t N) { return (int64_t)((N + 255) / 256) * K * 256; }
int64_t q35_q8f_tiled_scale_count(int32_t K, int32_t N) { return (int64_t)((N + 255) / 256) * K * 4; }

int q35_q8f_pack_kn_tiled(const int8_t* q_host, const float* scale_host, int32_t K, int32_t N, int8_t* q_tiled_host,
                          float* scale_tiled_host) {
  if (!q_host || !scale_host || !q_tiled_host || !scale_tiled_host) return fail(Q35_E_ARG, "pack_kn_tiled: null pointer");
  if (K < 1 || N < 64 || (N % 64) != 0) return fail(Q35_E_SHAPE, "pack_kn_tiled: N must be a positive multiple of 64");
  pack_kn_tiled(q_host, scale_host, K, N, q_tiled_host, scale_tiled_host);
  return Q35_OK;
}

int q35_q8f_pack_kn_panel(const int8_t* q_host, const float* scale_host, int32_t K, int32_t N, int8_t* q_panel_host,
                          float* scale_panel_host) {
  if (!q_host || !scale_host || !q_panel_host || !scale_panel_host) return fail(Q35_E_ARG, "pack_kn_panel: null pointer");
  if (K < 1 || N < 64 || (N % 64) != 0) return fail(Q35_E_SHAPE, "pack_kn_panel: N must be a positive multiple of 64");
  const int64_t np = N / 16, nb = N / 64;
  parallel_for(np * K, [&](int64_t i0, int64_t i1) {  // i = panel * K + k
    for (int64_t i = i0; i < i1; ++i) {
      const int64_t p = i / K, k = i % K;
      std::memcpy(q_panel_host + i * 16, q_host + k * (int64_t)N + p * 16, 16);
    }
  });
  for (int64_t b = 0; b < nb; ++b)
    for (int64_t k = 0; k < K; ++k) scale_panel_host[b * K + k] = scale_host[k * nb + b];
  return Q35_OK;
}

int q35_synth_model_tensor(const q35_dims* d, uint64_t seed, const char* name, float* out_host, int64_t n) {
  if (!d || !name || !out_host) return fail(Q35_E_ARG, "synth_model_tensor: null pointer");
  for (const TensorSpec& t : model_specs(*d)) {
    if (t.name == name) {
      if (n != t.rows * t.cols) return fail(Q35_E_SHAPE, "synth_model_tensor: size mismatch for " + t.name);
      synth_values(t, seed, out_host);
      return Q35_OK;
    }
  }
  return fail(Q35_E_ARG, std::string("synth_model_tensor: unknown tensor ") + name);
}

}  // extern "C"
