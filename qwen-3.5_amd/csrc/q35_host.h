// Host-only declarations: synthetic init, quantiser, tensor table, model internals.
#pragma once
#include <functional>
#include <memory>
#include <string>
#include <vector>
#include "q35_internal.h"

namespace q35 {

enum { kF32 = 0, kQ8KN = 1, kQ8NK = 2 };
enum { kInitNormal = 0, kInitZeros = 1, kInitOnes = 2, kInitALog = 3 };

struct TensorSpec {
  std::string name;
  int64_t rows, cols;  // stored shape (Q8F blocks of 64 along cols)
  int kind;            // kF32 / kQ8KN / kQ8NK
  int init;            // kInit*
};

// Layer l is full attention iff (l + 1) % full_interval == 0 (text_config.rs layer_types:
// every 4th layer, indices 3, 7, ..., 23).
inline bool is_full_layer(const q35_dims& d, int l) { return ((l + 1) % d.full_interval) == 0; }

void parallel_for(int64_t n, const std::function<void(int64_t, int64_t)>& fn);
void fill_normal(uint64_t seed, uint64_t stream, int64_t offset, int64_t n, float sigma, float* out);
void fill_uniform(uint64_t seed, uint64_t stream, int64_t offset, int64_t n, float lo, float hi, float* out);
uint64_t fnv1a(const char* s);
void quantize_q8f(const float* w, int64_t rows, int64_t cols, int8_t* q, float* s);
// Q35_KN -> Q35_KN_TILED: q[t][K][256], s[t][K][4], columns past N zero
void pack_kn_tiled(const int8_t* q, const float* s, int64_t K, int64_t N, int8_t* qt, float* st);
std::vector<TensorSpec> model_specs(const q35_dims& d);
void synth_values(const TensorSpec& t, uint64_t seed, float* out);
int validate_dims(const q35_dims& d);

// safetensors checkpoint (weights.cpp)
struct SafeTensors;
struct SafeTensorsClose {
  void operator()(SafeTensors* s) const;
};
using SafeTensorsPtr = std::unique_ptr<SafeTensors, SafeTensorsClose>;
SafeTensorsPtr open_safetensors(const std::string& path, int* rc);
// the f32 values of decoder tensor t in the builder's layout (Linear weights transposed to [in][out])
int safetensors_values(const SafeTensors& st, const TensorSpec& t, float* out);

}  // namespace q35
