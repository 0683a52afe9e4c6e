// The decoder model's host-side state, shared by the model entry points (model.cpp) and the
// batched decoder (batch.cpp).  Not part of the C ABI.
#pragma once
#include "q35_host.h"

#include <map>
#include <string>
#include <vector>

struct q35_model {
  q35_dims d;
  uint64_t seed = 0;
  int32_t tmax = 0;
  int32_t host_pos = 0;  // host mirror of the device position
  struct Buf { void* p; size_t bytes; };
  std::map<std::string, Buf> tensors;
  std::vector<void*> allocs;
  struct Q8 { const int8_t* q; const float* s; int rows, cols; };
  struct Layer {
    bool full = false;
    const float *in_norm = nullptr, *post_norm = nullptr;
    Q8 qkv{}, z{}, out{}, q{}, k{}, v{}, o{}, gate{}, up{}, down{};
    const float *w_b = nullptr, *w_a = nullptr, *a_log = nullptr, *dt_bias = nullptr, *conv_w = nullptr, *norm_w = nullptr;
    const float *q_norm = nullptr, *k_norm = nullptr;
    float *conv_state = nullptr, *rec = nullptr, *kc = nullptr, *vc = nullptr;
  };
  std::vector<Layer> layers;
  Q8 embed{};
  const float* final_norm = nullptr;
  float *rope_cos = nullptr, *rope_sin = nullptr;
  q35::fx_t* h = nullptr;         // residual stream [hidden]
  q35::fx_t* acc_proj = nullptr;  // q|k|v|z (linear) or q|k|v (full) projection outputs
  q35::fx_t* acc_ba = nullptr;    // raw in_proj_b | in_proj_a sums [2*lin_heads]
  q35::fx_t* acc_gu = nullptr;    // gate | up [2*ffn]
  float *o_raw = nullptr, *attn = nullptr, *logits = nullptr;
  int64_t acc_proj_n = 0;
  int32_t *token = nullptr, *pos = nullptr, *prompt = nullptr, *plen = nullptr, *hist = nullptr;
  int32_t* pinned = nullptr;
  // host token stream of the persistent decode: pinned, coherent host memory [tmax] and its
  // device address (q35_model_decode_stream)
  int32_t* tok_stream = nullptr;
  int32_t* tok_stream_dev = nullptr;
  int32_t stream_p0 = 0, stream_max = 0;  // the last streamed launch: start position, steps given
  void* ws = nullptr;
  size_t ws_bytes = 0;
  hipStream_t own_stream = nullptr;
  hipGraphExec_t exec = nullptr;
  hipGraph_t graph = nullptr;
  // persistent decode-step kernel (launch mode 2)
  int step_grid = 0;
  int step_rc = Q35_OK;  // why the persistent kernel cannot run here, if it cannot
  std::string step_msg;
  q35::StepArgs step_args{};
  bool step_failed = false;  // a check found the sticky error word set (cleared by reset)
  const char* step_fail_msg = "";
  int step_fail_code = Q35_E_HIP;  // Q35_E_HIP (a wait timed out) or Q35_E_RANGE
  // prompt path (allocated on first use): up to pf_cap tokens per pass
  int pf_cap = 0, pf_ldy = 0, pf_lda = 0;
  float *pf_x = nullptr, *pf_xn = nullptr, *pf_y = nullptr, *pf_a = nullptr, *pf_core = nullptr;
  float *pf_bg = nullptr, *pf_q = nullptr, *pf_scr = nullptr, *pf_part = nullptr, *pf_aux = nullptr;
  float* pf_act_max = nullptr;  // row maxima of the SwiGLU rows (down_proj's input)
  // batched decode (allocated on first use): every projection again in the MB layout of the
  // matrix-core batch kernels (q[N/64][K/16][64][16], scale[N/64][K])
  struct Mb {
    const int8_t* q = nullptr;
    const int8_t* qs = nullptr;   // the same bytes in stream order (batched decode; mb_stream_launch)
    const float* s = nullptr;
    const float* f = nullptr;     // batched RMS launches: split factor per column block
    const float* smax = nullptr;  // max |scale| (prompt GEMMs)
  };
  // gu: gate and up interleaved by 64-column block (the prompt GEMM's fused SwiGLU; built with
  // the prompt buffers)
  struct MbLayer { Mb qkv, z, out, q, k, v, o, gate, up, down, gu; };
  std::vector<MbLayer> mb;
  const float* embed_scale_t = nullptr;  // the embedding table's scales transposed [hidden/64][vocab]
  const int8_t* embed_lm = nullptr;      // the embedding table in the batched lm_head's load order
};

namespace q35 {

int dev_alloc(q35_model* m, const std::string& name, size_t bytes, void** out);
template <class T>
int dev_alloc_t(q35_model* m, const std::string& name, size_t n, T** out) {
  void* p = nullptr;
  int rc = dev_alloc(m, name, n * sizeof(T), &p);
  *out = static_cast<T*>(p);
  return rc;
}
hipStream_t pick(q35_model* m, void* s);

// Where a prompt pass reads and writes one sequence's state: per-layer caches (null where a layer
// has none), the token slot, the position and the history (positions 0 .. tmax-1).
struct SeqView {
  std::vector<float*> conv, rec, kc, vc;
  int32_t *token = nullptr, *pos = nullptr, *hist = nullptr;
  int32_t tmax = 0;
};
SeqView model_view(q35_model* m);
// Allocates the prompt-path scratch and builds the MB weight copies on first use.
int ensure_prefill(q35_model* m, hipStream_t st);
// One prompt pass of T <= m->pf_cap tokens (device ids) at positions p0.. of sequence v.
int prefill_pass(q35_model* m, const SeqView& v, const int32_t* ids, int T, int p0, hipStream_t st);
// Builds the MB-layout copies of the projection weights on first use.
int ensure_mb(q35_model* m, hipStream_t st);

}  // namespace q35
