// q35_q8_gemv_noalloc: the Q8F matvec of q35_q8_gemv for callers that cannot allocate device
// memory (code under hipGraph capture, serving loops, harnesses that forbid hipMalloc).  The
// split-K path of the KN / KN_TILED layouts needs scratch (one completion counter per 256-column
// tile and M x N fixed-point accumulators); here it lives in a file-scope device array of fixed
// size instead of a caller workspace.  The panel and NK layouts need no scratch and take the same
// kernels as q35_q8_gemv.
//
// The array's host-side name is only a stand-in for the symbol: its device address is fetched
// once per device with hipGetSymbolAddress (with that device current) and only that address is
// passed to kernels.  Every GPU holds its own copy until the process ends.  The counters and
// accumulators must be zero when a call starts; the load-time image is zero, a fill kernel clears
// the array once more on the first call on each device, and every call leaves both zero again
// (the last block of each tile re-zeroes its accumulators and its counter).
#include "q35_host.h"

#include <mutex>

namespace q35 {

namespace {

constexpr size_t kNoAllocAccBytes = (size_t)1 << 20;  // M * N <= 131072 fixed-point sums
constexpr size_t kNoAllocBytes = kCounterBytes + kNoAllocAccBytes;
constexpr int kMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kNoAllocBytes];

struct DevScratch {
  void* ptr = nullptr;
  bool ready = false;
};
DevScratch g_dev[kMaxDevices];
std::mutex g_mu;

__global__ __launch_bounds__(256) void clear_kernel(unsigned long long* p, size_t n) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) p[i] = 0ull;
}

// Device address of this device's scratch (set up on the first call on the device: symbol
// address, then one clearing kernel on the caller's stream, ahead of the caller's kernels).
int scratch_for_device(hipStream_t st, void** out) {
  int dev = 0;
  Q35_HIP_TRY(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxDevices) return fail(Q35_E_ARG, "q8_gemv_noalloc: device index out of range");
  std::lock_guard<std::mutex> lock(g_mu);
  DevScratch& d = g_dev[dev];
  if (!d.ready) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(Q35_E_HIP, std::string("q8_gemv_noalloc: hipGetSymbolAddress: ") + hipGetErrorString(e));
    hipLaunchKernelGGL(clear_kernel, dim3(64), dim3(256), 0, st, static_cast<unsigned long long*>(p),
                       kNoAllocBytes / sizeof(unsigned long long));
    Q35_HIP_TRY(hipGetLastError());
    d.ptr = p;
    d.ready = true;
  }
  *out = d.ptr;
  return Q35_OK;
}

}  // namespace

}  // namespace q35

using namespace q35;

extern "C" int q35_q8_gemv_noalloc(const float* x, int32_t M, q35_q8f W, float* y, void* stream) {
  if (!x || !y) return fail(Q35_E_ARG, "q8_gemv_noalloc: null x or y");
  if (M < 1 || M > 64) return fail(Q35_E_SHAPE, "q8_gemv_noalloc: M must be in [1, 64]");
  if (W.layout != Q35_KN && W.layout != Q35_KN_TILED)  // these need no scratch
    return q35_q8_gemv(x, M, W, y, nullptr, 0, stream);
  if (!W.q || !W.scale) return fail(Q35_E_ARG, "q8_gemv_noalloc: null Q8F pointer");
  const int K = W.rows, N = W.cols;
  if (K < 1 || N < 64 || (N % 64) != 0) return fail(Q35_E_SHAPE, "q8_gemv_noalloc: N must be a positive multiple of 64");
  const int mg = M < 8 ? M : 8;  // rows per launch
  if ((size_t)mg * N * sizeof(fx_t) > kNoAllocAccBytes)
    return fail(Q35_E_SHAPE, "q8_gemv_noalloc: min(M, 8) * N must be <= 131072 (its fixed scratch holds 1 MiB of "
                             "split-K sums); use q35_q8_gemv with a workspace");
  if ((N + 255) / 256 > kMaxCounters) return fail(Q35_E_SHAPE, "q8_gemv_noalloc: too many column tiles");
  hipStream_t st = static_cast<hipStream_t>(stream);
  void* ws = nullptr;
  int rc = scratch_for_device(st, &ws);
  if (rc) return rc;
  // the scratch has a workspace's layout: counters, then the accumulators
  return q35_q8_gemv(x, M, W, y, ws, kNoAllocBytes, stream);
}
