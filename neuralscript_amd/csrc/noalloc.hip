// Allocation-free entry point: the embedding weight gradient with its
// scratch in a fixed, file-scope device array instead of a workspace the
// caller allocates (or the library allocates).  For callers that cannot
// call hipMalloc: code under HIP graph capture, serving loops, harnesses
// that forbid allocation.
//
// `scratch` holds the counting-sort state of launch_embedding_grad (ints:
// count [V], start [V+1], cursor [V], order [n], tmp [n]); it exists once
// per GPU for the life of the process.  Its address on a device comes from
// hipGetSymbolAddress, made once per device with that device current; the
// array's name itself is only a host-side stand-in and is never passed to a
// kernel or a copy.
#include <hip/hip_runtime.h>

#include <mutex>
#include <string>

#include "common.h"
#include "kernels.h"
#include "nship.h"

namespace nship {
namespace {

constexpr int64_t kScratchInts = NSH_EMBEDDING_GRAD_NOALLOC_MAX_INTS;
constexpr int kMaxDevices = 64;

static __device__ __align__(256) int scratch[kScratchInts];

struct DeviceScratch {
  std::once_flag once;
  void* ptr = nullptr;
  hipError_t err = hipSuccess;
};
DeviceScratch g_scratch[kMaxDevices];

// The scratch array's address on the current device (resolved once per device).
int scratch_on_current_device(int** out) {
  int dev = -1;
  NSH_CHECK(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxDevices) {
    set_error("embedding_grad_noalloc: device index out of range");
    return -1;
  }
  DeviceScratch& d = g_scratch[dev];
  std::call_once(d.once, [&d]() {
    void* p = nullptr;
    d.err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (d.err == hipSuccess) d.ptr = p;
  });
  if (d.err != hipSuccess || !d.ptr) {
    set_error(std::string("embedding_grad_noalloc: hipGetSymbolAddress: ") + hipGetErrorString(d.err));
    return -1;
  }
  *out = static_cast<int*>(d.ptr);
  return 0;
}

}  // namespace
}  // namespace nship

using namespace nship;

extern "C" int nsh_op_embedding_grad_noalloc(const float* dout, const float* idx, float* dW, int64_t n, int64_t V,
                                             int64_t D, void* stream) {
  if (n < 0 || V < 0 || D < 0 || (V * D > 0 && !dW) || (n > 0 && (!dout || !idx))) {
    set_error("embedding_grad_noalloc: null pointer or bad size");
    return -1;
  }
  if (V == 0 || D == 0) return 0;  // dW is empty, as in nsh_op_embedding_grad
  if ((int64_t)embedding_grad_workspace(n, V) > kScratchInts) {
    set_error("embedding_grad_noalloc: 3*V + 1 + 2*n = " + std::to_string(embedding_grad_workspace(n, V)) +
              " ints exceeds the static scratch of " + std::to_string(kScratchInts) +
              " ints; use nsh_op_embedding_grad with a workspace");
    return -1;
  }
  int* ws = nullptr;
  if (scratch_on_current_device(&ws) != 0) return -1;
  return launch_embedding_grad(dout, idx, dW, n, V, D, ws, static_cast<hipStream_t>(stream));
}
