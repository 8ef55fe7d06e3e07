// On-device peak microbenchmarks: the attainable fp32 MFMA rate and HBM copy
// bandwidth of the running GPU, against which the kernels' roofline
// fractions can be read (the published peaks assume the 2.4 GHz clock, which
// dense MFMA work does not hold).  No reference counterpart: the reference
// has no timing at all.
#include "common.h"
#include "kernels.h"

#include <algorithm>

namespace nship {
namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));

// Every wave issues iters x 4 independent 32x32x2 fp32 MFMAs on register
// operands (no memory traffic in the loop).  The result is stored only on a
// value the accumulators never reach, so the loop cannot be removed.
__global__ __launch_bounds__(256) void mfma_peak_kernel(float* __restrict__ out, int iters) {
  floatx16 acc[4];
#pragma unroll
  for (int j = 0; j < 4; j++)
#pragma unroll
    for (int v = 0; v < 16; v++) acc[j][v] = 0.f;
  const float a = 1e-3f * (float)(threadIdx.x & 63), b = 1e-3f;
  for (int i = 0; i < iters; i++) {
#pragma unroll
    for (int j = 0; j < 4; j++) acc[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, acc[j], 0, 0, 0);
  }
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < 4; j++)
#pragma unroll
    for (int v = 0; v < 16; v++) s += acc[j][v];
  if (s == -1.f) out[threadIdx.x] = s;
}

// dst = src, float4 per thread and step, grid-stride.
__global__ __launch_bounds__(256) void copy4_kernel(const float4* __restrict__ src, float4* __restrict__ dst,
                                                    int64_t n4) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += (int64_t)gridDim.x * 256) dst[i] = src[i];
}

}  // namespace

int bench_mfma_peak(int iters, int blocks, float* out, float* ms) {
  hipEvent_t a, b;
  NSH_CHECK(hipEventCreate(&a));
  NSH_CHECK(hipEventCreate(&b));
  hipLaunchKernelGGL(mfma_peak_kernel, dim3(blocks), dim3(256), 0, nullptr, out, iters);  // warm-up
  NSH_LAUNCHED();
  NSH_CHECK(hipEventRecord(a, nullptr));
  hipLaunchKernelGGL(mfma_peak_kernel, dim3(blocks), dim3(256), 0, nullptr, out, iters);
  NSH_LAUNCHED();
  NSH_CHECK(hipEventRecord(b, nullptr));
  NSH_CHECK(hipEventSynchronize(b));
  NSH_CHECK(hipEventElapsedTime(ms, a, b));
  NSH_CHECK(hipEventDestroy(a));
  NSH_CHECK(hipEventDestroy(b));
  return 0;
}

int bench_copy(const float* src, float* dst, int64_t n, int reps, float* ms) {
  const int64_t n4 = n / 4;
  const unsigned grid = (unsigned)std::min<int64_t>(ceil_div(n4, 256), 16384);
  hipEvent_t a, b;
  NSH_CHECK(hipEventCreate(&a));
  NSH_CHECK(hipEventCreate(&b));
  hipLaunchKernelGGL(copy4_kernel, dim3(grid), dim3(256), 0, nullptr, (const float4*)src, (float4*)dst, n4);
  NSH_LAUNCHED();
  NSH_CHECK(hipEventRecord(a, nullptr));
  for (int r = 0; r < reps; r++) {
    hipLaunchKernelGGL(copy4_kernel, dim3(grid), dim3(256), 0, nullptr, (const float4*)src, (float4*)dst, n4);
    NSH_LAUNCHED();
  }
  NSH_CHECK(hipEventRecord(b, nullptr));
  NSH_CHECK(hipEventSynchronize(b));
  NSH_CHECK(hipEventElapsedTime(ms, a, b));
  *ms /= (float)reps;
  NSH_CHECK(hipEventDestroy(a));
  NSH_CHECK(hipEventDestroy(b));
  return 0;
}

}  // namespace nship
