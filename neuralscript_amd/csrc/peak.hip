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

namespace {
// Deterministic values in [-0.5, 0.5) (a multiplicative hash of the index).
__global__ __launch_bounds__(256) void fill_hash_kernel(float* __restrict__ p, int64_t n, float scale) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
    p[i] = scale * ((float)(((uint32_t)i * 2654435761u) >> 8) * (1.0f / 16777216.0f) - 0.5f);
}

int fill_hash(float* p, int64_t n, float scale) {
  hipLaunchKernelGGL(fill_hash_kernel, dim3((unsigned)std::min<int64_t>(ceil_div(n, 256), 8192)), dim3(256), 0,
                     nullptr, p, n, scale);
  NSH_LAUNCHED();
  return 0;
}
}  // namespace

// The row kernels of a training step at one shape, each timed over `reps`
// back-to-back launches between one pair of events (a launch's own event
// pair adds microseconds, a large share of a 10-50 us kernel).  us[0..4]:
// embedding gather, LayerNorm, LayerNorm gradient, embedding gradient,
// softmax cross-entropy with its gradient.
int bench_rowops(const float* idx, const float* labels, int64_t M, int64_t D, int64_t V, int64_t C, int reps,
                 double* us) {
  float *W = nullptr, *x = nullptr, *y = nullptr, *d = nullptr, *logits = nullptr, *grad = nullptr, *row = nullptr,
        *loss = nullptr;
  int* ws = nullptr;
  hipEvent_t a = nullptr, b = nullptr;
  int rc = -1;
  auto run = [&](int k, auto&& launch) -> int {
    if (launch() != 0) return -1;  // warm-up
    NSH_CHECK(hipEventRecord(a, nullptr));
    for (int r = 0; r < reps; r++)
      if (launch() != 0) return -1;
    NSH_CHECK(hipEventRecord(b, nullptr));
    NSH_CHECK(hipEventSynchronize(b));
    float ms = 0.f;
    NSH_CHECK(hipEventElapsedTime(&ms, a, b));
    us[k] = (double)ms * 1e3 / reps;
    return 0;
  };
  do {
    const size_t md = (size_t)M * D;
    if (hipMalloc(&W, (size_t)V * D * 4) != hipSuccess || hipMalloc(&x, md * 4) != hipSuccess ||
        hipMalloc(&y, md * 4) != hipSuccess || hipMalloc(&d, md * 4) != hipSuccess ||
        hipMalloc(&logits, (size_t)M * C * 4) != hipSuccess || hipMalloc(&grad, (size_t)M * C * 4) != hipSuccess ||
        hipMalloc(&row, (size_t)M * 4) != hipSuccess || hipMalloc(&loss, 4) != hipSuccess ||
        hipMalloc(&ws, embedding_grad_workspace(M, V) * sizeof(int)) != hipSuccess) {
      set_error("bench_rowops: hipMalloc failed");
      break;
    }
    if (fill_hash(W, (int64_t)V * D, 0.04f) || fill_hash(x, (int64_t)md, 2.f) || fill_hash(d, (int64_t)md, 2e-3f) ||
        fill_hash(logits, M * C, 4.f))
      break;
    if (hipEventCreate(&a) != hipSuccess || hipEventCreate(&b) != hipSuccess) {
      set_error("bench_rowops: hipEventCreate failed");
      break;
    }
    if (run(0, [&] { return launch_embedding(W, idx, y, M, V, D, nullptr); }) ||
        run(1, [&] { return launch_layernorm(x, y, M, D, nullptr); }) ||
        run(2, [&] { return launch_layernorm_grad(d, x, y, M, D, nullptr); }) ||
        run(3, [&] { return launch_embedding_grad(d, idx, W, M, V, D, ws, nullptr); }) ||
        run(4, [&] { return launch_softmax_xent(logits, labels, grad, row, loss, M, C, true, nullptr); }))
      break;
    rc = 0;
  } while (false);
  if (a) hipEventDestroy(a);
  if (b) hipEventDestroy(b);
  for (void* p : {(void*)W, (void*)x, (void*)y, (void*)d, (void*)logits, (void*)grad, (void*)row, (void*)loss,
                  (void*)ws})
    if (p) hipFree(p);
  return rc;
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
