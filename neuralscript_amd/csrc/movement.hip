// Forward-only elementwise and data-movement instructions of the reference's
// CPU emitter, as HIP kernels on device buffers:
//
//   binop      ns_binop        codegen.cpp:1267-1278   C[i] = A[i] op B[i % nb]  (nb = 0: B = 0)
//   softmax    ns_softmax      codegen.cpp:1293-1303   rows of `last`, max / expf / sum / divide
//   transpose  ns_transpose2d  codegen.cpp:1638-1644
//   concat     ns_concat2/0    codegen.cpp:1646-1661
//   slice      ns_slice2/rows  codegen.cpp:1663-1676
//   index      ns_index2/rows  codegen.cpp:1678-1691
//   scatter    ns_scatter2/rows codegen.cpp:1693-1709 (later indices win)
//   dropout    train-mode mask apply, codegen.cpp:2874-2893, :3066-3073
//
// All are HBM-bound copies or single-pass elementwise work; the launchers
// assume the host has checked every index against its buffer.
#include "common.h"
#include "kernels.h"

namespace nship {
namespace {

__global__ __launch_bounds__(256) void binop_kernel(const float* __restrict__ A, const float* __restrict__ B,
                                                    float* __restrict__ C, int64_t na, int64_t nb, int code) {
#pragma clang fp contract(off)
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= na) return;
  const float a = A[i];
  const float b = nb > 0 ? B[i % nb] : 0.f;
  float c;
  switch (code) {
    case 1: c = a - b; break;
    case 2: c = a * b; break;
    case 3: c = a / b; break;
    default: c = a + b; break;
  }
  C[i] = c;
}

// One wave per row of `last` values.
__global__ __launch_bounds__(256) void softmax_rows_kernel(const float* __restrict__ in, float* __restrict__ out,
                                                           int64_t rows, int64_t last) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;
  const float* x = in + r * last;
  float* y = out + r * last;
  float mx = -INFINITY;
  for (int64_t j = lane; j < last; j += 64) mx = fmaxf(mx, x[j]);
  mx = wave_max(mx);
  float s = 0.f;
  for (int64_t j = lane; j < last; j += 64) s += expf(x[j] - mx);
  s = wave_sum(s);
  for (int64_t j = lane; j < last; j += 64) y[j] = expf(x[j] - mx) / s;
}

// out[j * R + i] = in[i * C + j], 32 x 32 tiles through LDS.
__global__ __launch_bounds__(256) void transpose_kernel(const float* __restrict__ in, float* __restrict__ out,
                                                        int64_t R, int64_t C) {
  __shared__ float t[32][33];
  const int64_t i0 = (int64_t)blockIdx.y * 32, j0 = (int64_t)blockIdx.x * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 x 8
  for (int k = ty; k < 32; k += 8) {
    const int64_t i = i0 + k, j = j0 + tx;
    if (i < R && j < C) t[k][tx] = in[i * C + j];
  }
  __syncthreads();
  for (int k = ty; k < 32; k += 8) {
    const int64_t j = j0 + k, i = i0 + tx;
    if (i < R && j < C) out[j * R + i] = t[tx][k];
  }
}

__global__ __launch_bounds__(256) void concat_cols_kernel(const float* __restrict__ a, const float* __restrict__ b,
                                                          float* __restrict__ out, int64_t R, int64_t ca,
                                                          int64_t cb) {
  const int64_t co = ca + cb;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= R * co) return;
  const int64_t r = i / co, c = i % co;
  out[i] = c < ca ? a[r * ca + c] : b[r * cb + (c - ca)];
}

// out[r, j] = in[r * C + s + j], j < w  (column slice)
__global__ __launch_bounds__(256) void slice_cols_kernel(const float* __restrict__ in, float* __restrict__ out,
                                                         int64_t M, int64_t C, int64_t s, int64_t w) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= M * w) return;
  const int64_t r = i / w, j = i % w;
  out[i] = in[r * C + s + j];
}

// axis 1: out[r, k] = in[r * C + idx[k]];  axis 0: out[k, c] = in[idx[k] * C + c]
__global__ __launch_bounds__(256) void index_kernel(const float* __restrict__ in, const int64_t* __restrict__ idx,
                                                    float* __restrict__ out, int64_t M, int64_t C, int64_t L,
                                                    int axis) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (axis == 1) {
    if (i >= M * L) return;
    const int64_t r = i / L, k = i % L;
    out[i] = in[r * C + idx[k]];
  } else {
    if (i >= L * C) return;
    const int64_t k = i / C, c = i % C;
    out[i] = in[idx[k] * C + c];
  }
}

// Scatter as a gather of the final values: element (r, c) of the R x C result
// takes the update of the LAST k that targets it (the reference writes the
// updates in k order), else the input.
//   axis 1: targets are columns, update (r, k) = upd[r * L + k]
//   axis 0: targets are rows,    update (k, c) = upd[k * C + c]
__global__ __launch_bounds__(256) void scatter_kernel(const float* __restrict__ in, const int64_t* __restrict__ idx,
                                                      const float* __restrict__ upd, float* __restrict__ out,
                                                      int64_t R, int64_t C, int64_t L, int axis) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= R * C) return;
  const int64_t r = i / C, c = i % C;
  const int64_t target = axis == 1 ? c : r;
  int64_t hit = -1;
  for (int64_t k = 0; k < L; k++)
    if (idx[k] == target) hit = k;
  if (hit < 0) out[i] = in[i];
  else out[i] = axis == 1 ? upd[r * L + hit] : upd[hit * C + c];
}

// y = x * m, m = keep ? scale : 0 (codegen.cpp:2887 forward, :3066-3073
// backward with the same mask).
__global__ __launch_bounds__(256) void dropout_kernel(const float* __restrict__ x, const uint8_t* __restrict__ keep,
                                                      float* __restrict__ y, int64_t n, float scale) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const float m = keep[i] ? scale : 0.f;
  y[i] = x[i] * m;
}

__global__ void fill_kernel(float* __restrict__ out, int64_t n, float v) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) out[i] = v;
}

__global__ void copy_kernel(const float* __restrict__ in, float* __restrict__ out, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) out[i] = in[i];
}

unsigned blocks(int64_t n) { return (unsigned)ceil_div(n, 256); }

}  // namespace

int launch_binop(const float* A, const float* B, float* C, int64_t na, int64_t nb, int code, hipStream_t s) {
  if (na <= 0) return 0;
  hipLaunchKernelGGL(binop_kernel, dim3(blocks(na)), dim3(256), 0, s, A, B, C, na, nb, code);
  NSH_LAUNCHED();
  return 0;
}

int launch_softmax(const float* in, float* out, int64_t n, int64_t last, hipStream_t s) {
  if (n <= 0) return 0;
  if (last < 1) last = 1;
  const int64_t rows = n / last, tail = n - rows * last;
  if (rows > 0) {
    hipLaunchKernelGGL(softmax_rows_kernel, dim3((unsigned)ceil_div(rows, 4)), dim3(256), 0, s, in, out, rows, last);
    NSH_LAUNCHED();
  }
  if (tail > 0) return launch_copy(in + rows * last, out + rows * last, tail, s);
  return 0;
}

int launch_transpose(const float* in, float* out, int64_t R, int64_t C, hipStream_t s) {
  if (R <= 0 || C <= 0) return 0;
  hipLaunchKernelGGL(transpose_kernel, dim3((unsigned)ceil_div(C, 32), (unsigned)ceil_div(R, 32)), dim3(256), 0, s,
                     in, out, R, C);
  NSH_LAUNCHED();
  return 0;
}

int launch_concat_cols(const float* a, const float* b, float* out, int64_t R, int64_t ca, int64_t cb, hipStream_t s) {
  if (R <= 0 || ca + cb <= 0) return 0;
  hipLaunchKernelGGL(concat_cols_kernel, dim3(blocks(R * (ca + cb))), dim3(256), 0, s, a, b, out, R, ca, cb);
  NSH_LAUNCHED();
  return 0;
}

int launch_slice_cols(const float* in, float* out, int64_t M, int64_t C, int64_t start, int64_t width,
                      hipStream_t s) {
  if (M <= 0 || width <= 0) return 0;
  hipLaunchKernelGGL(slice_cols_kernel, dim3(blocks(M * width)), dim3(256), 0, s, in, out, M, C, start, width);
  NSH_LAUNCHED();
  return 0;
}

int launch_index(const float* in, const int64_t* idx, float* out, int64_t M, int64_t C, int64_t L, int axis,
                 hipStream_t s) {
  const int64_t n = axis == 1 ? M * L : L * C;
  if (n <= 0) return 0;
  hipLaunchKernelGGL(index_kernel, dim3(blocks(n)), dim3(256), 0, s, in, idx, out, M, C, L, axis);
  NSH_LAUNCHED();
  return 0;
}

int launch_scatter(const float* in, const int64_t* idx, const float* upd, float* out, int64_t R, int64_t C,
                   int64_t L, int axis, hipStream_t s) {
  if (R * C <= 0) return 0;
  hipLaunchKernelGGL(scatter_kernel, dim3(blocks(R * C)), dim3(256), 0, s, in, idx, upd, out, R, C, L, axis);
  NSH_LAUNCHED();
  return 0;
}

int launch_dropout(const float* x, const uint8_t* keep, float* y, int64_t n, float scale, hipStream_t s) {
  if (n <= 0) return 0;
  hipLaunchKernelGGL(dropout_kernel, dim3(blocks(n)), dim3(256), 0, s, x, keep, y, n, scale);
  NSH_LAUNCHED();
  return 0;
}

int launch_fill(float* out, int64_t n, float v, hipStream_t s) {
  if (n <= 0) return 0;
  hipLaunchKernelGGL(fill_kernel, dim3(blocks(n)), dim3(256), 0, s, out, n, v);
  NSH_LAUNCHED();
  return 0;
}

int launch_copy(const float* in, float* out, int64_t n, hipStream_t s) {
  if (n <= 0) return 0;
  hipLaunchKernelGGL(copy_kernel, dim3(blocks(n)), dim3(256), 0, s, in, out, n);
  NSH_LAUNCHED();
  return 0;
}

}  // namespace nship
