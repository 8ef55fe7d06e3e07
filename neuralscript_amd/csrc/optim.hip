// Fused optimizer step (OPT_STEP), codegen.cpp:3088-3124.
//
// Rule by shape (codegen.cpp:3097): Muon iff r > 1, c > 1, min(r, c) >= 8,
// else AdamW.
//
// AdamW (codegen.cpp:3108-3119), per weight step counter t:
//   m = 0.9 m + 0.1 g;  v = 0.999 v + 0.001 g g
//   w -= lr (m / b1t) / (sqrt(v / b2t) + 1e-8) + (0.01 lr) w,  b1t = 1 - 0.9^t ...
// evaluated in the same operation order with contraction off, so given the
// same gradient the update is bit-identical to the reference's.
//
// Muon (codegen.cpp:3099-3107): the momentum buffer is cleared after every
// apply, so m = g; Q = MGS(g) over columns (r >= c) or rows (r < c),
// ns_orthonom codegen.cpp:1617-1633; w -= lr sqrt(min(r,c)) Q + (0.01 lr) w.
//
// MGS on the GPU, right-looking: at step j every later vector v_c is
// projected against q_j = v_j / (|v_j| + 1e-30).  Each vector receives the
// same projections in the same order as in the reference's left-looking
// loop; only the order inside each dot product differs (tree reductions).
// All Muon matrices of the step advance together: one launch per column
// index j, each workgroup owning a few later vectors of one matrix and
// recomputing |v_j| itself (same reduction tree in every workgroup, so every
// workgroup sees the same norm).  Vectors are stored contiguously in a
// work buffer T[C][R] (a transpose of g for r >= c).
#include "common.h"
#include "kernels.h"

namespace nship {
namespace {

constexpr int kCPB = 4;  // later vectors per workgroup per step

__global__ __launch_bounds__(256) void adamw_kernel(float* __restrict__ w, const float* __restrict__ g,
                                                    float* __restrict__ m, float* __restrict__ v, int64_t n, float lr,
                                                    float b1t, float b2t) {
#pragma clang fp contract(off)
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const float gg = g[i];
  const float mi = 0.9f * m[i] + 0.1f * gg;
  const float vi = 0.999f * v[i] + 0.001f * gg * gg;
  m[i] = mi;
  v[i] = vi;
  const float mh = mi / b1t, vh = vi / b2t;
  const float wi = w[i];
  w[i] = wi - ((lr * mh / (sqrtf(vh) + 1e-8f)) + (0.01f * lr) * wi);
}

// Block-wide sum (256 threads), fixed tree.
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  return (red[0] + red[1]) + (red[2] + red[3]);
}

__global__ __launch_bounds__(256) void muon_gather_kernel(const MuonMat* __restrict__ mats, int nmat) {
  // grid.y = matrix; each thread copies one element of g into T (vector-major)
  const MuonMat& M = mats[blockIdx.y];
  const int64_t n = (int64_t)M.R * M.C;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    // T[j][k]: vector j, element k
    if (M.transposed) {
      M.T[i] = M.g[i];  // rows of g are the vectors
    } else {
      const int64_t j = i / M.R, k = i % M.R;  // g[k][j], g is [R][C]
      M.T[i] = M.g[k * M.C + j];
    }
  }
  (void)nmat;
}

__global__ __launch_bounds__(256) void mgs_step_kernel(const MuonMat* __restrict__ mats, int nmat, int j) {
  __shared__ float red[4];
  // locate this workgroup's matrix
  int b = blockIdx.x, mi = 0;
  while (mi < nmat && b >= mats[mi].nblk) {
    b -= mats[mi].nblk;
    mi++;
  }
  if (mi >= nmat) return;
  const MuonMat& M = mats[mi];
  if (j >= M.C) return;
  const int R = M.R;
  const float* __restrict__ vj = M.T + (int64_t)j * R;
  float s = 0.f;
  for (int k = threadIdx.x; k < R; k += 256) s += vj[k] * vj[k];
  const float nrm = sqrtf(block_sum(s, red)) + 1e-30f;
  if (b == 0 && threadIdx.x == 0) M.norms[j] = nrm;
  const int c0 = j + 1 + b * kCPB;
  for (int c = c0; c < c0 + kCPB && c < M.C; c++) {
    float* __restrict__ vc = M.T + (int64_t)c * R;
    float d = 0.f;
    for (int k = threadIdx.x; k < R; k += 256) d += (vj[k] / nrm) * vc[k];
    const float dot = block_sum(d, red);
    for (int k = threadIdx.x; k < R; k += 256) vc[k] -= dot * (vj[k] / nrm);
  }
}

// w -= le * q + (0.01 lr) * w with q = T / norm (the final normalisation).
__global__ __launch_bounds__(256) void muon_update_kernel(const MuonMat* __restrict__ mats, int nmat) {
#pragma clang fp contract(off)
  const MuonMat& M = mats[blockIdx.y];
  const int64_t n = (int64_t)M.R * M.C;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    // element i of w ([r][c] row-major) -> vector j, position k
    int64_t j, k;
    if (M.transposed) { j = i / M.R; k = i % M.R; }
    else { k = i / M.C; j = i % M.C; }
    const float q = M.T[j * M.R + k] / M.norms[j];
    const float wi = M.w[i];
    M.w[i] = wi - (M.le * q + M.decay * wi);
  }
  (void)nmat;
}

}  // namespace

int launch_adamw(float* w, const float* g, float* m, float* v, int64_t n, float lr, float b1t, float b2t,
                 hipStream_t s) {
  if (n <= 0) return 0;
  hipLaunchKernelGGL(adamw_kernel, dim3((unsigned)ceil_div(n, 256)), dim3(256), 0, s, w, g, m, v, n, lr, b1t, b2t);
  NSH_LAUNCHED();
  return 0;
}

int muon_blocks(int C) { return (int)ceil_div(C, kCPB) > 0 ? (int)ceil_div(C, kCPB) : 1; }

int launch_muon_gather(const MuonMat* d_mats, int nmat, int64_t max_elems, hipStream_t s) {
  if (nmat <= 0) return 0;
  const unsigned gx = (unsigned)std::min<int64_t>(ceil_div(max_elems, 256), 2048);
  hipLaunchKernelGGL(muon_gather_kernel, dim3(gx, nmat), dim3(256), 0, s, d_mats, nmat);
  NSH_LAUNCHED();
  return 0;
}

int launch_mgs_steps(const MuonMat* d_mats, int nmat, int total_blocks, int max_c, hipStream_t s) {
  for (int j = 0; j < max_c; j++) {
    hipLaunchKernelGGL(mgs_step_kernel, dim3(total_blocks), dim3(256), 0, s, d_mats, nmat, j);
    NSH_LAUNCHED();
  }
  return 0;
}

int launch_muon_update(const MuonMat* d_mats, int nmat, int64_t max_elems, hipStream_t s) {
  if (nmat <= 0) return 0;
  const unsigned gx = (unsigned)std::min<int64_t>(ceil_div(max_elems, 256), 2048);
  hipLaunchKernelGGL(muon_update_kernel, dim3(gx, nmat), dim3(256), 0, s, d_mats, nmat);
  NSH_LAUNCHED();
  return 0;
}

}  // namespace nship
