// Row-wise and gather/scatter kernels (HBM-bound), wave64 throughout.
//
//   embedding gather        ns_embedding        codegen.cpp:1711-1718
//   LayerNorm forward       ns_layernorm        codegen.cpp:1280-1291
//   LayerNorm backward      ns_layernorm_grad   codegen.cpp:1346-1371
//   cross-entropy + seed    ns_cross_entropy / ns_loss_grad  codegen.cpp:1582-1613
//   activation backward     ns_act_grad         codegen.cpp:1340-1343
//   embedding weight grad   ns_embedding_grad_w codegen.cpp:1374-1383
//
// One wave owns one row: the row is loaded once into registers (float4,
// coalesced), reduced with xor-shuffles, and written once, so each kernel
// moves the algorithmic minimum of bytes.  The embedding gradient is
// deterministic and bit-exact: each output element sums its tokens in token
// order, as the reference's sequential scatter-add does -- in one launch
// through per-row token bitmaps in LDS up to 32768 tokens, beyond that
// through a stable counting sort of the tokens by row.
#include <algorithm>

#include "common.h"
#include "kernels.h"

namespace nship {

// Resolved embedding row of a float index, -1 if out of range.  Same
// predicate as C truncation followed by the reference's range check, but
// defined for NaN and huge values (which x86 turns into INT64_MIN).
__device__ __forceinline__ int64_t emb_row(float f, int64_t V) {
  if (!(f > -1.0f) || !(f < (float)V)) return -1;
  const int64_t k = (int64_t)f;
  return (k < 0 || k >= V) ? -1 : k;
}

// ---- embedding gather ----------------------------------------------------
// One wave per output row; D % 4 == 0 uses float4.
template <bool VEC>
__global__ __launch_bounds__(256) void embedding_kernel(const float* __restrict__ W, const float* __restrict__ idx,
                                                        float* __restrict__ out, int64_t n, int64_t V, int64_t D) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= n) return;
  int64_t k = emb_row(idx[row], V);
  if (k < 0) k = 0;
  const float* src = W + k * D;
  float* dst = out + row * D;
  if (VEC) {
    const float4* s4 = reinterpret_cast<const float4*>(src);
    float4* d4 = reinterpret_cast<float4*>(dst);
    for (int64_t j = lane; j < D / 4; j += 64) d4[j] = s4[j];
  } else {
    for (int64_t j = lane; j < D; j += 64) dst[j] = src[j];
  }
}

int launch_embedding(const float* W, const float* idx, float* out, int64_t n, int64_t V, int64_t D, hipStream_t s) {
  if (n <= 0) return 0;
  const dim3 grid((unsigned)ceil_div(n, 4));
  const bool vec = (D % 4 == 0) && ((uintptr_t)W % 16 == 0) && ((uintptr_t)out % 16 == 0);
  if (vec) hipLaunchKernelGGL(embedding_kernel<true>, grid, dim3(256), 0, s, W, idx, out, n, V, D);
  else hipLaunchKernelGGL(embedding_kernel<false>, grid, dim3(256), 0, s, W, idx, out, n, V, D);
  NSH_LAUNCHED();
  return 0;
}

// ---- LayerNorm forward -----------------------------------------------------
// Rows held in registers: NV float4 per lane covers up to 256*NV columns;
// each wave normalises RW rows, all of their loads issued before the first
// reduction (more bytes in flight per wave for short rows).
template <int NV, int RW>
__global__ __launch_bounds__(256) void layernorm_kernel(const float* __restrict__ x, float* __restrict__ y,
                                                        int64_t rows, int last) {
  const int lane = threadIdx.x & 63;
  const int64_t r0 = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * RW;
  if (r0 >= rows) return;
  float4 v[RW][NV];
  float sum[RW];
#pragma unroll
  for (int q = 0; q < RW; q++) {
    const float* xr = x + (r0 + q) * last;
    const bool ok = r0 + q < rows;
    sum[q] = 0.f;
#pragma unroll
    for (int i = 0; i < NV; i++) {
      const int c = (lane + 64 * i) * 4;
      v[q][i] = ok && c < last ? *reinterpret_cast<const float4*>(xr + c) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }
#pragma unroll
  for (int q = 0; q < RW; q++) {
#pragma unroll
    for (int i = 0; i < NV; i++) sum[q] += (v[q][i].x + v[q][i].y) + (v[q][i].z + v[q][i].w);
    sum[q] = wave_sum(sum[q]);
  }
#pragma unroll
  for (int q = 0; q < RW; q++) {
    if (r0 + q >= rows) break;
    const float mean = sum[q] / (float)last;
    float sq = 0.f;
#pragma unroll
    for (int i = 0; i < NV; i++) {
      const int c = (lane + 64 * i) * 4;
      if (c < last) {
        const float a = v[q][i].x - mean, b = v[q][i].y - mean, d = v[q][i].z - mean, e = v[q][i].w - mean;
        sq += (a * a + b * b) + (d * d + e * e);
      }
    }
    const float var = wave_sum(sq) / (float)last;
    const float inv = 1.f / sqrtf(var + 1e-5f);
    float* yr = y + (r0 + q) * last;
#pragma unroll
    for (int i = 0; i < NV; i++) {
      const int c = (lane + 64 * i) * 4;
      if (c < last)
        *reinterpret_cast<float4*>(yr + c) = make_float4((v[q][i].x - mean) * inv, (v[q][i].y - mean) * inv,
                                                         (v[q][i].z - mean) * inv, (v[q][i].w - mean) * inv);
    }
  }
}

// Any width: three streaming passes.
__global__ __launch_bounds__(256) void layernorm_any_kernel(const float* __restrict__ x, float* __restrict__ y,
                                                            int64_t rows, int last) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;
  const float* xr = x + r * last;
  float sum = 0.f;
  for (int c = lane; c < last; c += 64) sum += xr[c];
  const float mean = wave_sum(sum) / (float)last;
  float sq = 0.f;
  for (int c = lane; c < last; c += 64) { const float a = xr[c] - mean; sq += a * a; }
  const float inv = 1.f / sqrtf(wave_sum(sq) / (float)last + 1e-5f);
  float* yr = y + r * last;
  for (int c = lane; c < last; c += 64) yr[c] = (xr[c] - mean) * inv;
}

int launch_layernorm(const float* x, float* y, int64_t rows, int64_t last, hipStream_t s) {
  if (rows <= 0) return 0;
  const dim3 grid((unsigned)ceil_div(rows, 4)), block(256);
  const dim3 grid2((unsigned)ceil_div(rows, 8));
  const bool vec = last % 4 == 0 && (uintptr_t)x % 16 == 0 && (uintptr_t)y % 16 == 0;
  const int L = (int)last;
  if (vec && last <= 256) hipLaunchKernelGGL((layernorm_kernel<1, 2>), grid2, block, 0, s, x, y, rows, L);
  else if (vec && last <= 512) hipLaunchKernelGGL((layernorm_kernel<2, 2>), grid2, block, 0, s, x, y, rows, L);
  else if (vec && last <= 1024) hipLaunchKernelGGL((layernorm_kernel<4, 1>), grid, block, 0, s, x, y, rows, L);
  else if (vec && last <= 2048) hipLaunchKernelGGL((layernorm_kernel<8, 1>), grid, block, 0, s, x, y, rows, L);
  else hipLaunchKernelGGL(layernorm_any_kernel, grid, block, 0, s, x, y, rows, L);
  NSH_LAUNCHED();
  return 0;
}

// ---- LayerNorm backward ------------------------------------------------------
// dx = (d - mean(d) - (x - mean(x)) * mean((x - mean(x)) * d)) / sqrt(var + eps),
// exactly the reference's formula (its projection term has no 1/(var+eps)).
__global__ __launch_bounds__(256) void layernorm_grad_kernel(const float* __restrict__ dout,
                                                             const float* __restrict__ x,
                                                             float* __restrict__ dx, int64_t rows, int last) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;
  const float* xr = x + r * last;
  const float* dr = dout + r * last;
  float sx = 0.f, sd = 0.f;
  for (int c = lane; c < last; c += 64) { sx += xr[c]; sd += dr[c]; }
  const float mx = wave_sum(sx) / (float)last;
  const float md = wave_sum(sd) / (float)last;
  float sv = 0.f, sg = 0.f;
  for (int c = lane; c < last; c += 64) {
    const float a = xr[c] - mx;
    sv += a * a;
    sg += a * dr[c];
  }
  const float var = wave_sum(sv) / (float)last;
  const float gamma = wave_sum(sg) / (float)last;
  const float inv = 1.f / sqrtf(var + 1e-5f);
  float* o = dx + r * last;
  for (int c = lane; c < last; c += 64) o[c] = (dr[c] - md - (xr[c] - mx) * gamma) * inv;
}

// The same formula with both rows held in registers (NV float4 per lane,
// up to 256*NV columns): x and d are read once and dx written once.
template <int NV>
__global__ __launch_bounds__(256) void layernorm_grad_vec_kernel(const float* __restrict__ dout,
                                                                 const float* __restrict__ x,
                                                                 float* __restrict__ dx, int64_t rows, int last) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;
  const gfloat* xr = as_global(x + r * last);
  const gfloat* dr = as_global(dout + r * last);
  fvec4 xv[NV], dv[NV];
  float sx = 0.f, sd = 0.f;
#pragma unroll
  for (int i = 0; i < NV; i++) {
    const int c = (lane + 64 * i) * 4;
    const bool in = c < last;
    xv[i] = in ? *(const gfloat4*)(xr + c) : fvec4{0.f, 0.f, 0.f, 0.f};
    dv[i] = in ? *(const gfloat4*)(dr + c) : fvec4{0.f, 0.f, 0.f, 0.f};
    sx += (xv[i].x + xv[i].y) + (xv[i].z + xv[i].w);
    sd += (dv[i].x + dv[i].y) + (dv[i].z + dv[i].w);
  }
  const float mx = wave_sum(sx) / (float)last;
  const float md = wave_sum(sd) / (float)last;
  float sv = 0.f, sg = 0.f;
#pragma unroll
  for (int i = 0; i < NV; i++) {
    if ((lane + 64 * i) * 4 < last) {
      const fvec4 a = xv[i] - mx;
      sv += (a.x * a.x + a.y * a.y) + (a.z * a.z + a.w * a.w);
      sg += (a.x * dv[i].x + a.y * dv[i].y) + (a.z * dv[i].z + a.w * dv[i].w);
    }
  }
  const float var = wave_sum(sv) / (float)last;
  const float gamma = wave_sum(sg) / (float)last;
  const float inv = 1.f / sqrtf(var + 1e-5f);
  gfloat* o = as_global(dx + r * last);
#pragma unroll
  for (int i = 0; i < NV; i++) {
    const int c = (lane + 64 * i) * 4;
    if (c < last) *(gfloat4*)(o + c) = (dv[i] - md - (xv[i] - mx) * gamma) * inv;
  }
}

int launch_layernorm_grad(const float* dout, const float* x, float* dx, int64_t rows, int64_t last, hipStream_t s) {
  if (rows <= 0) return 0;
  const dim3 grid((unsigned)ceil_div(rows, 4)), block(256);
  const bool vec = last % 4 == 0 && ((uintptr_t)dout | (uintptr_t)x | (uintptr_t)dx) % 16 == 0;
  const int L = (int)last;
  if (vec && last <= 256) hipLaunchKernelGGL(layernorm_grad_vec_kernel<1>, grid, block, 0, s, dout, x, dx, rows, L);
  else if (vec && last <= 512) hipLaunchKernelGGL(layernorm_grad_vec_kernel<2>, grid, block, 0, s, dout, x, dx, rows, L);
  else if (vec && last <= 1024) hipLaunchKernelGGL(layernorm_grad_vec_kernel<4>, grid, block, 0, s, dout, x, dx, rows, L);
  else hipLaunchKernelGGL(layernorm_grad_kernel, grid, block, 0, s, dout, x, dx, rows, L);
  NSH_LAUNCHED();
  return 0;
}

// ---- softmax cross-entropy: loss terms and the gradient seed in one pass ----
// Per row: max, sum of exp, then for every column p = exp(x - max) / sum,
// grad = (p - y) / rows, and -log(p) summed over columns with y > 0 into
// row_loss[row].  Three passes over the row (max, sum of exp, outputs).
__global__ __launch_bounds__(256) void softmax_xent_kernel(const float* __restrict__ logits,
                                                           const float* __restrict__ labels,
                                                           float* __restrict__ grad, float* __restrict__ row_loss,
                                                           int64_t rows, int64_t C, int write_grad) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;
  const float* xr = logits + r * C;
  const float* yr = labels + r * C;
  float mx = -INFINITY;
  for (int64_t c = lane; c < C; c += 64) mx = fmaxf(mx, xr[c]);
  mx = wave_max(mx);
  float s = 0.f;
  for (int64_t c = lane; c < C; c += 64) s += expf(xr[c] - mx);
  s = wave_sum(s);
  const float inv_rows = 1.f / (float)rows;
  float loss = 0.f;
  float* gr = grad + r * C;
  for (int64_t c = lane; c < C; c += 64) {
    const float p = expf(xr[c] - mx) / s;
    const float y = yr[c];
    if (y > 0.f) loss -= logf(p);
    if (write_grad) gr[c] = (p - y) * inv_rows;
  }
  loss = wave_sum(loss);
  if (lane == 0) row_loss[r] = loss;
}

// Same, for rows of 16-byte aligned float4s (C % 4 == 0): pass 1 keeps a
// per-lane running max and rescaled sum of exp (online softmax) over float4
// loads, then combines the lanes; pass 2 re-reads the row (cache-resident)
// for p, the loss terms and the gradient.
__global__ __launch_bounds__(256) void softmax_xent_vec_kernel(const float* __restrict__ logits,
                                                               const float* __restrict__ labels,
                                                               float* __restrict__ grad, float* __restrict__ row_loss,
                                                               int64_t rows, int64_t C, int write_grad) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;
  const float4* xr = reinterpret_cast<const float4*>(logits + r * C);
  const float4* yr = reinterpret_cast<const float4*>(labels + r * C);
  const int64_t C4 = C / 4;
  float mx = -INFINITY, s = 0.f;
  for (int64_t c = lane; c < C4; c += 64) {
    const float4 x = xr[c];
    const float m4 = fmaxf(fmaxf(x.x, x.y), fmaxf(x.z, x.w));
    if (m4 > mx) {
      s *= expf(mx - m4);  // exp(-inf) = 0 on the first block
      mx = m4;
    }
    s += (expf(x.x - mx) + expf(x.y - mx)) + (expf(x.z - mx) + expf(x.w - mx));
  }
  const float gmx = wave_max(mx);
  s = wave_sum(mx == -INFINITY ? 0.f : s * expf(mx - gmx));
  const float inv_rows = 1.f / (float)rows;
  float loss = 0.f;
  float4* gr = reinterpret_cast<float4*>(grad + r * C);
  for (int64_t c = lane; c < C4; c += 64) {
    const float4 x = xr[c], y = yr[c];
    const float p0 = expf(x.x - gmx) / s, p1 = expf(x.y - gmx) / s;
    const float p2 = expf(x.z - gmx) / s, p3 = expf(x.w - gmx) / s;
    if (y.x > 0.f) loss -= logf(p0);
    if (y.y > 0.f) loss -= logf(p1);
    if (y.z > 0.f) loss -= logf(p2);
    if (y.w > 0.f) loss -= logf(p3);
    if (write_grad)
      gr[c] = make_float4((p0 - y.x) * inv_rows, (p1 - y.y) * inv_rows, (p2 - y.z) * inv_rows, (p3 - y.w) * inv_rows);
  }
  loss = wave_sum(loss);
  if (lane == 0) row_loss[r] = loss;
}

// One workgroup (256 threads) per row of up to 1024 * NV4 floats, the row
// held in registers (NV4 float4 per thread): logits and labels are read
// once.  Same per-element operations as the reference (max, expf(x - max),
// sum, divide, -logf(p) where y > 0, (p - y) / rows); sums over a fixed tree.
// Logits, labels and the gradient stream through non-temporal loads and
// stores (each byte is touched once): c5's 1.6 GB per step at 5.7 TB/s
// instead of 4.8.
template <int NV4>
__global__ __launch_bounds__(256) void softmax_xent_row_kernel(const float* __restrict__ logits,
                                                               const float* __restrict__ labels,
                                                               float* __restrict__ grad, float* __restrict__ row_loss,
                                                               int64_t rows, int64_t C, int write_grad) {
  __shared__ float red[3][4];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int64_t r = blockIdx.x;
  const int64_t C4 = C / 4;
  const gfloat4* xr = reinterpret_cast<const gfloat4*>(as_global(logits + r * C));
  const gfloat4* yr = reinterpret_cast<const gfloat4*>(as_global(labels + r * C));
  fvec4 x[NV4], y[NV4];
  float mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < NV4; i++) {
    const int64_t c = t + 256 * i;
    const bool in = c < C4;
    x[i] = in ? __builtin_nontemporal_load(xr + c) : fvec4{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
    y[i] = in ? __builtin_nontemporal_load(yr + c) : fvec4{0.f, 0.f, 0.f, 0.f};
    mx = fmaxf(mx, fmaxf(fmaxf(x[i].x, x[i].y), fmaxf(x[i].z, x[i].w)));
  }
  mx = wave_max(mx);
  if (lane == 0) red[0][w] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0][0], red[0][1]), fmaxf(red[0][2], red[0][3]));
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < NV4; i++) {
    x[i] = fvec4{expf(x[i].x - mx), expf(x[i].y - mx), expf(x[i].z - mx), expf(x[i].w - mx)};
    s += (x[i].x + x[i].y) + (x[i].z + x[i].w);
  }
  s = wave_sum(s);
  if (lane == 0) red[1][w] = s;
  __syncthreads();
  s = (red[1][0] + red[1][1]) + (red[1][2] + red[1][3]);
  const float inv_rows = 1.f / (float)rows;
  gfloat4* gr = reinterpret_cast<gfloat4*>(as_global(grad + r * C));
  float loss = 0.f;
#pragma unroll
  for (int i = 0; i < NV4; i++) {
    const int64_t c = t + 256 * i;
    const float p0 = x[i].x / s, p1 = x[i].y / s, p2 = x[i].z / s, p3 = x[i].w / s;
    if (y[i].x > 0.f) loss -= logf(p0);
    if (y[i].y > 0.f) loss -= logf(p1);
    if (y[i].z > 0.f) loss -= logf(p2);
    if (y[i].w > 0.f) loss -= logf(p3);
    if (write_grad && c < C4) {
      const fvec4 gv{(p0 - y[i].x) * inv_rows, (p1 - y[i].y) * inv_rows, (p2 - y[i].z) * inv_rows,
                     (p3 - y[i].w) * inv_rows};
      __builtin_nontemporal_store(gv, gr + c);
    }
  }
  loss = wave_sum(loss);
  if (lane == 0) red[2][w] = loss;
  __syncthreads();
  if (t == 0) row_loss[r] = (red[2][0] + red[2][1]) + (red[2][2] + red[2][3]);
}

// Deterministic single-workgroup sum of row losses / rows: 1024 threads,
// each summing 4 consecutive losses per step (float4 where the buffer is
// 16-byte aligned), then a fixed tree over the 16 waves.
__global__ __launch_bounds__(1024) void mean_loss_kernel(const float* __restrict__ row_loss, int64_t rows,
                                                         float* __restrict__ out) {
  __shared__ float part[16];
  const gfloat* rl = as_global(row_loss);
  const int64_t n4 = ((uintptr_t)row_loss % 16 == 0) ? rows / 4 : 0;
  float s = 0.f;
  for (int64_t i = threadIdx.x; i < n4; i += 1024) {
    const fvec4 v = ((const gfloat4*)rl)[i];
    s += (v.x + v.y) + (v.z + v.w);
  }
  for (int64_t i = 4 * n4 + threadIdx.x; i < rows; i += 1024) s += rl[i];
  s = wave_sum(s);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) {
    float t[8];
#pragma unroll
    for (int k = 0; k < 8; k++) t[k] = part[2 * k] + part[2 * k + 1];
    out[0] = (((t[0] + t[1]) + (t[2] + t[3])) + ((t[4] + t[5]) + (t[6] + t[7]))) / (float)rows;
  }
}

int launch_softmax_xent(const float* logits, const float* labels, float* grad, float* row_loss, float* loss,
                        int64_t rows, int64_t C, bool write_grad, hipStream_t s) {
  // no whole row: the reference's mean is 0.f / 0 (codegen.cpp:1612), a NaN
  if (rows <= 0) return loss ? launch_fill(loss, 1, __builtin_nanf(""), s) : 0;
  const bool vec = C % 4 == 0 && ((uintptr_t)logits | (uintptr_t)labels | (uintptr_t)grad) % 16 == 0;
  const int64_t nv4 = ceil_div(C / 4, 256);
  if (vec && C >= 2048 && nv4 <= 8) {
    const dim3 g((unsigned)rows);
#define NSH_XENT(N_)                                                                                        \
  hipLaunchKernelGGL(softmax_xent_row_kernel<N_>, g, dim3(256), 0, s, logits, labels, grad, row_loss, rows, C, \
                     write_grad ? 1 : 0)
    if (nv4 <= 2) NSH_XENT(2);
    else if (nv4 <= 4) NSH_XENT(4);
    else NSH_XENT(8);
#undef NSH_XENT
  } else if (vec)
    hipLaunchKernelGGL(softmax_xent_vec_kernel, dim3((unsigned)ceil_div(rows, 4)), dim3(256), 0, s, logits, labels,
                       grad, row_loss, rows, C, write_grad ? 1 : 0);
  else
    hipLaunchKernelGGL(softmax_xent_kernel, dim3((unsigned)ceil_div(rows, 4)), dim3(256), 0, s, logits, labels, grad,
                       row_loss, rows, C, write_grad ? 1 : 0);
  NSH_LAUNCHED();
  hipLaunchKernelGGL(mean_loss_kernel, dim3(1), dim3(1024), 0, s, row_loss, rows, loss);
  NSH_LAUNCHED();
  return 0;
}

// ---- activation backward (elementwise) ------------------------------------------
__global__ void act_grad_kernel(const float* __restrict__ din, const float* __restrict__ pre,
                                float* __restrict__ dout, int64_t n, int code) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) dout[i] = din[i] * act_deriv(pre[i], code);
}

int launch_act_grad(const float* din, const float* pre, float* dout, int64_t n, int code, hipStream_t s) {
  if (n <= 0) return 0;
  hipLaunchKernelGGL(act_grad_kernel, dim3((unsigned)ceil_div(n, 256)), dim3(256), 0, s, din, pre, dout, n, code);
  NSH_LAUNCHED();
  return 0;
}

// ---- embedding weight gradient --------------------------------------------------
// Stable counting sort of tokens by row (counts, exclusive scan, in-order
// placement), then one wave per vocabulary row sums its tokens' gradient
// rows in token order and writes the dW row once (zero rows included).
__global__ __launch_bounds__(256) void emb_count_kernel(const float* __restrict__ idx, int64_t n, int64_t V,
                                                        int* __restrict__ count) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const int64_t r = emb_row(idx[i], V);
  if (r >= 0) atomicAdd(&count[r], 1);
}

// Exclusive scan of V counts by one workgroup (V up to a few million).
__global__ __launch_bounds__(1024) void exclusive_scan_kernel(const int* __restrict__ in, int* __restrict__ out,
                                                              int64_t n) {
  __shared__ int part[1024];
  const int t = threadIdx.x;
  const int64_t per = (n + 1023) / 1024;
  const int64_t b = t * per, e = b + per < n ? b + per : n;
  int s = 0;
  if (per <= 8) {
    // all of the chunk's loads in flight at once (n <= 8192)
    int v[8];
#pragma unroll
    for (int k = 0; k < 8; k++) v[k] = b + k < e ? in[b + k] : 0;
#pragma unroll
    for (int k = 0; k < 8; k++) s += v[k];
  } else {
    for (int64_t i = b; i < e; i++) s += in[i];
  }
  part[t] = s;
  __syncthreads();
  for (int o = 1; o < 1024; o <<= 1) {
    const int v = t >= o ? part[t - o] : 0;
    __syncthreads();
    part[t] += v;
    __syncthreads();
  }
  int run = part[t] - s;
  for (int64_t i = b; i < e; i++) {
    const int c = in[i];
    out[i] = run;
    run += c;
  }
  if (t == 1023) out[n] = part[1023];
}

// Placement: each token takes a slot of its row's segment through an atomic
// cursor (arbitrary order); sorting every segment by token id then restores
// token order, which is the stable order the reference's loop accumulates in.
__global__ __launch_bounds__(256) void emb_place_kernel(const float* __restrict__ idx, int64_t n, int64_t V,
                                                        const int* __restrict__ start, int* __restrict__ cursor,
                                                        int* __restrict__ order) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const int64_t r = emb_row(idx[i], V);
  if (r < 0) return;
  const int pos = atomicAdd(&cursor[r], 1);
  order[start[r] + pos] = (int)i;
}

// Sort the segments of rows [256*block, 256*block + 256).  The block's
// segment bounds are staged in LDS once.  Short segments (<= 32 tokens) are
// insertion-sorted by their own thread; each longer one is listed and then
// ranked by the whole workgroup (rank = number of smaller token ids in the
// segment, ids are distinct) through `tmp`.
__global__ __launch_bounds__(256) void emb_sort_segments_kernel(const int* __restrict__ start, int64_t V,
                                                                int* __restrict__ order, int* __restrict__ tmp) {
  __shared__ int st[257];
  __shared__ int longrow[256];
  __shared__ int nlong;
  const int t = threadIdx.x;
  const int64_t r0 = (int64_t)blockIdx.x * 256;
  const int nr = (int)(r0 + 256 < V ? 256 : V - r0);
  if (t == 0) nlong = 0;
  for (int i = t; i <= nr; i += 256) st[i] = start[r0 + i];
  __syncthreads();
  if (t < nr) {
    const int b = st[t], e = st[t + 1];
    if (e - b <= 32) {
      for (int i = b + 1; i < e; i++) {
        const int v = order[i];
        int j = i - 1;
        while (j >= b && order[j] > v) {
          order[j + 1] = order[j];
          j--;
        }
        order[j + 1] = v;
      }
    } else {
      longrow[atomicAdd(&nlong, 1)] = t;  // segments are disjoint: any listing order
    }
  }
  __syncthreads();
  const int nl = nlong;
  for (int k = 0; k < nl; k++) {
    const int b = st[longrow[k]], e = st[longrow[k] + 1];
    for (int i = b + t; i < e; i += 256) {
      const int v = order[i];
      int rank = 0;
      for (int j = b; j < e; j++) rank += order[j] < v;
      tmp[b + rank] = v;
    }
    __syncthreads();
    for (int i = b + t; i < e; i += 256) order[i] = tmp[i];
    __syncthreads();
  }
}

// dW[r,:] = sum over the row's tokens (ascending) of dout[token,:].
__global__ __launch_bounds__(256) void emb_grad_rows_kernel(const float* __restrict__ dout,
                                                            const int* __restrict__ start,
                                                            const int* __restrict__ order, float* __restrict__ dW,
                                                            int64_t V, int64_t D) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= V) return;
  const int b = start[r], e = start[r + 1];
  float* o = dW + r * D;
  for (int64_t c = lane; c < D; c += 64) {
    float acc = 0.f;
    for (int t = b; t < e; t++) acc += dout[(int64_t)order[t] * D + c];
    o[c] = acc;
  }
}

// The same sums for D % 4 == 0 on 16-byte aligned rows: NV float4 columns
// per lane (256 NV columns per pass), the next token's rows loaded before
// the current one is added, each column still summed in ascending token
// order.
template <int NV>
__global__ __launch_bounds__(256) void emb_grad_rows_vec_kernel(const float* __restrict__ dout,
                                                                const int* __restrict__ start,
                                                                const int* __restrict__ order,
                                                                float* __restrict__ dW, int64_t V, int64_t D) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= V) return;
  const int b = start[r], e = start[r + 1];
  const int64_t D4 = D / 4;
  const float4* __restrict__ src = reinterpret_cast<const float4*>(dout);
  float4* __restrict__ o = reinterpret_cast<float4*>(dW + r * D);
  for (int64_t c0 = lane; c0 < D4; c0 += 64 * NV) {
    float4 acc[NV], x[NV];
#pragma unroll
    for (int j = 0; j < NV; j++) acc[j] = x[j] = make_float4(0.f, 0.f, 0.f, 0.f);
    int64_t row = b < e ? (int64_t)order[b] * D4 : 0;
#pragma unroll
    for (int j = 0; j < NV; j++)
      if (b < e && c0 + 64 * j < D4) x[j] = src[row + c0 + 64 * j];
    for (int t = b; t < e; t++) {
      float4 cur[NV];
#pragma unroll
      for (int j = 0; j < NV; j++) cur[j] = x[j];
      if (t + 1 < e) {
        row = (int64_t)order[t + 1] * D4;
#pragma unroll
        for (int j = 0; j < NV; j++)
          if (c0 + 64 * j < D4) x[j] = src[row + c0 + 64 * j];
      }
#pragma unroll
      for (int j = 0; j < NV; j++) {
        acc[j].x += cur[j].x; acc[j].y += cur[j].y; acc[j].z += cur[j].z; acc[j].w += cur[j].w;
      }
    }
#pragma unroll
    for (int j = 0; j < NV; j++)
      if (c0 + 64 * j < D4) o[c0 + 64 * j] = acc[j];
  }
}

// ---- embedding weight gradient in one launch (no sort, no workspace) --------
// G = 2^lg workgroups; workgroup b owns the vocabulary rows b, b + G, b + 2G,
// ... (16 * RPW of them; strided, so that the frequent ids, which cluster at
// the low ids of a vocabulary, land on different CUs).  It reads every token
// id once (the ids are shared by all workgroups, so they come from L2) and
// marks the tokens that hit its rows in one LDS bitmap per row, bit t =
// token t, counting each row's tokens.  Walking a row's bitmap word by word
// and bit by bit visits its tokens in ascending order, so each output
// element is the reference's sequential sum with no sort at all.  Each wave
// owns RPW rows: it gathers a row's tokens' gradient rows (kEmbAhead loads in
// flight) and adds them in token order, then writes the dW row once (zeros
// if no token).  Two rows per wave halve the workgroups that each scan all
// ids (c5's 16384 ids over 8192 rows: 18.3 -> 15.2 us); they are used when
// the grid still holds a workgroup per CU.
constexpr int kEmbWaves = 16;  // 16 waves of 64 lanes
// LDS budget of the bitmaps: 16 * RPW * ceil(n/32) words (128 KB at RPW 2).
constexpr int64_t kEmbFusedMaxTokens = 32768;
// A float4 row hit by more than kEmbHeavy tokens is summed by the whole
// workgroup instead: one wave's chain of gathers would hold the launch (a
// Zipf-distributed batch put ~2900 of 16384 ids on row 0: 1.6 ms).  Its
// tokens are listed in order in LDS, kEmbList at a time.
constexpr int kEmbHeavy = 64;
constexpr int kEmbList = 2048;
// LDS words of the fused kernel: bitmaps, per-row token counts, token list,
// per-wave sums.
static size_t emb_fused_lds_words(int64_t n, int rows) {
  return (size_t)rows * (size_t)((n + 31) >> 5) + (size_t)rows + (size_t)kEmbList + kEmbWaves;
}

// Value of lane (lane + S) of the same 16-lane row (lane + S stays in the
// row for the lanes that use the result).
template <int S>
__device__ __forceinline__ float row_shl(float v) {
  if constexpr (S == 0) return v;
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x100 + S, 0xF, 0xF, false));
}

// Inclusive prefix sum over the 64 lanes of a wave.
__device__ __forceinline__ int wave_prefix_sum(int v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int u = __shfl_up(v, d, 64);
    if (lane >= d) v += u;
  }
  return v;
}

template <bool VEC, int NV, int kEmbAhead, bool VEC_IDX, int RPW>
__global__ __launch_bounds__(1024) void emb_grad_fused_kernel(const float* __restrict__ dout,
                                                              const float* __restrict__ idx,
                                                              float* __restrict__ dW, int64_t n, int64_t V,
                                                              int64_t D, int lg) {
  constexpr int kRows = kEmbWaves * RPW;
  extern __shared__ unsigned emb_bits[];
  const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
  const int nw = (int)((n + 31) >> 5);
  const int b = blockIdx.x, gmask = (1 << lg) - 1;
  int* const row_cnt = reinterpret_cast<int*>(emb_bits + kRows * nw);  // tokens per local row
  int* const tok_list = row_cnt + kRows;                                 // kEmbList ints
  int* const wsum = tok_list + kEmbList;                                 // kEmbWaves ints
  // the first batch of ids is in flight while the bitmaps are cleared
  const float4* __restrict__ idx4 = reinterpret_cast<const float4*>(idx);
  const int64_t n4 = n >> 2;
  float4 f0[4];
  if (VEC_IDX) {
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const int64_t j = (int64_t)k * 1024 + t;
      f0[k] = j < n4 ? idx4[j] : make_float4(-1.f, -1.f, -1.f, -1.f);
    }
  }
  for (int i = t; i < kRows * nw + kRows; i += 1024) emb_bits[i] = 0u;
  __syncthreads();
  // A token hits row (int)id when -1 < id < V (exact in float: V <= 2^24;
  // ids in (-1, 0) truncate to row 0; NaN fails both tests).  Row g is local
  // row g >> lg of workgroup g & (G - 1).
  const float vhi = (float)V;
  auto mark = [&](float f, int64_t i) {
    if (f > -1.0f && f < vhi) {
      const int g = (int)f;
      if ((g & gmask) == b) {
        const int row = g >> lg;
        atomicOr(&emb_bits[row * nw + (int)(i >> 5)], 1u << (i & 31));
        atomicAdd(&row_cnt[row], 1);
      }
    }
  };
  if (VEC_IDX) {  // float4 of ids, 4 per thread in flight, then the n % 4 tail
    for (int64_t base = 0; base < n4; base += 4 * 1024) {
      float4 f[4];
#pragma unroll
      for (int k = 0; k < 4; k++) {
        const int64_t j = base + k * 1024 + t;
        f[k] = base == 0 ? f0[k] : j < n4 ? idx4[j] : make_float4(-1.f, -1.f, -1.f, -1.f);
      }
#pragma unroll
      for (int k = 0; k < 4; k++) {
        const int64_t i = 4 * (base + k * 1024 + t);
        mark(f[k].x, i); mark(f[k].y, i + 1); mark(f[k].z, i + 2); mark(f[k].w, i + 3);
      }
    }
    if (t < (int)(n & 3)) mark(idx[4 * n4 + t], 4 * n4 + t);
  } else {  // batches of 8 per thread, all 8 loads issued before any is used
    for (int64_t base = 0; base < n; base += 8 * 1024) {
      float f[8];
#pragma unroll
      for (int k = 0; k < 8; k++) {
        const int64_t i = base + k * 1024 + t;
        f[k] = i < n ? idx[i] : -1.0f;
      }
#pragma unroll
      for (int k = 0; k < 8; k++) mark(f[k], base + k * 1024 + t);
    }
  }
  __syncthreads();
  // Local rows the whole workgroup sums (float4 rows only): one bit each,
  // the same mask in every wave.
  const uint64_t heavy = VEC ? __ballot(lane < kRows && row_cnt[lane] > kEmbHeavy) : 0ull;
  // Columns per pass: 64 lanes x NV float4 (VEC) or 64 lanes x NV floats.
  constexpr int W = VEC ? 4 : 1;
  const int64_t DW = D / W;
  for (int rr = 0; rr < RPW; rr++) {
    const int j = wv + kEmbWaves * rr;
    const int64_t r = b + ((int64_t)j << lg);
    if (r >= V) break;
    if ((heavy >> j) & 1) continue;  // the workgroup's, below
    const unsigned* __restrict__ bits = emb_bits + j * nw;
    // The pass loop is wave-uniform (every lane takes part in the ballots and
    // lane reads below); lanes past the row's end only skip their loads/stores.
    for (int64_t cb = 0; cb < DW; cb += 64 * NV) {
      const int64_t c0 = cb + lane;
      float acc[NV][W];
      float buf[kEmbAhead][NV][W];
#pragma unroll
      for (int jj = 0; jj < NV; jj++)
#pragma unroll
        for (int k = 0; k < W; k++) acc[jj][k] = 0.f;
      int pend = 0;  // loads in flight, oldest in slot (head % kEmbAhead)
      int head = 0;
      auto add_oldest = [&]() {
        const int sl = head % kEmbAhead;
#pragma unroll
        for (int q = 0; q < kEmbAhead; q++)
          if (q == sl)
#pragma unroll
            for (int jj = 0; jj < NV; jj++)
#pragma unroll
              for (int k = 0; k < W; k++) acc[jj][k] += buf[q][jj][k];
        head++;
        pend--;
      };
      for (int w0 = 0; w0 < nw; w0 += 64) {
        const unsigned word = w0 + lane < nw ? bits[w0 + lane] : 0u;
        uint64_t nz = __ballot(word != 0u);
        while (nz) {
          const int l = __builtin_ctzll(nz);
          nz &= nz - 1;
          unsigned wd = (unsigned)__builtin_amdgcn_readlane((int)word, l);
          while (wd) {
            const int bt = __builtin_ctz(wd);
            wd &= wd - 1;
            const int64_t tok = (int64_t)(w0 + l) * 32 + bt;
            if (pend == kEmbAhead) add_oldest();
            const int sl = (head + pend) % kEmbAhead;
            const float* src = dout + tok * D;
#pragma unroll
            for (int q = 0; q < kEmbAhead; q++)
              if (q == sl)
#pragma unroll
                for (int jj = 0; jj < NV; jj++) {
                  const int64_t c = c0 + 64 * jj;
                  if (c < DW) {
                    if constexpr (VEC) {
                      const float4 v = reinterpret_cast<const float4*>(src)[c];
                      buf[q][jj][0] = v.x; buf[q][jj][1] = v.y; buf[q][jj][2] = v.z; buf[q][jj][3] = v.w;
                    } else {
                      buf[q][jj][0] = src[c];
                    }
                  } else {
#pragma unroll
                    for (int k = 0; k < W; k++) buf[q][jj][k] = 0.f;
                  }
                }
            pend++;
          }
        }
      }
      while (pend > 0) add_oldest();
      float* o = dW + r * D;
#pragma unroll
      for (int jj = 0; jj < NV; jj++) {
        const int64_t c = c0 + 64 * jj;
        if (c < DW) {
          if constexpr (VEC)
            reinterpret_cast<float4*>(o)[c] = make_float4(acc[jj][0], acc[jj][1], acc[jj][2], acc[jj][3]);
          else
            o[c] = acc[jj][0];
        }
      }
    }
  }
  if constexpr (VEC) {
    // Heavy rows, one after another, by all 16 waves.  Thread t holds bitmap
    // word t (n <= 32768 tokens: at most 1024 words) and the rank of its first
    // token; segments of kEmbList tokens are listed in order in LDS.  Wave w
    // takes column groups g = w, w + 16, ... of 8 float4; lane = 8 c + s loads
    // column 8 g + c of the token in slot s of a round of 8 consecutive tokens
    // (8 tokens x 128 B per load instruction), and the lanes with s = 0 add
    // the 8 slots in order (row_shl by s within the 16-lane row), so each
    // element is still the sequential sum in token order.  Rounds go 8 at a
    // time with the next 8 rounds' loads in flight.
    const int c = lane >> 3, sl = lane & 7;
    const int64_t G = (DW + 7) / 8;
    uint64_t hm = heavy;
    while (hm) {
      const int j = __builtin_ctzll(hm);
      hm &= hm - 1;
      const int64_t r = b + ((int64_t)j << lg);
      const int total = row_cnt[j];
      const unsigned word = t < nw ? emb_bits[j * nw + t] : 0u;
      const int pc = __popc(word);
      const int incl = wave_prefix_sum(pc);
      __syncthreads();  // wsum of the previous heavy row has been read
      if (lane == 63) wsum[wv] = incl;
      __syncthreads();
      int first = incl - pc;
      for (int u = 0; u < wv; u++) first += wsum[u];
      for (int64_t g0 = 0; g0 < G; g0 += kEmbWaves) {
        const int64_t col = (g0 + wv) * 8 + c;  // this lane's float4 column
        const bool cin = g0 + wv < G && col < DW;
        float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int seg = 0; seg < total; seg += kEmbList) {
          __syncthreads();  // the previous segment's list has been read
          if (word && first < seg + kEmbList && first + pc > seg) {
            int rk = first;
            for (unsigned wd = word; wd; wd &= wd - 1, rk++)
              if (rk >= seg && rk < seg + kEmbList) tok_list[rk - seg] = t * 32 + __builtin_ctz(wd);
          }
          __syncthreads();
          const int cnt = min(kEmbList, total - seg);
          const int nr = (cnt + 7) / 8;
          auto load_round = [&](int rd) {
            const int k = rd * 8 + sl;
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (cin && rd < nr && k < cnt) v = reinterpret_cast<const float4*>(dout + (int64_t)tok_list[k] * D)[col];
            return v;
          };
          float4 cur[8], nxt[8];
#pragma unroll
          for (int u = 0; u < 8; u++) cur[u] = load_round(u);
          for (int bt = 0; bt < nr; bt += 8) {
#pragma unroll
            for (int u = 0; u < 8; u++) nxt[u] = load_round(bt + 8 + u);
#pragma unroll
            for (int u = 0; u < 8; u++) {
              const int base = (bt + u) * 8;  // the round's first token
              const float4 v = cur[u];
#define NSH_ADD_SLOT(S)       \
  if (base + S < cnt) {       \
    acc.x += row_shl<S>(v.x); \
    acc.y += row_shl<S>(v.y); \
    acc.z += row_shl<S>(v.z); \
    acc.w += row_shl<S>(v.w); \
  }
              NSH_ADD_SLOT(0)
              NSH_ADD_SLOT(1)
              NSH_ADD_SLOT(2)
              NSH_ADD_SLOT(3)
              NSH_ADD_SLOT(4)
              NSH_ADD_SLOT(5)
              NSH_ADD_SLOT(6)
              NSH_ADD_SLOT(7)
#undef NSH_ADD_SLOT
            }
#pragma unroll
            for (int u = 0; u < 8; u++) cur[u] = nxt[u];
          }
        }
        if (cin && sl == 0) reinterpret_cast<float4*>(dW + r * D)[col] = acc;
      }
    }
  }
}

// Clears n ints.  A kernel rather than hipMemsetAsync, so that a caller may
// capture the launch sequence in a HIP graph (memset nodes are avoided).
__global__ __launch_bounds__(256) void fill_zero_ints_kernel(int* __restrict__ p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) p[i] = 0;
}

// Workspace: ints [V] count, [V+1] start, [V] cursor, [n] order, [n] tmp.
size_t embedding_grad_workspace(int64_t n, int64_t V) { return (size_t)(3 * V + 1 + 2 * n); }

// Rows per wave: 2 while that still leaves a workgroup for each of the 256
// CUs, else 1.  Workgroups: the power of two G >= ceil(V / rows per group).
static int emb_grad_rows_per_wave(int64_t V) { return ceil_div(V, 2 * kEmbWaves) >= 256 ? 2 : 1; }
static int emb_grad_lg(int64_t V) {
  const int64_t need = ceil_div(V, (int64_t)kEmbWaves * emb_grad_rows_per_wave(V));
  int lg = 0;
  while (((int64_t)1 << lg) < need) lg++;
  return lg;
}

// One launch without workspace when the bitmaps fit in LDS, the
// workgroups' shared reads of the ids stay small (n ids per workgroup) and
// row numbers are exact in float (V <= 2^24).
static bool emb_grad_fused_fits(int64_t n, int64_t V) {
  return n <= kEmbFusedMaxTokens && V <= ((int64_t)1 << 24) && (n << emb_grad_lg(V)) <= ((int64_t)1 << 26);
}

template <bool VEC, bool VEC_IDX, int RPW>
static void launch_emb_grad_fused_rpw(const float* dout, const float* idx, float* dW, int64_t n, int64_t V, int64_t D,
                                      hipStream_t s) {
  const int lg = emb_grad_lg(V);
  const dim3 g(1u << lg);
  const size_t lds = emb_fused_lds_words(n, kEmbWaves * RPW) * sizeof(unsigned);
  const int64_t DW = VEC ? D / 4 : D;
  // NV columns per lane per pass, AH rows in flight: NV * AH float4 of loads.
  // At c5's D = 512 (128 float4) one row in flight is the fastest: 12.5 us
  // per launch against 13.0 with 2, 13.4 with 3 and 14.5 with 4 (rows of
  // ~2 tokens leave little to overlap and each further slot adds selects).
  if (DW > 128)
    hipLaunchKernelGGL((emb_grad_fused_kernel<VEC, 4, 2, VEC_IDX, RPW>), g, dim3(1024), lds, s, dout, idx, dW, n, V, D,
                       lg);
  else if (DW > 64)
    hipLaunchKernelGGL((emb_grad_fused_kernel<VEC, 2, 1, VEC_IDX, RPW>), g, dim3(1024), lds, s, dout, idx, dW, n, V, D,
                       lg);
  else
    hipLaunchKernelGGL((emb_grad_fused_kernel<VEC, 1, 4, VEC_IDX, RPW>), g, dim3(1024), lds, s, dout, idx, dW, n, V, D,
                       lg);
}

template <bool VEC, bool VEC_IDX>
static void launch_emb_grad_fused(const float* dout, const float* idx, float* dW, int64_t n, int64_t V, int64_t D,
                                  hipStream_t s) {
  if (emb_grad_rows_per_wave(V) == 2)
    launch_emb_grad_fused_rpw<VEC, VEC_IDX, 2>(dout, idx, dW, n, V, D, s);
  else
    launch_emb_grad_fused_rpw<VEC, VEC_IDX, 1>(dout, idx, dW, n, V, D, s);
}

template <bool VEC>
static void launch_emb_grad_fused_ids(const float* dout, const float* idx, float* dW, int64_t n, int64_t V, int64_t D,
                                      hipStream_t s) {
  if ((uintptr_t)idx % 16 == 0)
    launch_emb_grad_fused<VEC, true>(dout, idx, dW, n, V, D, s);
  else
    launch_emb_grad_fused<VEC, false>(dout, idx, dW, n, V, D, s);
}

int launch_embedding_grad(const float* dout, const float* idx, float* dW, int64_t n, int64_t V, int64_t D, int* ws,
                          hipStream_t s) {
  if (V <= 0 || D <= 0) return 0;  // dW is empty
  if (emb_grad_fused_fits(n, V)) {
    if (D % 4 == 0 && ((uintptr_t)dout | (uintptr_t)dW) % 16 == 0)
      launch_emb_grad_fused_ids<true>(dout, idx, dW, n, V, D, s);
    else
      launch_emb_grad_fused_ids<false>(dout, idx, dW, n, V, D, s);
    NSH_LAUNCHED();
    return 0;
  }
  int* count = ws;
  int* start = ws + V;
  int* cursor = ws + 2 * V + 1;
  int* order = ws + 3 * V + 1;
  int* tmp = order + n;
  // count [0, V) and cursor [2V+1, 3V+1) start at zero; start in between is
  // written whole by the scan, so one fill covers [0, 3V+1)
  {
    const int64_t nz = 3 * V + 1;
    hipLaunchKernelGGL(fill_zero_ints_kernel, dim3((unsigned)std::min<int64_t>(ceil_div(nz, 256), 1024)), dim3(256), 0,
                       s, ws, nz);
    NSH_LAUNCHED();
  }
  if (n > 0) {
    hipLaunchKernelGGL(emb_count_kernel, dim3((unsigned)ceil_div(n, 256)), dim3(256), 0, s, idx, n, V, count);
    NSH_LAUNCHED();
  }
  hipLaunchKernelGGL(exclusive_scan_kernel, dim3(1), dim3(1024), 0, s, count, start, V);
  NSH_LAUNCHED();
  if (n > 0) {
    hipLaunchKernelGGL(emb_place_kernel, dim3((unsigned)ceil_div(n, 256)), dim3(256), 0, s, idx, n, V, start, cursor,
                       order);
    NSH_LAUNCHED();
    hipLaunchKernelGGL(emb_sort_segments_kernel, dim3((unsigned)ceil_div(V, 256)), dim3(256), 0, s, start, V, order,
                       tmp);
    NSH_LAUNCHED();
  }
  const dim3 rg((unsigned)ceil_div(V, 4));
  if (D % 4 == 0 && ((uintptr_t)dout | (uintptr_t)dW) % 16 == 0) {
    const int64_t D4 = D / 4;
    if (D4 >= 256)
      hipLaunchKernelGGL(emb_grad_rows_vec_kernel<4>, rg, dim3(256), 0, s, dout, start, order, dW, V, D);
    else if (D4 >= 128)
      hipLaunchKernelGGL(emb_grad_rows_vec_kernel<2>, rg, dim3(256), 0, s, dout, start, order, dW, V, D);
    else
      hipLaunchKernelGGL(emb_grad_rows_vec_kernel<1>, rg, dim3(256), 0, s, dout, start, order, dW, V, D);
  } else {
    hipLaunchKernelGGL(emb_grad_rows_kernel, rg, dim3(256), 0, s, dout, start, order, dW, V, D);
  }
  NSH_LAUNCHED();
  return 0;
}

}  // namespace nship
