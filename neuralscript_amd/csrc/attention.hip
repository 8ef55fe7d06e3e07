// Multi-head self-attention core over one sequence (S = all rows of the
// call, as the reference does: codegen.cpp:2224-2235, S = BS), flash-style
// for head sizes up to 128: no S x S matrix is ever materialised.  Larger
// head sizes take the wide path near the end of this file (blocks of query
// rows' scores materialised, multiplied by the GEMM kernels).
//
//   reference arithmetic: ns_attention_fwd, codegen.cpp:1724-1777
//   (per head: s = (q . k) * 1/sqrt(Dk); row softmax; ctx = P V)
//
// gfx950 design (wave64, fp32 MFMA 32x32x2):
//  * Workgroup = 4 waves = 128 queries of one head; each wave owns 32
//    queries.  Keys/values stream through LDS in 64-key tiles, double
//    buffered with register prefetch.
//  * Transposed products: S^T = K . Q^T and O^T = V^T . P^T.  In the 32x32
//    accumulator layout a lane then holds one QUERY column (lane % 32) and 16
//    keys / 16 head dims, so the online-softmax statistics of a query are
//    per-lane scalars (combined with the partner lane^32), and the score
//    accumulators are exactly the B operands of the P.V MFMAs -- probability
//    tiles never leave registers.
//  * exp2 with scores pre-multiplied by scale*log2(e); the final 1/l and the
//    transpose back to row-major go through LDS for coalesced stores.
#include <algorithm>
#include <cstdlib>

#include "common.h"
#include "kernels.h"

namespace nship {

typedef float floatx16 __attribute__((ext_vector_type(16)));

namespace {

// x if `keep`, else zeros; component-wise (a select on the struct itself is
// lowered through scratch memory).
__device__ __forceinline__ float4 keep4(bool keep, float4 x) {
  return make_float4(keep ? x.x : 0.f, keep ? x.y : 0.f, keep ? x.z : 0.f, keep ? x.w : 0.f);
}

constexpr int kBQ = 128;  // queries (keys) per workgroup of the backward kernels
constexpr int kFW = 8;     // forward: waves per workgroup (32 queries each), sharing every K/V tile
constexpr int kBK = 64;   // keys per tile

// Same bijective XCD-contiguous remap as the GEMM.
__device__ __forceinline__ int remap_xcd(int b, int T) {
  const int per = T >> 3, rem = T & 7;
  const int x = b & 7, i = b >> 3;
  return x * per + (x < rem ? x : rem) + i;
}

template <int DK>
struct KVTile {
  static constexpr int P = DK + 4;             // LDS row pitch (floats)
  static constexpr int kFloats = kBK * P;      // one of K or V
  static constexpr int kVec = kBK * DK / 4;    // float4 per tile
  static constexpr int kPer = kVec / 256;      // float4 per thread
  float4 k[kPer], v[kPer];
  int lim = 0;  // tile rows below lim exist

  // Rows past the end load a clamped row; store() zeroes them, so nothing
  // between load() and store() waits for the loads.
  __device__ void load(const float* __restrict__ K, const float* __restrict__ V, int64_t ld, int hcol, int key0,
                       int S, int t) {
    lim = S - key0;
#pragma unroll
    for (int i = 0; i < kPer; i++) {
      const int idx = t + 256 * i;
      const int key = idx / (DK / 4), c = (idx % (DK / 4)) * 4;
      const int64_t row = key < lim ? key0 + key : S - 1;
      k[i] = *reinterpret_cast<const float4*>(K + row * ld + hcol + c);
      v[i] = *reinterpret_cast<const float4*>(V + row * ld + hcol + c);
    }
  }
  __device__ void store(float* __restrict__ ks, int t) const {
    float* vs = ks + kFloats;
#pragma unroll
    for (int i = 0; i < kPer; i++) {
      const int idx = t + 256 * i;
      const int key = idx / (DK / 4), c = (idx % (DK / 4)) * 4;
      *reinterpret_cast<float4*>(ks + key * P + c) = keep4(key < lim, k[i]);
      *reinterpret_cast<float4*>(vs + key * P + c) = keep4(key < lim, v[i]);
    }
  }
};

// One K or V tile (64 keys x DK) in registers on its way to LDS (row pitch
// DK + 4); rows past the end load a clamped row and are zeroed by store(),
// so nothing between load() and store() waits for the loads.
template <int DK, int NTH>
struct HalfTile {
  static constexpr int P = DK + 4;
  static constexpr int kPer = kBK * DK / 4 / NTH;
  float4 r[kPer];
  int lim = 0;  // tile rows below lim exist
  __device__ void load(const float* __restrict__ X, int64_t ld, int hcol, int key0, int S, int t) {
    lim = S - key0;
#pragma unroll
    for (int i = 0; i < kPer; i++) {
      const int idx = t + NTH * i;
      const int key = idx / (DK / 4), c = (idx % (DK / 4)) * 4;
      const int64_t row = key < lim ? key0 + key : S - 1;
      r[i] = *reinterpret_cast<const float4*>(X + row * ld + hcol + c);
    }
  }
  __device__ void store(float* __restrict__ xs, int t) const {
#pragma unroll
    for (int i = 0; i < kPer; i++) {
      const int idx = t + NTH * i;
      const int key = idx / (DK / 4);
      *reinterpret_cast<float4*>(xs + key * P + (idx % (DK / 4)) * 4) = keep4(key < lim, r[i]);
    }
  }
};

// S^T tile (64 keys x this wave's 32 queries) = K_tile Q^T, in log2 units
// (Q is pre-scaled by scale * log2(e)).
template <int DK>
__device__ __forceinline__ void score_tile(const float* __restrict__ ks, const float (&qf)[DK / 2], int l32, int kh,
                                           floatx16 (&sc)[2]) {
  constexpr int P = DK + 4;
#pragma unroll
  for (int kb = 0; kb < 2; kb++)
#pragma unroll
    for (int v = 0; v < 16; v++) sc[kb][v] = 0.f;
#pragma unroll
  for (int g = 0; g < DK / 8; g++)
#pragma unroll
    for (int kb = 0; kb < 2; kb++) {
      const float4 kv = *reinterpret_cast<const float4*>(ks + (kb * 32 + l32) * P + 8 * g + 4 * kh);
      sc[kb] = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.x, qf[4 * g + 0], sc[kb], 0, 0, 0);
      sc[kb] = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.y, qf[4 * g + 1], sc[kb], 0, 0, 0);
      sc[kb] = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.z, qf[4 * g + 2], sc[kb], 0, 0, 0);
      sc[kb] = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.w, qf[4 * g + 3], sc[kb], 0, 0, 0);
    }
}

// Software-pipelined over key tiles: iteration `it` issues the score MFMAs
// of tile it+1 alongside the softmax of tile it, then O^T += V_it^T P_it^T.
// LDS holds two K tiles (it+1 in use, the other free for it+2) and two V
// tiles (it in use, the other free for it+1).  The rescale of O by
// exp2(m_old - m_new) is skipped when no lane's running max moved (the factor
// would be exactly 1).
template <int DK>
__global__ __launch_bounds__(kFW * 64) void flash_fwd_kernel(const float* __restrict__ Q, const float* __restrict__ K,
                                                        const float* __restrict__ V, float* __restrict__ ctx,
                                                        float* __restrict__ lse, int S, int H, int64_t ld,
                                                        float scale_log2, int nqb) {
  constexpr int P = DK + 4;
  constexpr int TF = kBK * P;   // floats of one K or V tile in LDS
  constexpr int NDB = DK / 32;  // 32-wide head-dim blocks of the output
  __shared__ __attribute__((aligned(16))) float sm[4 * TF];
  float* const kbuf = sm;           // K tile i at kbuf + (i & 1) * TF
  float* const vbuf = sm + 2 * TF;  // V tile i at vbuf + (i & 1) * TF

  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int l32 = lane & 31, kh = lane >> 5;
  const int L = remap_xcd(blockIdx.x, nqb * H);
  const int h = L / nqb, q0 = (L % nqb) * (32 * kFW);
  const int hcol = h * DK;
  const int qrow = q0 + w * 32 + l32;

  // B operand of S^T = K Q^T: this lane's query (pre-scaled), head dims 8g + 4kh + (0..3).
  float qf[DK / 2];
#pragma unroll
  for (int g = 0; g < DK / 8; g++) {
    const int64_t row = qrow < S ? qrow : S - 1;
    const float4 x = keep4(qrow < S, *reinterpret_cast<const float4*>(Q + row * ld + hcol + 8 * g + 4 * kh));
    qf[4 * g] = x.x * scale_log2; qf[4 * g + 1] = x.y * scale_log2;
    qf[4 * g + 2] = x.z * scale_log2; qf[4 * g + 3] = x.w * scale_log2;
  }

  floatx16 o[NDB];
#pragma unroll
  for (int d = 0; d < NDB; d++)
#pragma unroll
    for (int v = 0; v < 16; v++) o[d][v] = 0.f;
  float m = -INFINITY, l = 0.f;

  const int nkv = (S + kBK - 1) / kBK;
  HalfTile<DK, kFW * 64> tk, tv;
  tk.load(K, ld, hcol, 0, S, t);
  tv.load(V, ld, hcol, 0, S, t);
  tk.store(kbuf, t);
  tv.store(vbuf, t);
  tk.load(K, ld, hcol, (nkv > 1 ? 1 : 0) * kBK, S, t);
  tk.store(kbuf + TF, t);
  __syncthreads();
  floatx16 sc[2], sn[2];
  score_tile<DK>(kbuf, qf, l32, kh, sc);
  __syncthreads();  // kbuf tile 0 is overwritten at the end of iteration 0

  for (int it = 0; it < nkv; it++) {
    // prefetch K tile it+2 and V tile it+1 (clamped: the last tiles reload)
    tk.load(K, ld, hcol, min(it + 2, nkv - 1) * kBK, S, t);
    tv.load(V, ld, hcol, min(it + 1, nkv - 1) * kBK, S, t);
    // MFMA bursts run at raised wave priority, so a SIMD's other wave fills
    // the gaps with its softmax work rather than competing for issue
    __builtin_amdgcn_s_setprio(1);
    if (it + 1 < nkv) score_tile<DK>(kbuf + ((it + 1) & 1) * TF, qf, l32, kh, sn);
    __builtin_amdgcn_s_setprio(0);

    // Online softmax for this lane's query (keys 8*(v/4) + 4kh + v%4 of each block).
    const int kbase = it * kBK;
    if (kbase + kBK > S) {
#pragma unroll
      for (int kb = 0; kb < 2; kb++)
#pragma unroll
        for (int v = 0; v < 16; v++) {
          const int key = kbase + kb * 32 + 8 * (v >> 2) + 4 * kh + (v & 3);
          if (key >= S) sc[kb][v] = -INFINITY;
        }
    }
    float mloc = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; kb++)
#pragma unroll
      for (int v = 0; v < 16; v++) mloc = fmaxf(mloc, sc[kb][v]);
    mloc = fmaxf(mloc, __shfl_xor(mloc, 32, 64));
    const float mnew = fmaxf(m, mloc);
    if (__any(mnew > m)) {
      const float corr = exp2_hw(m - mnew);
      l *= corr;
#pragma unroll
      for (int d = 0; d < NDB; d++)
#pragma unroll
        for (int v = 0; v < 16; v++) o[d][v] *= corr;
    }
    float lsum = 0.f;
#pragma unroll
    for (int kb = 0; kb < 2; kb++)
#pragma unroll
      for (int v = 0; v < 16; v++) {
        const float p = exp2_hw(sc[kb][v] - mnew);
        sc[kb][v] = p;
        lsum += p;
      }
    lsum += __shfl_xor(lsum, 32, 64);
    l += lsum;
    m = mnew;

    // O^T += V^T P^T: step s of key block kb pairs key 8*(s/4)+4kh+s%4.
    __builtin_amdgcn_s_setprio(1);
    const float* vs = vbuf + (it & 1) * TF;
#pragma unroll
    for (int kb = 0; kb < 2; kb++)
#pragma unroll
      for (int s = 0; s < 16; s++) {
        const int key = kb * 32 + 8 * (s >> 2) + 4 * kh + (s & 3);
#pragma unroll
        for (int d = 0; d < NDB; d++)
          o[d] = __builtin_amdgcn_mfma_f32_32x32x2f32(vs[key * P + d * 32 + l32], sc[kb][s], o[d], 0, 0, 0);
      }
    __builtin_amdgcn_s_setprio(0);

    // K tile it (consumed last iteration) and V tile it-1 (consumed last
    // iteration) are free: fill them with K tile it+2 and V tile it+1.
    tk.store(kbuf + (it & 1) * TF, t);
    tv.store(vbuf + ((it + 1) & 1) * TF, t);
    __syncthreads();
#pragma unroll
    for (int kb = 0; kb < 2; kb++) sc[kb] = sn[kb];
  }

  // Row statistics for the backward pass: log2-sum-exp of the scaled scores.
  if (lse && kh == 0 && qrow < S) lse[(int64_t)h * S + qrow] = m + log2f(l);

  // O^T (d, query) / l  ->  LDS [query][d]  ->  coalesced rows of ctx.
  static_assert(kFW * 32 * (DK + 1) <= 4 * TF, "output staging fits the K/V buffers");
  const float inv = 1.f / l;
  float* T = sm + w * 32 * (DK + 1);
#pragma unroll
  for (int d = 0; d < NDB; d++)
#pragma unroll
    for (int v = 0; v < 16; v++) T[l32 * (DK + 1) + d * 32 + 8 * (v >> 2) + 4 * kh + (v & 3)] = o[d][v] * inv;
  __syncthreads();
  for (int r = 0; r < 32; r++) {
    const int q = q0 + w * 32 + r;
    if (q >= S) break;
    for (int c = lane; c < DK; c += 64) ctx[(int64_t)q * ld + hcol + c] = T[r * (DK + 1) + c];
  }
}

// Head sizes the tiled kernels do not take directly (dk not 32, 64 or 128,
// or rows not 16-byte aligned) run on a padded copy: every head's dk columns
// padded with zeros to DKP (the next of 32, 64, 128), row pitch H * DKP.
// Zero columns add nothing to a score q . k and give zero output columns,
// which unpad drops, so the padded problem computes the same attention (the
// scale stays 1/sqrt(dk)).
// dst[s, h*dkp + c] = c < dk ? src[s*ld + h*dk + c] : 0
__global__ __launch_bounds__(256) void attn_pad_kernel(const float* __restrict__ src, int64_t ld,
                                                       float* __restrict__ dst, int S, int H, int dk, int dkp) {
  const int64_t n = (int64_t)S * H * dkp, row = (int64_t)H * dkp;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const int64_t s = i / row;
    const int r = (int)(i - s * row), h = r / dkp, c = r - h * dkp;
    dst[i] = c < dk ? src[s * ld + (int64_t)h * dk + c] : 0.f;
  }
}

// dst[s*ld + h*dk + c] = src[s, h*dkp + c] for c < dk
__global__ __launch_bounds__(256) void attn_unpad_kernel(const float* __restrict__ src, float* __restrict__ dst,
                                                         int64_t ld, int S, int H, int dk, int dkp) {
  const int64_t n = (int64_t)S * H * dk, row = (int64_t)H * dk;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const int64_t s = i / row;
    const int r = (int)(i - s * row), h = r / dk, c = r - h * dk;
    dst[s * ld + r] = src[s * ((int64_t)H * dkp) + (int64_t)h * dkp + c];
  }
}


// ============================================================================
// Backward.  For one head, with c = scale * log2(e) and the forward's
// lse[q] = log2 sum_k 2^(c S[q,k]):
//   P = 2^(c S - lse),  dP = dO V^T,  dS = P (dP - delta),
//   delta[q] = sum_d dO[q,d] O[q,d]  (= sum_k P dP, the reference's `dot`)
//   dV = P^T dO,  dK = scale dS^T Q,  dQ = scale dS K
// (ns_attention_bwd, codegen.cpp:1785-1907, computes the same quantities
// with explicit S x S matrices.)  Two kernels, no atomics:
//  * dk/dv: one workgroup per 128 keys (32 per wave) loops over query tiles;
//    it forms S = Q K^T with the KEY as the lane column, so P and dS are the
//    A operands of dV = P^T dO and dK = dS^T Q directly from registers.
//  * dq: one workgroup per 128 queries loops over key tiles in the forward's
//    transposed layout (lane = query): dS^T feeds dQ^T = K^T dS^T.
// ============================================================================

template <int DK>
struct QTile {  // one 64-query tile of Q and dO (row pitch P) plus lse, delta
  static constexpr int P = DK + 4;
  static constexpr int kFloats = 2 * 64 * P + 128;
  static constexpr int kPer = 64 * DK / 4 / 256;  // float4 per thread per matrix
  float4 q[kPer], g[kPer];
  float l = 0.f, d = 0.f;
  int lim = 0;  // tile rows below lim exist
  // Rows past the end load a clamped row; store() zeroes them, so nothing
  // between load() and store() waits for the loads.
  __device__ void load(const float* __restrict__ Q, const float* __restrict__ dO, const float* __restrict__ lse,
                       const float* __restrict__ delta, int64_t ld, int hcol, int hS, int q0, int S, int t) {
    lim = S - q0;
#pragma unroll
    for (int i = 0; i < kPer; i++) {
      const int idx = t + 256 * i;
      const int r = idx / (DK / 4), c = (idx % (DK / 4)) * 4;
      const int64_t row = r < lim ? q0 + r : S - 1;
      q[i] = *reinterpret_cast<const float4*>(Q + row * ld + hcol + c);
      g[i] = *reinterpret_cast<const float4*>(dO + row * ld + hcol + c);
    }
    if (t < 64) {
      const int gq = q0 + t;
      // rows past the end: lse = +inf makes P = 0 there
      l = gq < S ? lse[hS + gq] : INFINITY;
      d = gq < S ? delta[hS + gq] : 0.f;
    }
  }
  __device__ void store(float* __restrict__ sm, int t) const {
#pragma unroll
    for (int i = 0; i < kPer; i++) {
      const int idx = t + 256 * i;
      const int r = idx / (DK / 4), c = (idx % (DK / 4)) * 4;
      *reinterpret_cast<float4*>(sm + r * P + c) = keep4(r < lim, q[i]);
      *reinterpret_cast<float4*>(sm + 64 * P + r * P + c) = keep4(r < lim, g[i]);
    }
    if (t < 64) {
      sm[2 * 64 * P + t] = l;
      sm[2 * 64 * P + 64 + t] = d;
    }
  }
};

// STORE_DS: also write dS = P o (dP - delta) (unscaled) to dS[h][query][key]
// for flash_bwd_dq_ds_kernel; requires S % 64 == 0.
// Two workgroups per CU up to DK = 64; at DK = 128 a lane's K and V rows and
// its dK / dV accumulators (4 x DK/2 registers) need one wave per SIMD.
template <int DK, bool STORE_DS>
__global__ __launch_bounds__(256, DK >= 128 ? 1 : 2) void flash_bwd_dkdv_kernel(const float* __restrict__ Q, const float* __restrict__ K,
                                                             const float* __restrict__ V, const float* __restrict__ dO,
                                                             const float* __restrict__ lse,
                                                             const float* __restrict__ delta, float* __restrict__ dK,
                                                             float* __restrict__ dV, float* __restrict__ dS, int S,
                                                             int H, int64_t ld, float scale, float c_log2, int nkb) {
  using Tile = QTile<DK>;
  constexpr int NDB = DK / 32;
  __shared__ __attribute__((aligned(16))) float sm[2 * Tile::kFloats];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int l32 = lane & 31, kh = lane >> 5;
  const int L = remap_xcd(blockIdx.x, nkb * H);
  const int h = L / nkb, k0 = (L % nkb) * kBQ;
  const int hcol = h * DK;
  const int64_t hS = (int64_t)h * S;
  const int key = k0 + w * 32 + l32;  // this lane's key (column of S)
  const float kneg = key < S ? 0.f : -INFINITY;

  // B operands: K and V rows of this lane's key, head dims 8g + 4kh + (0..3).
  float kf[DK / 2], vf[DK / 2];
#pragma unroll
  for (int g = 0; g < DK / 8; g++) {
    const int64_t row = key < S ? key : S - 1;
    const float4 a = keep4(key < S, *reinterpret_cast<const float4*>(K + row * ld + hcol + 8 * g + 4 * kh));
    const float4 b = keep4(key < S, *reinterpret_cast<const float4*>(V + row * ld + hcol + 8 * g + 4 * kh));
    kf[4 * g] = a.x; kf[4 * g + 1] = a.y; kf[4 * g + 2] = a.z; kf[4 * g + 3] = a.w;
    vf[4 * g] = b.x; vf[4 * g + 1] = b.y; vf[4 * g + 2] = b.z; vf[4 * g + 3] = b.w;
  }
  floatx16 dk[NDB], dv[NDB];
#pragma unroll
  for (int d = 0; d < NDB; d++)
#pragma unroll
    for (int v = 0; v < 16; v++) { dk[d][v] = 0.f; dv[d][v] = 0.f; }

  Tile tile;
  const int nq = (S + 63) / 64;
  tile.load(Q, dO, lse, delta, ld, hcol, (int)hS, 0, S, t);
  tile.store(sm, t);
  __syncthreads();
  for (int it = 0; it < nq; it++) {
    const int cur = it & 1;
    const bool more = it + 1 < nq;
    if (more) tile.load(Q, dO, lse, delta, ld, hcol, (int)hS, (it + 1) * 64, S, t);
    const float* qs = sm + cur * Tile::kFloats;
    const float* gs = qs + 64 * Tile::P;
    const float* ls = qs + 2 * 64 * Tile::P;
    const float* ds = ls + 64;
#pragma unroll 1
    for (int qb = 0; qb < 2; qb++) {
      floatx16 sc, dp;
#pragma unroll
      for (int v = 0; v < 16; v++) { sc[v] = 0.f; dp[v] = 0.f; }
      // MFMA phases at raised wave priority (as in the forward)
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int g = 0; g < DK / 8; g++) {
        const float4 qa = *reinterpret_cast<const float4*>(qs + (qb * 32 + l32) * Tile::P + 8 * g + 4 * kh);
        const float4 ga = *reinterpret_cast<const float4*>(gs + (qb * 32 + l32) * Tile::P + 8 * g + 4 * kh);
        sc = __builtin_amdgcn_mfma_f32_32x32x2f32(qa.x, kf[4 * g + 0], sc, 0, 0, 0);
        sc = __builtin_amdgcn_mfma_f32_32x32x2f32(qa.y, kf[4 * g + 1], sc, 0, 0, 0);
        sc = __builtin_amdgcn_mfma_f32_32x32x2f32(qa.z, kf[4 * g + 2], sc, 0, 0, 0);
        sc = __builtin_amdgcn_mfma_f32_32x32x2f32(qa.w, kf[4 * g + 3], sc, 0, 0, 0);
        dp = __builtin_amdgcn_mfma_f32_32x32x2f32(ga.x, vf[4 * g + 0], dp, 0, 0, 0);
        dp = __builtin_amdgcn_mfma_f32_32x32x2f32(ga.y, vf[4 * g + 1], dp, 0, 0, 0);
        dp = __builtin_amdgcn_mfma_f32_32x32x2f32(ga.z, vf[4 * g + 2], dp, 0, 0, 0);
        dp = __builtin_amdgcn_mfma_f32_32x32x2f32(ga.w, vf[4 * g + 3], dp, 0, 0, 0);
      }
      __builtin_amdgcn_s_setprio(0);
      // element v: query qb*32 + 8(v/4) + 4kh + v%4, key = this lane's
#pragma unroll
      for (int v = 0; v < 16; v++) {
        const int qr = qb * 32 + 8 * (v >> 2) + 4 * kh + (v & 3);
        // keys past the end: exponent -inf (kneg), p = 0; lse is finite or
        // +inf, so no NaN, and no per-element branch
        const float p = exp2_hw(fmaf(sc[v], c_log2, kneg) - ls[qr]);
        sc[v] = p;
        dp[v] = p * (dp[v] - ds[qr]);
      }
      if (STORE_DS && key < S) {
        // lanes 0-31 / 32-63 write 32 consecutive keys of one query row each;
        // every query row of the tile exists (S % 64 == 0)
        // element v sits in row 8 (v / 4) + v % 4: walk a single pointer
        float* __restrict__ dst = dS + ((int64_t)h * S + it * 64 + qb * 32 + 4 * kh) * S + key;
#pragma unroll
        for (int g = 0; g < 4; g++) {
#pragma unroll
          for (int j = 0; j < 4; j++) {
            *dst = dp[4 * g + j];
            dst += S;
          }
          dst += 4 * (int64_t)S;
        }
      }
      __builtin_amdgcn_s_setprio(1);
      // dV += P^T dO, dK += dS^T Q: step s pairs query 8(s/4) + 4kh + s%4.
#pragma unroll
      for (int s = 0; s < 16; s++) {
        const int qr = qb * 32 + 8 * (s >> 2) + 4 * kh + (s & 3);
#pragma unroll
        for (int d = 0; d < NDB; d++) {
          dv[d] = __builtin_amdgcn_mfma_f32_32x32x2f32(sc[s], gs[qr * Tile::P + d * 32 + l32], dv[d], 0, 0, 0);
          dk[d] = __builtin_amdgcn_mfma_f32_32x32x2f32(dp[s], qs[qr * Tile::P + d * 32 + l32], dk[d], 0, 0, 0);
        }
      }
    }
    __builtin_amdgcn_s_setprio(0);
    if (more) tile.store(sm + (cur ^ 1) * Tile::kFloats, t);
    __syncthreads();
  }
  // accumulator v of block d: key w*32 + 8(v/4) + 4kh + v%4, head dim d*32 + l32
#pragma unroll
  for (int d = 0; d < NDB; d++)
#pragma unroll
    for (int v = 0; v < 16; v++) {
      const int kr = k0 + w * 32 + 8 * (v >> 2) + 4 * kh + (v & 3);
      if (kr < S) {
        dK[(int64_t)kr * ld + hcol + d * 32 + l32] = dk[d][v] * scale;
        dV[(int64_t)kr * ld + hcol + d * 32 + l32] = dv[d][v];
      }
    }
}

template <int DK>
__global__ __launch_bounds__(256) void flash_bwd_dq_kernel(const float* __restrict__ Q, const float* __restrict__ K,
                                                           const float* __restrict__ V, const float* __restrict__ dO,
                                                           const float* __restrict__ lse,
                                                           const float* __restrict__ delta, float* __restrict__ dQ,
                                                           int S, int H, int64_t ld, float scale, float c_log2,
                                                           int nqb) {
  using Tile = KVTile<DK>;
  constexpr int NDB = DK / 32;
  __shared__ __attribute__((aligned(16))) float sm[2 * 2 * Tile::kFloats];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int l32 = lane & 31, kh = lane >> 5;
  const int L = remap_xcd(blockIdx.x, nqb * H);
  const int h = L / nqb, q0 = (L % nqb) * kBQ;
  const int hcol = h * DK;
  const int qrow = q0 + w * 32 + l32;
  float qf[DK / 2], gf[DK / 2];
#pragma unroll
  for (int g = 0; g < DK / 8; g++) {
    const int64_t row = qrow < S ? qrow : S - 1;
    const float4 a = keep4(qrow < S, *reinterpret_cast<const float4*>(Q + row * ld + hcol + 8 * g + 4 * kh));
    const float4 b = keep4(qrow < S, *reinterpret_cast<const float4*>(dO + row * ld + hcol + 8 * g + 4 * kh));
    qf[4 * g] = a.x; qf[4 * g + 1] = a.y; qf[4 * g + 2] = a.z; qf[4 * g + 3] = a.w;
    gf[4 * g] = b.x; gf[4 * g + 1] = b.y; gf[4 * g + 2] = b.z; gf[4 * g + 3] = b.w;
  }
  const float lq = qrow < S ? lse[(int64_t)h * S + qrow] : INFINITY;
  const float dq_delta = qrow < S ? delta[(int64_t)h * S + qrow] : 0.f;
  floatx16 acc[NDB];
#pragma unroll
  for (int d = 0; d < NDB; d++)
#pragma unroll
    for (int v = 0; v < 16; v++) acc[d][v] = 0.f;

  Tile tile;
  const int nkv = (S + kBK - 1) / kBK;
  tile.load(K, V, ld, hcol, 0, S, t);
  tile.store(sm, t);
  __syncthreads();
  for (int it = 0; it < nkv; it++) {
    const int cur = it & 1;
    const bool more = it + 1 < nkv;
    if (more) tile.load(K, V, ld, hcol, (it + 1) * kBK, S, t);
    const float* ks = sm + cur * 2 * Tile::kFloats;
    const float* vs = ks + Tile::kFloats;
    floatx16 sc[2], dp[2];
#pragma unroll
    for (int kb = 0; kb < 2; kb++)
#pragma unroll
      for (int v = 0; v < 16; v++) { sc[kb][v] = 0.f; dp[kb][v] = 0.f; }
#pragma unroll
    for (int g = 0; g < DK / 8; g++)
#pragma unroll
      for (int kb = 0; kb < 2; kb++) {
        const float4 ka = *reinterpret_cast<const float4*>(ks + (kb * 32 + l32) * Tile::P + 8 * g + 4 * kh);
        const float4 va = *reinterpret_cast<const float4*>(vs + (kb * 32 + l32) * Tile::P + 8 * g + 4 * kh);
        sc[kb] = __builtin_amdgcn_mfma_f32_32x32x2f32(ka.x, qf[4 * g + 0], sc[kb], 0, 0, 0);
        sc[kb] = __builtin_amdgcn_mfma_f32_32x32x2f32(ka.y, qf[4 * g + 1], sc[kb], 0, 0, 0);
        sc[kb] = __builtin_amdgcn_mfma_f32_32x32x2f32(ka.z, qf[4 * g + 2], sc[kb], 0, 0, 0);
        sc[kb] = __builtin_amdgcn_mfma_f32_32x32x2f32(ka.w, qf[4 * g + 3], sc[kb], 0, 0, 0);
        dp[kb] = __builtin_amdgcn_mfma_f32_32x32x2f32(va.x, gf[4 * g + 0], dp[kb], 0, 0, 0);
        dp[kb] = __builtin_amdgcn_mfma_f32_32x32x2f32(va.y, gf[4 * g + 1], dp[kb], 0, 0, 0);
        dp[kb] = __builtin_amdgcn_mfma_f32_32x32x2f32(va.z, gf[4 * g + 2], dp[kb], 0, 0, 0);
        dp[kb] = __builtin_amdgcn_mfma_f32_32x32x2f32(va.w, gf[4 * g + 3], dp[kb], 0, 0, 0);
      }
    const int kbase = it * kBK;
#pragma unroll
    for (int kb = 0; kb < 2; kb++)
#pragma unroll
      for (int v = 0; v < 16; v++) {
        const int kr = kbase + kb * 32 + 8 * (v >> 2) + 4 * kh + (v & 3);
        const float p = exp2_hw(fmaf(sc[kb][v], c_log2, kr < S ? 0.f : -INFINITY) - lq);
        dp[kb][v] = p * (dp[kb][v] - dq_delta);
      }
    // dQ^T += K^T dS^T: step s of key block kb pairs key 8(s/4) + 4kh + s%4.
#pragma unroll
    for (int kb = 0; kb < 2; kb++)
#pragma unroll
      for (int s = 0; s < 16; s++) {
        const int kr = kb * 32 + 8 * (s >> 2) + 4 * kh + (s & 3);
#pragma unroll
        for (int d = 0; d < NDB; d++)
          acc[d] = __builtin_amdgcn_mfma_f32_32x32x2f32(ks[kr * Tile::P + d * 32 + l32], dp[kb][s], acc[d], 0, 0, 0);
      }
    if (more) tile.store(sm + (cur ^ 1) * 2 * Tile::kFloats, t);
    __syncthreads();
  }
  // dQ^T (d, query) -> LDS [query][d] -> rows of dQ
  float* T = sm + w * 32 * (DK + 1);
#pragma unroll
  for (int d = 0; d < NDB; d++)
#pragma unroll
    for (int v = 0; v < 16; v++) T[l32 * (DK + 1) + d * 32 + 8 * (v >> 2) + 4 * kh + (v & 3)] = acc[d][v] * scale;
  __syncthreads();
  for (int r = 0; r < 32; r++) {
    const int q = q0 + w * 32 + r;
    if (q >= S) break;
    for (int c = lane; c < DK; c += 64) dQ[(int64_t)q * ld + hcol + c] = T[r * (DK + 1) + c];
  }
}

// dQ = scale * dS K from the stored dS (S % 64 == 0): the dq kernel's
// transposed product dQ^T += K^T dS^T without recomputing S and dP.  Lane =
// query; its dS operands of a 64-key tile are 8 float4 read straight from its
// row, dlo/dhi[j] = keys key0 + 32 kb + 8 j + 4 kh + (0..3) for kb = 0/1
// (drow includes the 4 kh offset; a lane past the end reads row S - 1 and its
// operands are zeroed where they are taken).  Each half is reloaded for the
// next tile as soon as its MFMAs have taken it, and each K tile (float4 i of
// thread t: key (t + 256 i) / (DK/4), dims 4 ((t + 256 i) % (DK/4))) is
// loaded an iteration before it is written to LDS, so both prefetches cross
// the loop's back edge and the compiler cannot sink them next to their use.
template <int DK>
__global__ __launch_bounds__(256) void flash_bwd_dq_ds_kernel(const float* __restrict__ K,
                                                              const float* __restrict__ dS, float* __restrict__ dQ,
                                                              int S, int H, int64_t ld, float scale, int nqb) {
  constexpr int NDB = DK / 32;
  constexpr int P = DK + 4;
  constexpr int kPer = kBK * DK / 4 / 256;
  __shared__ __attribute__((aligned(16))) float sm[2 * kBK * P > 4 * 32 * (DK + 1) ? 2 * kBK * P : 4 * 32 * (DK + 1)];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int l32 = lane & 31, kh = lane >> 5;
  const int L = remap_xcd(blockIdx.x, nqb * H);
  const int h = L / nqb, q0 = (L % nqb) * kBQ;
  const int hcol = h * DK;
  const int qrow = q0 + w * 32 + l32;
  const bool qin = qrow < S;
  const float* __restrict__ drow = dS + ((int64_t)h * S + (qin ? qrow : S - 1)) * S + 4 * kh;
  floatx16 acc[NDB];
#pragma unroll
  for (int d = 0; d < NDB; d++)
#pragma unroll
    for (int v = 0; v < 16; v++) acc[d][v] = 0.f;

  // native vectors: an array of HIP float4 carried across the loop stays in
  // scratch memory, these stay in registers
  fvec4 kt[kPer];
  float4 dlo[4], dhi[4];
  auto load_k = [&](int key0) {
#pragma unroll
    for (int i = 0; i < kPer; i++) {
      const int idx = t + 256 * i;
      kt[i] = *reinterpret_cast<const fvec4*>(K + (int64_t)(key0 + idx / (DK / 4)) * ld + hcol + (idx % (DK / 4)) * 4);
    }
  };
  auto store_k = [&](float* __restrict__ ks) {
#pragma unroll
    for (int i = 0; i < kPer; i++) {
      const int idx = t + 256 * i;
      *reinterpret_cast<fvec4*>(ks + (idx / (DK / 4)) * P + (idx % (DK / 4)) * 4) = kt[i];
    }
  };
  auto load_d = [&](float4(&dd)[4], int key0) {
#pragma unroll
    for (int j = 0; j < 4; j++) dd[j] = *reinterpret_cast<const float4*>(drow + key0 + 8 * j);
  };
  // the MFMAs of one 32-key half: step s pairs key 32 kb + 8 (s/4) + 4 kh + s%4
  auto half = [&](const float* __restrict__ ks, float4(&dd)[4], int kb, int next) {
    float dv[16];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const float4 x = keep4(qin, dd[j]);
      dv[4 * j] = x.x; dv[4 * j + 1] = x.y; dv[4 * j + 2] = x.z; dv[4 * j + 3] = x.w;
    }
    load_d(dd, next + 32 * kb);
    __builtin_amdgcn_sched_barrier(0);  // issue the reload before the MFMAs
#pragma unroll
    for (int s2 = 0; s2 < 16; s2++) {
      const int kr = kb * 32 + 8 * (s2 >> 2) + 4 * kh + (s2 & 3);
#pragma unroll
      for (int d = 0; d < NDB; d++)
        acc[d] = __builtin_amdgcn_mfma_f32_32x32x2f32(ks[kr * P + d * 32 + l32], dv[s2], acc[d], 0, 0, 0);
    }
  };

  const int nkv = S / kBK;
  load_k(0);
  store_k(sm);
  // the loop's issue order (K tile, then the two halves), so that each wait
  // in the loop covers only the loads it needs
  load_k((nkv > 1 ? 1 : 0) * kBK);
  load_d(dlo, 0);
  load_d(dhi, 32);
  __syncthreads();
  for (int it = 0; it < nkv; it++) {
    const int cur = it & 1;
    // K tile it+1 (loaded an iteration ago) into the buffer that the last
    // iteration read; the barrier at this iteration's end publishes it.  The
    // last iteration stores a tile that nothing reads.
    store_k(sm + (cur ^ 1) * kBK * P);
    load_k(min(it + 2, nkv - 1) * kBK);
    __builtin_amdgcn_sched_barrier(0);
    const int next = min(it + 1, nkv - 1) * kBK;  // the last step reloads its own tile
    const float* ks = sm + cur * kBK * P;
    half(ks, dlo, 0, next);
    half(ks, dhi, 1, next);
    __syncthreads();
  }
  // dQ^T (d, query) -> LDS [query][d] -> rows of dQ
  float* T = sm + w * 32 * (DK + 1);
#pragma unroll
  for (int d = 0; d < NDB; d++)
#pragma unroll
    for (int v = 0; v < 16; v++) T[l32 * (DK + 1) + d * 32 + 8 * (v >> 2) + 4 * kh + (v & 3)] = acc[d][v] * scale;
  __syncthreads();
  for (int r = 0; r < 32; r++) {
    const int q = q0 + w * 32 + r;
    if (q >= S) break;
    for (int c = lane; c < DK; c += 64) dQ[(int64_t)q * ld + hcol + c] = T[r * (DK + 1) + c];
  }
}

// delta for DK in {32, 64} on 16-byte aligned rows: one wave per query row,
// one float4 per lane and pass, DK/4 lanes per head (a head's lanes are all
// in or all out of a pass, so the shuffles stay among active lanes).
template <int DK>
__global__ __launch_bounds__(256) void attn_delta_rows_kernel(const float* __restrict__ dO,
                                                              const float* __restrict__ O, float* __restrict__ delta,
                                                              int S, int H, int64_t ld) {
  constexpr int LPH = DK / 4;
  const int q = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (q >= S) return;
  const int D = H * DK;
  for (int c = lane * 4; c < D; c += 256) {
    const float4 a = *reinterpret_cast<const float4*>(dO + (int64_t)q * ld + c);
    const float4 b = *reinterpret_cast<const float4*>(O + (int64_t)q * ld + c);
    float p = a.x * b.x + a.y * b.y + a.z * b.z + a.w * b.w;
#pragma unroll
    for (int o = LPH / 2; o > 0; o >>= 1) p += __shfl_xor(p, o, 64);
    if ((lane & (LPH - 1)) == 0) delta[(int64_t)(c / DK) * S + q] = p;
  }
}

// Head sizes above 128 (the wide path): the scores of a block of query rows
// are materialised as [H][rows][S] by the MFMA GEMM kernels, and these row
// kernels apply the reference's per-row arithmetic to them
// (codegen.cpp:1746-1766 forward, :1868-1873 backward).  One workgroup per
// row; VEC: the row length is a multiple of 4 (rows 16-byte aligned).

// Sum or max over the 256 threads; every thread gets the result.
template <bool MAX>
__device__ __forceinline__ float wide_block_reduce(float v, float* red) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float u = __shfl_xor(v, o, 64);
    v = MAX ? fmaxf(v, u) : v + u;
  }
  __syncthreads();  // earlier readers of red are done
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  v = red[0];
#pragma unroll
  for (int i = 1; i < 4; i++) v = MAX ? fmaxf(v, red[i]) : v + red[i];
  return v;
}

// Row r of P (the raw dots q . k) becomes softmax(dots * scale): the scaled
// score rounded as the reference stores it, exp(score - max), divided by the
// row's sum.  lse (optional): row r = h * nq + i writes lse[h * S + q0 + i]
// in the flash kernels' log2 units.
template <bool VEC>
__global__ __launch_bounds__(256) void wide_softmax_kernel(float* __restrict__ P, int S, float scale,
                                                           float* __restrict__ lse, int nq, int q0) {
#pragma clang fp contract(off)
  __shared__ float red[4];
  float* __restrict__ row = P + (int64_t)blockIdx.x * S;
  const int t = threadIdx.x;
  float m = -INFINITY, l = 0.f;
  if constexpr (VEC) {
    float4* r4 = reinterpret_cast<float4*>(row);
    const int n4 = S / 4;
    for (int j = t; j < n4; j += 256) {
      const float4 a = r4[j];
      m = fmaxf(fmaxf(m, fmaxf(a.x * scale, a.y * scale)), fmaxf(a.z * scale, a.w * scale));
    }
    m = wide_block_reduce<true>(m, red);
    for (int j = t; j < n4; j += 256) {
      const float4 a = r4[j];
      const float4 e = make_float4(expf(a.x * scale - m), expf(a.y * scale - m), expf(a.z * scale - m),
                                   expf(a.w * scale - m));
      r4[j] = e;
      l += e.x + e.y + e.z + e.w;
    }
    l = wide_block_reduce<false>(l, red);
    for (int j = t; j < n4; j += 256) {
      const float4 e = r4[j];
      r4[j] = make_float4(e.x / l, e.y / l, e.z / l, e.w / l);
    }
  } else {
    for (int j = t; j < S; j += 256) m = fmaxf(m, row[j] * scale);
    m = wide_block_reduce<true>(m, red);
    for (int j = t; j < S; j += 256) {
      const float e = expf(row[j] * scale - m);
      row[j] = e;
      l += e;
    }
    l = wide_block_reduce<false>(l, red);
    for (int j = t; j < S; j += 256) row[j] = row[j] / l;
  }
  if (lse && t == 0) {
    const int h = blockIdx.x / nq, i = blockIdx.x % nq;
    lse[(int64_t)h * S + q0 + i] = m * 1.4426950408889634f + log2f(l);
  }
}

// The same two row kernels with the row held in registers, for rows of up
// to 16 K floats that are a multiple of 4 (one read and one write of each
// element instead of three reads and two writes): 1024 threads, float4
// chunks t + 1024 i, i < EPT / 4.
template <bool MAX>
__device__ __forceinline__ float wide_block_reduce16(float v, float* red) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float u = __shfl_xor(v, o, 64);
    v = MAX ? fmaxf(v, u) : v + u;
  }
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  v = red[0];
#pragma unroll
  for (int i = 1; i < 16; i++) v = MAX ? fmaxf(v, red[i]) : v + red[i];
  return v;
}

template <int EPT>
__global__ __launch_bounds__(1024) void wide_softmax_reg_kernel(float* __restrict__ P, int S, float scale,
                                                                float* __restrict__ lse, int nq, int q0) {
#pragma clang fp contract(off)
  __shared__ float red[16];
  float4* __restrict__ r4 = reinterpret_cast<float4*>(P + (int64_t)blockIdx.x * S);
  const int t = threadIdx.x, n4 = S / 4;
  float4 x[EPT / 4];
  float m = -INFINITY;
#pragma unroll
  for (int i = 0; i < EPT / 4; i++) {
    const int c = t + 1024 * i;
    x[i] = c < n4 ? r4[c] : make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
    if (c < n4) m = fmaxf(fmaxf(m, fmaxf(x[i].x * scale, x[i].y * scale)), fmaxf(x[i].z * scale, x[i].w * scale));
  }
  m = wide_block_reduce16<true>(m, red);
  float l = 0.f;
#pragma unroll
  for (int i = 0; i < EPT / 4; i++)
    if (t + 1024 * i < n4) {
      x[i] = make_float4(expf(x[i].x * scale - m), expf(x[i].y * scale - m), expf(x[i].z * scale - m),
                         expf(x[i].w * scale - m));
      l += x[i].x + x[i].y + x[i].z + x[i].w;
    }
  l = wide_block_reduce16<false>(l, red);
#pragma unroll
  for (int i = 0; i < EPT / 4; i++) {
    const int c = t + 1024 * i;
    if (c < n4) r4[c] = make_float4(x[i].x / l, x[i].y / l, x[i].z / l, x[i].w / l);
  }
  if (lse && t == 0) {
    const int h = blockIdx.x / nq, i = blockIdx.x % nq;
    lse[(int64_t)h * S + q0 + i] = m * 1.4426950408889634f + log2f(l);
  }
}

template <int EPT>
__global__ __launch_bounds__(1024) void wide_dsoftmax_reg_kernel(const float* __restrict__ P, float* __restrict__ G,
                                                                 int S, float scale) {
#pragma clang fp contract(off)
  __shared__ float red[16];
  const int64_t off = (int64_t)blockIdx.x * S;
  const float4* __restrict__ p4 = reinterpret_cast<const float4*>(P + off);
  float4* __restrict__ g4 = reinterpret_cast<float4*>(G + off);
  const int t = threadIdx.x, n4 = S / 4;
  float4 a[EPT / 4], b[EPT / 4];
  float dot = 0.f;
#pragma unroll
  for (int i = 0; i < EPT / 4; i++) {
    const int c = t + 1024 * i;
    if (c < n4) {
      a[i] = p4[c];
      b[i] = g4[c];
      dot += a[i].x * b[i].x + a[i].y * b[i].y + a[i].z * b[i].z + a[i].w * b[i].w;
    }
  }
  dot = wide_block_reduce16<false>(dot, red);
#pragma unroll
  for (int i = 0; i < EPT / 4; i++) {
    const int c = t + 1024 * i;
    if (c < n4)
      g4[c] = make_float4(a[i].x * (b[i].x - dot) * scale, a[i].y * (b[i].y - dot) * scale,
                          a[i].z * (b[i].z - dot) * scale, a[i].w * (b[i].w - dot) * scale);
  }
}

// Row r of G (dP = dO V^T) becomes scale * P o (dP - sum_j P dP): dS with
// the 1/sqrt(dk) of dQ and dK folded in.
template <bool VEC>
__global__ __launch_bounds__(256) void wide_dsoftmax_kernel(const float* __restrict__ P, float* __restrict__ G, int S,
                                                            float scale) {
#pragma clang fp contract(off)
  __shared__ float red[4];
  const int64_t off = (int64_t)blockIdx.x * S;
  const float* __restrict__ p = P + off;
  float* __restrict__ g = G + off;
  const int t = threadIdx.x;
  float dot = 0.f;
  if constexpr (VEC) {
    const float4* p4 = reinterpret_cast<const float4*>(p);
    float4* g4 = reinterpret_cast<float4*>(g);
    const int n4 = S / 4;
    for (int j = t; j < n4; j += 256) {
      const float4 a = p4[j], b = g4[j];
      dot += a.x * b.x + a.y * b.y + a.z * b.z + a.w * b.w;
    }
    dot = wide_block_reduce<false>(dot, red);
    for (int j = t; j < n4; j += 256) {
      const float4 a = p4[j], b = g4[j];
      g4[j] = make_float4(a.x * (b.x - dot) * scale, a.y * (b.y - dot) * scale, a.z * (b.z - dot) * scale,
                          a.w * (b.w - dot) * scale);
    }
  } else {
    for (int j = t; j < S; j += 256) dot += p[j] * g[j];
    dot = wide_block_reduce<false>(dot, red);
    for (int j = t; j < S; j += 256) g[j] = p[j] * (g[j] - dot) * scale;
  }
}

}  // namespace

// The tiled kernels' head sizes; others up to 128 are padded to the next one.
static int64_t padded_dk(int64_t dk) { return dk <= 32 ? 32 : dk <= 64 ? 64 : dk <= 128 ? 128 : 0; }

// Query rows per block of the wide path: all S when H * S * S floats fit
// 1 GiB, else as many as do (at least one).  The environment variable
// NSHIP_ATTN_WIDE_ROWS (a positive integer) lowers it, so that small cases
// can run several blocks.
static int64_t wide_rows(int64_t S, int64_t H) {
  constexpr int64_t kWideFloats = int64_t(1) << 28;
  int64_t r = std::max<int64_t>(1, std::min<int64_t>(S, kWideFloats / std::max<int64_t>(1, H * S)));
  if (const char* e = getenv("NSHIP_ATTN_WIDE_ROWS")) {
    const long long v = atoll(e);
    if (v > 0) r = std::min<int64_t>(r, v);
  }
  return r;
}

// P V (forward) and dS K (backward dQ) of a block of nq query rows:
// [nq, S] x [S, dk] per head.  K = S is long and the output has few tiles,
// so they split K (gemm_split_count) through a workspace placed after the
// score buffers, at a 64-float boundary.
static GemmArgs wide_pv_args(int64_t nq, int64_t S, int64_t dk) {
  GemmArgs g;
  g.M = (int)nq; g.N = (int)dk; g.K = (int)S;
  return g;
}

static size_t wide_split_floats(int64_t S, int64_t H, int64_t dk) {
  const int64_t rows = wide_rows(S, H);
  size_t m = 0;
  for (const int64_t nq : {rows, S % rows})
    if (nq > 0) {
      const GemmArgs g = wide_pv_args(nq, S, dk);
      m = std::max(m, gemm_split_workspace(g, (int)H, gemm_split_count(g, (int)H)));
    }
  return m;
}

static int64_t wide_score_floats(int64_t S, int64_t H, bool backward) {
  return ((backward ? 2 : 1) * H * wide_rows(S, H) * S + 63) / 64 * 64;
}

// Scores of query rows q0 .. q0 + nq of every head: P[h] = Q_h K_h^T (raw
// dots), [H][nq][S].
static int wide_scores(const float* Q, const float* K, float* P, int64_t q0, int64_t nq, int64_t S, int64_t H,
                       int64_t dk, int64_t ld, hipStream_t s) {
  GemmArgs g;
  g.A = Q + q0 * ld; g.lda = ld; g.sA = dk;
  g.B = K; g.ldb = ld; g.sB = dk;
  g.C = P; g.ldc = S; g.sC = nq * S;
  g.M = (int)nq; g.N = (int)S; g.K = (int)dk;
  return launch_gemm_ex(g, false, true, (int)H, s);
}

// Elements per thread of the register-resident row kernels (0: the row does
// not fit, or is not a whole number of 16-byte aligned float4).
static int wide_reg_ept(int64_t S, const void* a, const void* b) {
  if (S % 4 != 0 || (reinterpret_cast<uintptr_t>(a) & 15) || (reinterpret_cast<uintptr_t>(b) & 15)) return 0;
  return S <= 4096 ? 4 : S <= 8192 ? 8 : S <= 16384 ? 16 : 0;
}

static int wide_softmax(float* P, int64_t q0, int64_t nq, int64_t S, int64_t H, float scale, float* lse,
                        hipStream_t s) {
  const bool vec = S % 4 == 0 && (reinterpret_cast<uintptr_t>(P) & 15) == 0;
  const dim3 grid((unsigned)(H * nq)), block(256), big(1024);
  switch (wide_reg_ept(S, P, P)) {
    case 4: hipLaunchKernelGGL(wide_softmax_reg_kernel<4>, grid, big, 0, s, P, (int)S, scale, lse, (int)nq, (int)q0); break;
    case 8: hipLaunchKernelGGL(wide_softmax_reg_kernel<8>, grid, big, 0, s, P, (int)S, scale, lse, (int)nq, (int)q0); break;
    case 16: hipLaunchKernelGGL(wide_softmax_reg_kernel<16>, grid, big, 0, s, P, (int)S, scale, lse, (int)nq, (int)q0); break;
    default:
      if (vec) hipLaunchKernelGGL(wide_softmax_kernel<true>, grid, block, 0, s, P, (int)S, scale, lse, (int)nq, (int)q0);
      else hipLaunchKernelGGL(wide_softmax_kernel<false>, grid, block, 0, s, P, (int)S, scale, lse, (int)nq, (int)q0);
  }
  NSH_LAUNCHED();
  return 0;
}

// ctx = P V per block of query rows.
static int wide_fwd(const float* Q, const float* K, const float* V, float* ctx, float* lse, int64_t S, int64_t H,
                    int64_t dk, int64_t ld, float scale, float* ws, hipStream_t s) {
  const int64_t rows = wide_rows(S, H);
  for (int64_t q0 = 0; q0 < S; q0 += rows) {
    const int64_t nq = std::min(rows, S - q0);
    if (wide_scores(Q, K, ws, q0, nq, S, H, dk, ld, s) || wide_softmax(ws, q0, nq, S, H, scale, lse, s)) return -1;
    GemmArgs g = wide_pv_args(nq, S, dk);
    g.A = ws; g.lda = S; g.sA = nq * S;
    g.B = V; g.ldb = ld; g.sB = dk;
    g.C = ctx + q0 * ld; g.ldc = ld; g.sC = dk;
    if (launch_gemm_split(g, false, false, (int)H, gemm_split_count(g, (int)H), ws + wide_score_floats(S, H, false), s))
      return -1;
  }
  return 0;
}

// Per block of query rows: P again (as the forward computes it), G = dO V^T,
// G = scale * dS, then dV += P^T dO, dK += G^T Q (both summed over the
// blocks in order) and dQ = G K for the block's rows.
static int wide_bwd(const float* Q, const float* K, const float* V, const float* dO, float* dQ, float* dK, float* dV,
                    int64_t S, int64_t H, int64_t dk, int64_t ld, float scale, float* ws, hipStream_t s) {
  const int64_t rows = wide_rows(S, H);
  float *P = ws, *G = ws + H * rows * S;
  const bool vec = S % 4 == 0 && (reinterpret_cast<uintptr_t>(G) & 15) == 0 && (reinterpret_cast<uintptr_t>(P) & 15) == 0;
  for (int64_t q0 = 0; q0 < S; q0 += rows) {
    const int64_t nq = std::min(rows, S - q0);
    if (wide_scores(Q, K, P, q0, nq, S, H, dk, ld, s) || wide_softmax(P, q0, nq, S, H, scale, nullptr, s)) return -1;
    GemmArgs g;
    g.A = dO + q0 * ld; g.lda = ld; g.sA = dk;
    g.B = V; g.ldb = ld; g.sB = dk;
    g.C = G; g.ldc = S; g.sC = nq * S;
    g.M = (int)nq; g.N = (int)S; g.K = (int)dk;
    if (launch_gemm_ex(g, false, true, (int)H, s)) return -1;
    const dim3 grid((unsigned)(H * nq)), block(256), big(1024);
    switch (wide_reg_ept(S, P, G)) {
      case 4: hipLaunchKernelGGL(wide_dsoftmax_reg_kernel<4>, grid, big, 0, s, P, G, (int)S, scale); break;
      case 8: hipLaunchKernelGGL(wide_dsoftmax_reg_kernel<8>, grid, big, 0, s, P, G, (int)S, scale); break;
      case 16: hipLaunchKernelGGL(wide_dsoftmax_reg_kernel<16>, grid, big, 0, s, P, G, (int)S, scale); break;
      default:
        if (vec) hipLaunchKernelGGL(wide_dsoftmax_kernel<true>, grid, block, 0, s, P, G, (int)S, scale);
        else hipLaunchKernelGGL(wide_dsoftmax_kernel<false>, grid, block, 0, s, P, G, (int)S, scale);
    }
    NSH_LAUNCHED();
    const float* lhs[2] = {P, G};
    const float* rhs[2] = {dO + q0 * ld, Q + q0 * ld};
    float* out[2] = {dV, dK};
    for (int i = 0; i < 2; i++) {
      GemmArgs t;
      t.A = lhs[i]; t.lda = S; t.sA = nq * S;
      t.B = rhs[i]; t.ldb = ld; t.sB = dk;
      t.C = out[i]; t.ldc = ld; t.sC = dk;
      t.M = (int)S; t.N = (int)dk; t.K = (int)nq;
      t.mode = q0 == 0 ? kEpiAct : kEpiAccum;
      if (launch_gemm_ex(t, true, false, (int)H, s)) return -1;
    }
    GemmArgs q = wide_pv_args(nq, S, dk);
    q.A = G; q.lda = S; q.sA = nq * S;
    q.B = K; q.ldb = ld; q.sB = dk;
    q.C = dQ + q0 * ld; q.ldc = ld; q.sC = dk;
    if (launch_gemm_split(q, false, false, (int)H, gemm_split_count(q, (int)H), ws + wide_score_floats(S, H, true), s))
      return -1;
  }
  return 0;
}

bool attention_in_place(int64_t D, int64_t H, int64_t ld, const void* const* ptrs, int n) {
  if (H <= 0 || D % H != 0 || ld % 4 != 0) return false;
  const int64_t dk = D / H;
  if (dk != 32 && dk != 64 && dk != 128) return false;
  for (int i = 0; i < n; i++)
    if ((uintptr_t)ptrs[i] % 16 != 0) return false;
  return true;
}

size_t attention_pad_floats(int64_t S, int64_t D, int64_t H, bool backward) {
  if (S <= 0 || H <= 0 || D % H != 0) return 0;
  const int64_t dkp = padded_dk(D / H);
  // wide path: the score block, and in the backward its gradient
  if (!dkp) return (size_t)wide_score_floats(S, H, backward) + wide_split_floats(S, H, D / H);
  // forward: Q K V ctx; backward: Q K V O dO dQ dK dV
  return (size_t)((backward ? 8 : 4) * S * H * dkp);
}

static int pad_copy(const float* src, int64_t ld, float* dst, int64_t S, int64_t H, int64_t dk, int64_t dkp,
                    hipStream_t s) {
  const unsigned g = (unsigned)std::min<int64_t>(ceil_div(S * H * dkp, 256), 16384);
  hipLaunchKernelGGL(attn_pad_kernel, dim3(g), dim3(256), 0, s, src, ld, dst, (int)S, (int)H, (int)dk, (int)dkp);
  NSH_LAUNCHED();
  return 0;
}

static int unpad_copy(const float* src, float* dst, int64_t ld, int64_t S, int64_t H, int64_t dk, int64_t dkp,
                      hipStream_t s) {
  const unsigned g = (unsigned)std::min<int64_t>(ceil_div(S * H * dk, 256), 16384);
  hipLaunchKernelGGL(attn_unpad_kernel, dim3(g), dim3(256), 0, s, src, dst, ld, (int)S, (int)H, (int)dk, (int)dkp);
  NSH_LAUNCHED();
  return 0;
}

template <int DK>
static void flash_fwd(const float* Q, const float* K, const float* V, float* ctx, float* lse, int64_t S, int64_t H,
                      int64_t ld, float scale, hipStream_t s) {
  const int nqb = (int)ceil_div(S, 32 * kFW);
  hipLaunchKernelGGL(flash_fwd_kernel<DK>, dim3(nqb * (unsigned)H), dim3(64 * kFW), 0, s, Q, K, V, ctx, lse, (int)S,
                     (int)H, ld, scale * 1.4426950408889634f, nqb);
}

int launch_attention_fwd(const float* Q, const float* K, const float* V, float* ctx, float* lse, int64_t S, int64_t D,
                         int64_t H, int64_t ld, float* pad_ws, hipStream_t s) {
  if (S <= 0) return 0;
  if (H <= 0 || D % H != 0 || S > INT32_MAX) {
    set_error("attention: bad shape");
    return -1;
  }
  const int64_t DK = D / H;
  const float scale = 1.0f / sqrtf((float)DK);
  const void* ptrs[3] = {Q, K, V};  // read as float4 rows
  if (attention_in_place(D, H, ld, ptrs, 3)) {
    if (DK == 128) flash_fwd<128>(Q, K, V, ctx, lse, S, H, ld, scale, s);
    else if (DK == 64) flash_fwd<64>(Q, K, V, ctx, lse, S, H, ld, scale, s);
    else flash_fwd<32>(Q, K, V, ctx, lse, S, H, ld, scale, s);
    NSH_LAUNCHED();
    return 0;
  }
  const int64_t dkp = padded_dk(DK);
  if (!pad_ws) {
    set_error(dkp ? "attention: this head size or alignment needs the padding workspace"
                  : "attention: head sizes above 128 need the score workspace");
    return -1;
  }
  if (!dkp) return wide_fwd(Q, K, V, ctx, lse, S, H, DK, ld, scale, pad_ws, s);
  const int64_t ldp = H * dkp, n = S * ldp;
  float *Qp = pad_ws, *Kp = pad_ws + n, *Vp = pad_ws + 2 * n, *Op = pad_ws + 3 * n;
  if (pad_copy(Q, ld, Qp, S, H, DK, dkp, s) || pad_copy(K, ld, Kp, S, H, DK, dkp, s) ||
      pad_copy(V, ld, Vp, S, H, DK, dkp, s))
    return -1;
  if (dkp == 128) flash_fwd<128>(Qp, Kp, Vp, Op, lse, S, H, ldp, scale, s);
  else if (dkp == 64) flash_fwd<64>(Qp, Kp, Vp, Op, lse, S, H, ldp, scale, s);
  else flash_fwd<32>(Qp, Kp, Vp, Op, lse, S, H, ldp, scale, s);
  NSH_LAUNCHED();
  return unpad_copy(Op, ctx, ld, S, H, DK, dkp, s);
}

size_t attention_bwd_ds_floats(int64_t S, int64_t D, int64_t H) {
  if (S <= 0 || H <= 0 || D % H != 0 || S % kBK != 0 || !padded_dk(D / H)) return 0;
  const double bytes = 4.0 * (double)H * (double)S * (double)S;
  if (bytes > 16.0 * 1024 * 1024 * 1024) return 0;  // recompute beyond 16 GiB
  return (size_t)(H * S * S);
}

// The backward kernels of one tile width on arrays of row pitch ld.
template <int DK>
static int flash_bwd(const float* Q, const float* K, const float* V, const float* O, const float* dO,
                     const float* lse, float* delta, float* dQ, float* dK, float* dV, int64_t S, int64_t H,
                     int64_t ld, float scale, float* ds_ws, hipStream_t s) {
  const float cl2 = scale * 1.4426950408889634f;
  hipLaunchKernelGGL(attn_delta_rows_kernel<DK>, dim3((unsigned)ceil_div(S, 4)), dim3(256), 0, s, dO, O, delta,
                     (int)S, (int)H, ld);
  NSH_LAUNCHED();
  const int nb = (int)ceil_div(S, kBQ);
  const dim3 grid(nb * (unsigned)H), block(256);
  if (ds_ws) {
    hipLaunchKernelGGL((flash_bwd_dkdv_kernel<DK, true>), grid, block, 0, s, Q, K, V, dO, lse, delta, dK, dV, ds_ws,
                       (int)S, (int)H, ld, scale, cl2, nb);
    hipLaunchKernelGGL(flash_bwd_dq_ds_kernel<DK>, grid, block, 0, s, K, ds_ws, dQ, (int)S, (int)H, ld, scale, nb);
  } else {
    hipLaunchKernelGGL((flash_bwd_dkdv_kernel<DK, false>), grid, block, 0, s, Q, K, V, dO, lse, delta, dK, dV,
                       nullptr, (int)S, (int)H, ld, scale, cl2, nb);
    hipLaunchKernelGGL(flash_bwd_dq_kernel<DK>, grid, block, 0, s, Q, K, V, dO, lse, delta, dQ, (int)S, (int)H, ld,
                       scale, cl2, nb);
  }
  NSH_LAUNCHED();
  return 0;
}

template <typename... A>
static int flash_bwd_any(int64_t dk, A... a) {
  return dk == 128 ? flash_bwd<128>(a...) : dk == 64 ? flash_bwd<64>(a...) : flash_bwd<32>(a...);
}

int launch_attention_bwd(const float* Q, const float* K, const float* V, const float* O, const float* dO,
                         const float* lse, float* delta, float* dQ, float* dK, float* dV, int64_t S, int64_t D,
                         int64_t H, int64_t ld, float* ds_ws, float* pad_ws, hipStream_t s) {
  if (S <= 0) return 0;
  if (H <= 0 || D % H != 0 || S > INT32_MAX) {
    set_error("attention backward: bad shape");
    return -1;
  }
  const int64_t DK = D / H;
  const float scale = 1.0f / sqrtf((float)DK);
  float* ds = ds_ws && attention_bwd_ds_floats(S, D, H) > 0 && ((uintptr_t)ds_ws % 16) == 0 ? ds_ws : nullptr;
  const void* ptrs[5] = {Q, K, V, O, dO};  // read as float4 rows
  if (attention_in_place(D, H, ld, ptrs, 5))
    return flash_bwd_any(DK, Q, K, V, O, dO, lse, delta, dQ, dK, dV, S, H, ld, scale, ds, s);
  const int64_t dkp = padded_dk(DK);
  if (!pad_ws) {
    set_error(dkp ? "attention backward: this head size or alignment needs the padding workspace"
                  : "attention backward: head sizes above 128 need the score workspace");
    return -1;
  }
  if (!dkp) return wide_bwd(Q, K, V, dO, dQ, dK, dV, S, H, DK, ld, scale, pad_ws, s);
  const int64_t ldp = H * dkp, n = S * ldp;
  float* p[8];
  for (int i = 0; i < 8; i++) p[i] = pad_ws + i * n;
  const float* src[5] = {Q, K, V, O, dO};
  for (int i = 0; i < 5; i++)
    if (pad_copy(src[i], ld, p[i], S, H, DK, dkp, s) != 0) return -1;
  if (flash_bwd_any(dkp, p[0], p[1], p[2], p[3], p[4], lse, delta, p[5], p[6], p[7], S, H, ldp, scale, ds, s) != 0)
    return -1;
  float* dst[3] = {dQ, dK, dV};
  for (int i = 0; i < 3; i++)
    if (unpad_copy(p[5 + i], dst[i], ld, S, H, DK, dkp, s) != 0) return -1;
  return 0;
}

}  // namespace nship
