// Multi-head self-attention core over one sequence (S = all rows of the
// call, as the reference does: codegen.cpp:2224-2235, S = BS), flash-style:
// no S x S matrix is ever materialised.
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
#include "common.h"
#include "kernels.h"

namespace nship {

typedef float floatx16 __attribute__((ext_vector_type(16)));

namespace {

constexpr int kBQ = 128;  // queries per workgroup
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

  __device__ void load(const float* __restrict__ K, const float* __restrict__ V, int64_t ld, int hcol, int key0,
                       int S, int t) {
#pragma unroll
    for (int i = 0; i < kPer; i++) {
      const int idx = t + 256 * i;
      const int key = idx / (DK / 4), c = (idx % (DK / 4)) * 4;
      const int gk = key0 + key;
      if (gk < S) {
        k[i] = *reinterpret_cast<const float4*>(K + (int64_t)gk * ld + hcol + c);
        v[i] = *reinterpret_cast<const float4*>(V + (int64_t)gk * ld + hcol + c);
      } else {
        k[i] = make_float4(0.f, 0.f, 0.f, 0.f);
        v[i] = k[i];
      }
    }
  }
  __device__ void store(float* __restrict__ ks, int t) const {
    float* vs = ks + kFloats;
#pragma unroll
    for (int i = 0; i < kPer; i++) {
      const int idx = t + 256 * i;
      const int key = idx / (DK / 4), c = (idx % (DK / 4)) * 4;
      *reinterpret_cast<float4*>(ks + key * P + c) = k[i];
      *reinterpret_cast<float4*>(vs + key * P + c) = v[i];
    }
  }
};

template <int DK>
__global__ __launch_bounds__(256) void flash_fwd_kernel(const float* __restrict__ Q, const float* __restrict__ K,
                                                        const float* __restrict__ V, float* __restrict__ ctx,
                                                        float* __restrict__ lse, int S, int H, int64_t ld,
                                                        float scale_log2, int nqb) {
  using Tile = KVTile<DK>;
  constexpr int NS = DK / 2;    // MFMA steps of the score product
  constexpr int NDB = DK / 32;  // 32-wide head-dim blocks of the output
  __shared__ __attribute__((aligned(16))) float sm[2 * 2 * Tile::kFloats];

  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int l32 = lane & 31, kh = lane >> 5;
  const int L = remap_xcd(blockIdx.x, nqb * H);
  const int h = L / nqb, q0 = (L % nqb) * kBQ;
  const int hcol = h * DK;
  const int qrow = q0 + w * 32 + l32;

  // B operand of S^T = K Q^T: this lane's query, head dims 8g + 4kh + (0..3).
  float qf[NS];
#pragma unroll
  for (int g = 0; g < DK / 8; g++) {
    float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
    if (qrow < S) x = *reinterpret_cast<const float4*>(Q + (int64_t)qrow * ld + hcol + 8 * g + 4 * kh);
    qf[4 * g] = x.x; qf[4 * g + 1] = x.y; qf[4 * g + 2] = x.z; qf[4 * g + 3] = x.w;
  }

  floatx16 o[NDB];
#pragma unroll
  for (int d = 0; d < NDB; d++)
#pragma unroll
    for (int v = 0; v < 16; v++) o[d][v] = 0.f;
  float m = -INFINITY, l = 0.f;

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

    floatx16 sc[2];
#pragma unroll
    for (int kb = 0; kb < 2; kb++)
#pragma unroll
      for (int v = 0; v < 16; v++) sc[kb][v] = 0.f;
#pragma unroll
    for (int g = 0; g < DK / 8; g++)
#pragma unroll
      for (int kb = 0; kb < 2; kb++) {
        const float4 kv = *reinterpret_cast<const float4*>(ks + (kb * 32 + l32) * Tile::P + 8 * g + 4 * kh);
        sc[kb] = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.x, qf[4 * g + 0], sc[kb], 0, 0, 0);
        sc[kb] = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.y, qf[4 * g + 1], sc[kb], 0, 0, 0);
        sc[kb] = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.z, qf[4 * g + 2], sc[kb], 0, 0, 0);
        sc[kb] = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.w, qf[4 * g + 3], sc[kb], 0, 0, 0);
      }

    // Online softmax for this lane's query (keys 8*(v/4) + 4kh + v%4 of each block).
    const int kbase = it * kBK;
    float mloc = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; kb++)
#pragma unroll
      for (int v = 0; v < 16; v++) {
        const int key = kbase + kb * 32 + 8 * (v >> 2) + 4 * kh + (v & 3);
        const float x = key < S ? sc[kb][v] * scale_log2 : -INFINITY;
        sc[kb][v] = x;
        mloc = fmaxf(mloc, x);
      }
    mloc = fmaxf(mloc, __shfl_xor(mloc, 32, 64));
    const float mnew = fmaxf(m, mloc);
    const float corr = exp2f(m - mnew);
    float lsum = 0.f;
#pragma unroll
    for (int kb = 0; kb < 2; kb++)
#pragma unroll
      for (int v = 0; v < 16; v++) {
        const float p = exp2f(sc[kb][v] - mnew);
        sc[kb][v] = p;
        lsum += p;
      }
    lsum += __shfl_xor(lsum, 32, 64);
    l = l * corr + lsum;
    m = mnew;
#pragma unroll
    for (int d = 0; d < NDB; d++)
#pragma unroll
      for (int v = 0; v < 16; v++) o[d][v] *= corr;

    // O^T += V^T P^T: step s of key block kb pairs key 8*(s/4)+4kh+s%4.
#pragma unroll
    for (int kb = 0; kb < 2; kb++)
#pragma unroll
      for (int s = 0; s < 16; s++) {
        const int key = kb * 32 + 8 * (s >> 2) + 4 * kh + (s & 3);
#pragma unroll
        for (int d = 0; d < NDB; d++)
          o[d] = __builtin_amdgcn_mfma_f32_32x32x2f32(vs[key * Tile::P + d * 32 + l32], sc[kb][s], o[d], 0, 0, 0);
      }

    if (more) tile.store(sm + (cur ^ 1) * 2 * Tile::kFloats, t);
    __syncthreads();
  }

  // Row statistics for the backward pass: log2-sum-exp of the scaled scores.
  if (lse && kh == 0 && qrow < S) lse[(int64_t)h * S + qrow] = m + log2f(l);

  // O^T (d, query) / l  ->  LDS [query][d]  ->  coalesced rows of ctx.
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

// Any head size up to 128: one thread per (query, head), two passes over
// the keys.  Used for small test networks; not a performance path.
__global__ __launch_bounds__(64) void attention_fwd_small_kernel(const float* __restrict__ Q,
                                                                 const float* __restrict__ K,
                                                                 const float* __restrict__ V, float* __restrict__ ctx,
                                                                 float* __restrict__ lse, int S, int H, int DK,
                                                                 int64_t ld, float scale) {
  const int64_t gid = (int64_t)blockIdx.x * 64 + threadIdx.x;
  if (gid >= (int64_t)S * H) return;
  const int q = (int)(gid / H), h = (int)(gid % H);
  const float* qr = Q + (int64_t)q * ld + h * DK;
  float mx = -INFINITY;
  for (int j = 0; j < S; j++) {
    const float* kr = K + (int64_t)j * ld + h * DK;
    float a = 0.f;
    for (int d = 0; d < DK; d++) a += qr[d] * kr[d];
    mx = fmaxf(mx, a * scale);
  }
  float acc[128];
  for (int d = 0; d < DK; d++) acc[d] = 0.f;
  float sum = 0.f;
  for (int j = 0; j < S; j++) {
    const float* kr = K + (int64_t)j * ld + h * DK;
    float a = 0.f;
    for (int d = 0; d < DK; d++) a += qr[d] * kr[d];
    const float p = expf(a * scale - mx);
    sum += p;
    const float* vr = V + (int64_t)j * ld + h * DK;
    for (int d = 0; d < DK; d++) acc[d] += p * vr[d];
  }
  float* o = ctx + (int64_t)q * ld + h * DK;
  for (int d = 0; d < DK; d++) o[d] = acc[d] / sum;
  // same convention as the flash kernel: log2-sum-exp of scores * scale * log2(e)
  if (lse) lse[(int64_t)h * S + q] = mx * 1.4426950408889634f + log2f(sum);
}

}  // namespace

int launch_attention_fwd(const float* Q, const float* K, const float* V, float* ctx, float* lse, int64_t S, int64_t D,
                         int64_t H, int64_t ld, hipStream_t s) {
  if (S <= 0) return 0;
  if (H <= 0 || D % H != 0 || S > INT32_MAX) {
    set_error("attention: bad shape");
    return -1;
  }
  const int64_t DK = D / H;
  const float scale = 1.0f / sqrtf((float)DK);
  const bool aligned = ld % 4 == 0 && ((uintptr_t)Q | (uintptr_t)K | (uintptr_t)V) % 16 == 0;
  if (aligned && (DK == 64 || DK == 32)) {
    const int nqb = (int)ceil_div(S, kBQ);
    const dim3 grid(nqb * (unsigned)H), block(256);
    const float sl2 = scale * 1.4426950408889634f;
    if (DK == 64)
      hipLaunchKernelGGL(flash_fwd_kernel<64>, grid, block, 0, s, Q, K, V, ctx, lse, (int)S, (int)H, ld, sl2, nqb);
    else
      hipLaunchKernelGGL(flash_fwd_kernel<32>, grid, block, 0, s, Q, K, V, ctx, lse, (int)S, (int)H, ld, sl2, nqb);
  } else {
    if (DK > 128) {
      set_error("attention: head size above 128 is not supported");
      return -1;
    }
    hipLaunchKernelGGL(attention_fwd_small_kernel, dim3((unsigned)ceil_div(S * H, 64)), dim3(64), 0, s, Q, K, V, ctx,
                       lse, (int)S, (int)H, (int)DK, ld, scale);
  }
  NSH_LAUNCHED();
  return 0;
}

}  // namespace nship
