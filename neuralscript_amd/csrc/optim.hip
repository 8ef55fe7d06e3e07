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
// MGS on the GPU, right-looking and blocked in panels of kPB vectors.  Every
// vector receives the same projections in the same order as in the
// reference's loop (q_0, q_1, ... q_{c-1}, then its own normalisation
// v / (|v| + 1e-30)); only the order inside each dot product differs (per
// thread partial sums, then a fixed tree of DPP row sums and one LDS
// exchange).  One launch per panel: launch p applies the projections of
// panel p to every later vector, kPB vectors per workgroup held in
// registers, and the workgroup that owns panel p+1 then factorizes it in
// registers and stores its normalised q vectors.  All Muon matrices of the
// step advance together in the same launches; each workgroup spreads its
// vectors over the 1024 threads according to its own matrix's length.  Vectors live
// contiguously in a work buffer T[C][R] (a transpose of g when r >= c).
// Vectors longer than kMaxPanelR take the sliced path: every vector is cut
// into slices of kSliceLen elements, one workgroup per slice, and the
// columns go in panels of kSlicePanel.  Inside a panel, one launch per
// column j turns column j's per-slice partial sums (written by the previous
// launch) into |v_j| and the dots, normalises q_j, projects it out of the
// panel's later vectors in order and writes the partial sums of column j + 1
// (MGS, one grid-wide exchange per column).  The finished panel then
// projects out of every later vector at once, block Gram-Schmidt: the raw
// dots q_k . v_c of each panel vector with each later vector (per slice, then
// summed in a fixed order), then v_c -= sum_k (q_k . v_c) q_k, k ascending --
// each later vector is streamed three times per panel instead of twice per
// column.  Only the order of the cross-panel projections differs from the
// reference's MGS (the dots are taken from the vector before the panel), so
// vectors well inside the gradient's span get the same q; nearly dependent
// ones normalise rounding residue either way.
#include "common.h"
#include "kernels.h"

namespace nship {
namespace {

constexpr int kSliceThreads = 256;                        // sliced path: threads per workgroup
constexpr int kSliceEPT = 8;                              // elements of a vector per thread
constexpr int kSliceLen = kSliceThreads * kSliceEPT;      // elements per slice
constexpr int kSliceBatch = 8;                            // later vectors per block reduction
constexpr int kSlicePanel = 8;                            // columns per panel of the sliced path
constexpr int kPB = 8;   // panel width (vectors per workgroup, panel path)
// Panel path: 8 waves of up to 16 elements per vector a thread.  Fewer,
// fuller waves keep the block reductions of the lead chain short: every wave
// repeats a reduction's tail, so its cost grows with the wave count while the
// element work per workgroup does not.
constexpr int kPanelThreads = 512;
constexpr int kPanelWaves = kPanelThreads / 64;
constexpr int kMaxPanelR = 16 * kPanelThreads;

// x / d for a divisor d shared by many quotients, given rd = 1 / d (one
// correctly rounded division): q = x rd, then one correction q + (x - q d) rd
// with fused multiply-adds (Markstein's corrected quotient, P. Markstein,
// "IA-64 and Elementary Functions", 2000).  With x, d and the quotient normal
// it is the correctly rounded quotient, the value of x / d, at three
// instructions instead of a full division each; a subnormal quotient may
// differ from it in the last place.
__device__ __forceinline__ float div_shared(float x, float d, float rd) {
  const float q = x * rd;
  return __builtin_fmaf(__builtin_fmaf(-q, d, x), rd, q);
}

// One AdamW element (codegen.cpp:1617-1633), contraction off so every
// product and sum rounds as the reference's scalar code does.
__device__ __forceinline__ void adamw_elem(float& w, float gg, float& m, float& v, float lr, float b1t, float b2t) {
#pragma clang fp contract(off)
  const float mi = 0.9f * m + 0.1f * gg;
  const float vi = 0.999f * v + 0.001f * gg * gg;
  m = mi;
  v = vi;
  const float mh = mi / b1t, vh = vi / b2t;
  w = w - ((lr * mh / (sqrtf(vh) + 1e-8f)) + (0.01f * lr) * w);
}

// VEC: thread i updates elements 4i..4i+3 with float4 loads and stores (all
// four arrays 16-byte aligned; the n % 4 tail goes to the first threads);
// else one element per thread.
template <bool VEC>
__global__ __launch_bounds__(256) void adamw_kernel(float* __restrict__ w, const float* __restrict__ g,
                                                    float* __restrict__ m, float* __restrict__ v, int64_t n, float lr,
                                                    float b1t, float b2t) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if constexpr (VEC) {
    const int64_t n4 = n / 4;
    if (i < n4) {
      const fvec4 w4 = ((gfloat4*)as_global(w))[i], m4 = ((gfloat4*)as_global(m))[i];
      const fvec4 v4 = ((gfloat4*)as_global(v))[i], g4 = ((const gfloat4*)as_global(g))[i];
      float W[4] = {w4.x, w4.y, w4.z, w4.w}, Mo[4] = {m4.x, m4.y, m4.z, m4.w}, Vo[4] = {v4.x, v4.y, v4.z, v4.w};
      const float G[4] = {g4.x, g4.y, g4.z, g4.w};
#pragma unroll
      for (int e = 0; e < 4; e++) adamw_elem(W[e], G[e], Mo[e], Vo[e], lr, b1t, b2t);
      ((gfloat4*)as_global(m))[i] = fvec4{Mo[0], Mo[1], Mo[2], Mo[3]};
      ((gfloat4*)as_global(v))[i] = fvec4{Vo[0], Vo[1], Vo[2], Vo[3]};
      ((gfloat4*)as_global(w))[i] = fvec4{W[0], W[1], W[2], W[3]};
    }
    const int64_t t = 4 * n4 + i;
    if (i < 4 && t < n) adamw_elem(w[t], g[t], m[t], v[t], lr, b1t, b2t);
  } else {
    if (i < n) adamw_elem(w[i], g[i], m[i], v[i], lr, b1t, b2t);
  }
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

// float4 access needs R and C multiples of 4 and 16-byte aligned bases (the
// blob's matrices start anywhere a float can).
__device__ __forceinline__ bool vec4_ok(int64_t R, int64_t C, const void* a, const void* b) {
  return ((R | C) & 3) == 0 && (((uintptr_t)a | (uintptr_t)b) & 15) == 0;
}

// T = the vectors of g, contiguous: r < c, the rows (a copy); r >= c, the
// columns, T[j][k] = g[k][j], transposed through LDS so both sides are read
// and written along rows: 64 x 128 tiles with float4 on both sides (the odd
// LDS row pitch of 129 keeps the column reads conflict-free), or 32 x 32
// scalar tiles where float4 does not fit.  grid.y = matrix.
__global__ __launch_bounds__(256) void muon_gather_kernel(const MuonMat* __restrict__ mats, int nmat) {
  __shared__ float tile[64 * 129];
  const MuonMat& M = mats[blockIdx.y];
  const gfloat* __restrict__ g = as_global(M.g);
  gfloat* __restrict__ T = as_global(M.T);
  const int64_t R = M.R, C = M.C;
  const bool vec = vec4_ok(R, C, M.g, M.T);
  if (M.transposed) {
    if (vec) {
      const gfloat4* g4 = (const gfloat4*)g;
      gfloat4* T4 = (gfloat4*)T;
      for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < R * C / 4; i += (int64_t)gridDim.x * 256)
        T4[i] = g4[i];
    } else {
      for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < R * C; i += (int64_t)gridDim.x * 256)
        T[i] = g[i];
    }
    return;
  }
  if (vec) {
    // 64 (k) x 128 (j) tiles: each g row segment read is 512 contiguous
    // bytes and all 8 float4 loads of a thread are in flight together.
    // Thread: float4 column q (of 16 per 64-wide half row), rows rr + 16 i.
    const int q = threadIdx.x & 15, rr = threadIdx.x >> 4;
    const int64_t tc = (C + 127) / 128, tiles = ((R + 63) / 64) * tc;
    for (int64_t b = blockIdx.x; b < tiles; b += gridDim.x) {
      const int64_t k0 = (b / tc) * 64, j0 = (b % tc) * 128;
      fvec4 x[4][2];
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int hh = 0; hh < 2; hh++) {
          const int r = rr + 16 * i, jc = 64 * hh + 4 * q;
          x[i][hh] = (k0 + r < R && j0 + jc < C) ? *(const gfloat4*)(g + (k0 + r) * C + j0 + jc)
                                                 : fvec4{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int hh = 0; hh < 2; hh++) {
          float* t = tile + (rr + 16 * i) * 129 + 64 * hh + 4 * q;
          t[0] = x[i][hh].x, t[1] = x[i][hh].y, t[2] = x[i][hh].z, t[3] = x[i][hh].w;
        }
      __syncthreads();
#pragma unroll
      for (int i = 0; i < 8; i++) {
        const int jj = rr + 16 * i;
        if (j0 + jj < C && k0 + 4 * q < R) {
          const float* t = tile + 4 * q * 129 + jj;
          fvec4 y;
          y.x = t[0], y.y = t[129], y.z = t[258], y.w = t[387];
          *(gfloat4*)(T + (j0 + jj) * R + k0 + 4 * q) = y;
        }
      }
      __syncthreads();
    }
    return;
  }
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
  const int64_t tc = (C + 31) / 32, tiles = ((R + 31) / 32) * tc;
  for (int64_t b = blockIdx.x; b < tiles; b += gridDim.x) {
    const int64_t k0 = (b / tc) * 32, j0 = (b % tc) * 32;
    for (int r = ty; r < 32; r += 8)
      if (k0 + r < R && j0 + tx < C) tile[r * 33 + tx] = g[(k0 + r) * C + j0 + tx];
    __syncthreads();
    for (int r = ty; r < 32; r += 8)
      if (j0 + r < C && k0 + tx < R) T[(j0 + r) * R + k0 + tx] = tile[tx * 33 + r];
    __syncthreads();
  }
  (void)nmat;
}

__host__ __device__ __forceinline__ int mgs_slices(int64_t R) { return (int)((R + kSliceLen - 1) / kSliceLen); }

// Sum of the nsl per-slice partials at p, in a fixed order (lane-strided
// sums, then the xor butterfly): every wave of every workgroup gets the
// same bits.
__device__ __forceinline__ float slice_total(const float* __restrict__ p, int nsl) {
  const int lane = threadIdx.x & 63;
  float a = 0.f;
  for (int i = lane; i < nsl; i += 64) a += p[i];
  return wave_sum(a);
}

// The workgroup's long matrix (R > kMaxPanelR) and slice of it; false past
// the last long matrix's slices.
__device__ __forceinline__ bool slice_of(const MuonMat* __restrict__ mats, int nmat, int& mi, int& b) {
  b = blockIdx.x;
  for (mi = 0; mi < nmat; mi++) {
    const int n = mats[mi].R > kMaxPanelR ? mgs_slices(mats[mi].R) : 0;
    if (b < n) return true;
    b -= n;
  }
  return false;
}

// A thread's share of one slice of the vectors T[c][0..R): kSliceEPT
// elements, float4 groups when the rows allow (R % 4 == 0, 16-byte aligned).
// Vector c is T's vector lv[c] when a list lv is given (the nonzero
// vectors, in order), else vector c itself.
struct SliceIO {
  gfloat* __restrict__ T;
  int R;
  bool vec;
  int64_t s0;
  int t;
  const int* __restrict__ lv;
  __device__ SliceIO(const MuonMat& M, int b, const int* list = nullptr)
      : T(as_global(M.T)), R(M.R), vec(M.R % 4 == 0 && (reinterpret_cast<uintptr_t>(M.T) & 15) == 0),
        s0((int64_t)b * kSliceLen), t(threadIdx.x), lv(list) {}
  __device__ int64_t at(int e) const {
    return vec ? s0 + 4 * (t + kSliceThreads * (e >> 2)) + (e & 3) : s0 + t + kSliceThreads * e;
  }
  __device__ int64_t base(int c) const {
    return (int64_t)(lv ? __builtin_amdgcn_readfirstlane(lv[c]) : c) * R;  // c is the same in every lane
  }
  __device__ void load(int c, float (&x)[kSliceEPT]) const {
    const gfloat* row = T + base(c);
    if (vec) {
#pragma unroll
      for (int i = 0; i < kSliceEPT / 4; i++) {
        const int64_t k = at(4 * i);
        fvec4 v = {0.f, 0.f, 0.f, 0.f};
        if (k < R) v = *reinterpret_cast<const gfloat4*>(row + k);
        x[4 * i] = v.x; x[4 * i + 1] = v.y; x[4 * i + 2] = v.z; x[4 * i + 3] = v.w;
      }
    } else {
#pragma unroll
      for (int e = 0; e < kSliceEPT; e++) x[e] = at(e) < R ? row[at(e)] : 0.f;
    }
  }
  __device__ void store(int c, const float (&x)[kSliceEPT]) const {
    gfloat* row = T + base(c);
    if (vec) {
#pragma unroll
      for (int i = 0; i < kSliceEPT / 4; i++) {
        const int64_t k = at(4 * i);
        if (k < R) *reinterpret_cast<gfloat4*>(row + k) = fvec4{x[4 * i], x[4 * i + 1], x[4 * i + 2], x[4 * i + 3]};
      }
    } else {
#pragma unroll
      for (int e = 0; e < kSliceEPT; e++)
        if (at(e) < R) row[at(e)] = x[e];
    }
  }
};

// Workspace of a long matrix (M.red): column partials [2][C][nsl], the
// panel's raw dots per slice [kSlicePanel][C][nsl], and their totals
// [kSlicePanel][C].
__device__ __forceinline__ float* slice_dots(const MuonMat& M) { return M.red + (size_t)2 * M.C * mgs_slices(M.R); }
__device__ __forceinline__ float* slice_dot_totals(const MuonMat& M) {
  return slice_dots(M) + (size_t)kSlicePanel * M.C * mgs_slices(M.R);
}
// Then the vectors' liveness: per slice a bit mask of the vectors nonzero
// in it [nsl][ceil(C / 32)], the number of nonzero vectors, and their list.
__device__ __forceinline__ int slice_words(const MuonMat& M) { return (M.C + 31) >> 5; }
__device__ __forceinline__ unsigned* slice_masks(const MuonMat& M) {
  return reinterpret_cast<unsigned*>(slice_dot_totals(M) + (size_t)kSlicePanel * M.C);
}
__device__ __forceinline__ int* slice_nlive(const MuonMat& M) {
  return reinterpret_cast<int*>(slice_masks(M) + (size_t)mgs_slices(M.R) * slice_words(M));
}
__device__ __forceinline__ const int* slice_list(const MuonMat& M) { return slice_nlive(M) + 1; }

// A zero vector stays zero and changes no other: every projection onto it
// and of it is 0 * q, and it normalises to 0 / (0 + 1e-30) = 0 (a gradient
// of MoE expert weights holds zero rows for the experts without tokens).
// The sliced launches therefore run over the nonzero vectors only, in
// order (c indexes that list, slice_list), and leave the zero ones as they
// are.  First each slice's mask of the vectors nonzero in it, 32 vectors a
// word: a thread's elements of 8 vectors in flight, the bits OR-reduced
// over the workgroup.
__global__ __launch_bounds__(kSliceThreads) void mgs_slice_live_kernel(const MuonMat* __restrict__ mats, int nmat) {
  __shared__ unsigned wbits[4];
  int mi, b;
  if (!slice_of(mats, nmat, mi, b)) return;
  const MuonMat& M = mats[mi];
  const SliceIO io(M, b);
  const int t = threadIdx.x, w = t >> 6, C = M.C, W = slice_words(M);
  unsigned* __restrict__ out = slice_masks(M) + (size_t)b * W;
  for (int wd = 0; wd < W; wd++) {
    unsigned bits = 0u;
    for (int i0 = 0; i0 < 32; i0 += 8) {
      float x[8][kSliceEPT];
#pragma unroll
      for (int u = 0; u < 8; u++) {
        const int c = 32 * wd + i0 + u;
        if (c < C) {
          io.load(c, x[u]);
        } else {
#pragma unroll
          for (int e = 0; e < kSliceEPT; e++) x[u][e] = 0.f;
        }
      }
#pragma unroll
      for (int u = 0; u < 8; u++) {
        bool nz = false;
#pragma unroll
        for (int e = 0; e < kSliceEPT; e++) nz |= x[u][e] != 0.f;
        if (nz) bits |= 1u << (i0 + u);
      }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) bits |= (unsigned)__shfl_xor((int)bits, o, 64);
    __syncthreads();  // the previous word's readers are done
    if ((t & 63) == 0) wbits[w] = bits;
    __syncthreads();
    if (t == 0) out[wd] = wbits[0] | wbits[1] | wbits[2] | wbits[3];
  }
}

// Per long matrix (blockIdx.x), one workgroup: the masks OR-ed over the
// slices, then the nonzero vectors' list in ascending order and its length
// (every vector when the words do not fit the workgroup's table).
constexpr int kLiveWords = 2048;
__global__ __launch_bounds__(256) void mgs_slice_list_kernel(const MuonMat* __restrict__ mats, int nmat) {
  __shared__ unsigned words[kLiveWords];
  __shared__ int offs[kLiveWords];
  const MuonMat& M = mats[blockIdx.x];
  if (M.R <= kMaxPanelR) return;
  const int t = threadIdx.x, C = M.C, W = slice_words(M), nsl = mgs_slices(M.R);
  int* __restrict__ nlive = slice_nlive(M);
  int* __restrict__ list = nlive + 1;
  if (W > kLiveWords) {
    for (int c = t; c < C; c += 256) list[c] = c;
    if (t == 0) *nlive = C;
    return;
  }
  const unsigned* __restrict__ masks = slice_masks(M);
  if (W >= 64) {  // a thread per word
    for (int wd = t; wd < W; wd += 256) {
      unsigned m = 0u;
      for (int i = 0; i < nsl; i++) m |= masks[(size_t)i * W + wd];
      words[wd] = m;
    }
  } else {  // few words (few vectors), many slices: the slices over the threads
    __shared__ unsigned wpart[4];
    for (int wd = 0; wd < W; wd++) {
      unsigned m = 0u;
      for (int i = t; i < nsl; i += 256) m |= masks[(size_t)i * W + wd];
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) m |= (unsigned)__shfl_xor((int)m, o, 64);
      if ((t & 63) == 0) wpart[t >> 6] = m;
      __syncthreads();
      if (t == 0) words[wd] = wpart[0] | wpart[1] | wpart[2] | wpart[3];
      __syncthreads();
    }
  }
  __syncthreads();
  if (t == 0) {
    int o = 0;
    for (int wd = 0; wd < W; wd++) {
      offs[wd] = o;
      o += __popc(words[wd]);
    }
    *nlive = o;
  }
  __syncthreads();
  for (int wd = t; wd < W; wd += 256) {
    unsigned m = words[wd];
    int o = offs[wd];
    while (m) {
      const int i = __ffs(m) - 1;
      m &= m - 1;
      list[o++] = 32 * wd + i;
    }
  }
  (void)nmat;
}

// One column step of the sliced path inside a panel ending at column cend,
// over every long matrix; j = -1 only writes column 0's partials.
// Column partials: launch j reads buffer j & 1 and writes buffer (j + 1) & 1.
// The dots use the unnormalised v_j, dot_c = (v_j . v_c) / |v_j|, which
// equals q_j . v_c up to rounding; q_j itself is v_j / |v_j| element by
// element, as in the reference, and so is each projection v_c -= dot_c q_j.
__global__ __launch_bounds__(kSliceThreads) void mgs_slice_kernel(const MuonMat* __restrict__ mats, int nmat, int j,
                                                                  int cend) {
  __shared__ float red[4][kSliceBatch];
  int mi, b;
  if (!slice_of(mats, nmat, mi, b)) return;
  const MuonMat& M = mats[mi];
  const int C = M.C, nsl = mgs_slices(M.R), nlive = *slice_nlive(M), ce = min(nlive, cend);
  if (j >= nlive) return;
  const int t = threadIdx.x, w = t >> 6, lane = t & 63;
  const float* __restrict__ Pin = M.red + (size_t)(j & 1) * C * nsl;
  float* __restrict__ Pout = M.red + (size_t)((j + 1) & 1) * C * nsl;
  const SliceIO io(M, b, slice_list(M));

  float q[kSliceEPT], nrm = 1.f;
  if (j >= 0) {
    nrm = sqrtf(slice_total(Pin + (size_t)j * nsl, nsl)) + 1e-30f;
    const float rn = 1.f / nrm;
    io.load(j, q);
#pragma unroll
    for (int e = 0; e < kSliceEPT; e++) q[e] = div_shared(q[e], nrm, rn);
    io.store(j, q);
  }
  float piv[kSliceEPT];
  for (int c0 = j + 1; c0 < ce; c0 += kSliceBatch) {
    const int nb = min(kSliceBatch, ce - c0);
    float x[kSliceBatch][kSliceEPT], d[kSliceBatch];
#pragma unroll
    for (int u = 0; u < kSliceBatch; u++) {
      if (u < nb) {
        io.load(c0 + u, x[u]);
      } else {
#pragma unroll
        for (int e = 0; e < kSliceEPT; e++) x[u][e] = 0.f;
      }
      d[u] = j >= 0 && u < nb ? slice_total(Pin + (size_t)(c0 + u) * nsl, nsl) / nrm : 0.f;
    }
    if (j >= 0) {
#pragma unroll
      for (int u = 0; u < kSliceBatch; u++) {
        if (u >= nb) break;
#pragma unroll
        for (int e = 0; e < kSliceEPT; e++) x[u][e] -= d[u] * q[e];
        io.store(c0 + u, x[u]);
      }
    }
    if (c0 == j + 1) {
#pragma unroll
      for (int e = 0; e < kSliceEPT; e++) piv[e] = x[0][e];
    }
    // partial sums of column j + 1 over this slice: v_{j+1} . v_c, j + 1 <= c < ce
#pragma unroll
    for (int u = 0; u < kSliceBatch; u++) {
      float a = 0.f;
#pragma unroll
      for (int e = 0; e < kSliceEPT; e++) a += piv[e] * x[u][e];
      d[u] = wave_sum(a);
    }
    if (lane == 0) {
#pragma unroll
      for (int u = 0; u < kSliceBatch; u++) red[w][u] = d[u];
    }
    __syncthreads();
    if (t < nb) Pout[(size_t)(c0 + t) * nsl + b] = (red[0][t] + red[1][t]) + (red[2][t] + red[3][t]);
    __syncthreads();
  }
}

// The finished panel [j0, j0 + kSlicePanel) against every later vector:
// per slice, the raw dots q_k . v_c of each panel vector k with each vector
// c >= j0 + kSlicePanel, kDotBatch vectors at a time.
constexpr int kDotBatch = 4;
__global__ __launch_bounds__(kSliceThreads) void mgs_slice_dots_kernel(const MuonMat* __restrict__ mats, int nmat,
                                                                       int j0) {
  __shared__ float red[4][kDotBatch * kSlicePanel];
  int mi, b;
  if (!slice_of(mats, nmat, mi, b)) return;
  const MuonMat& M = mats[mi];
  const int C = M.C, nsl = mgs_slices(M.R), j1 = j0 + kSlicePanel, nlive = *slice_nlive(M);
  if (j1 >= nlive) return;
  const int t = threadIdx.x, w = t >> 6, lane = t & 63;
  const SliceIO io(M, b, slice_list(M));
  float* __restrict__ pd = slice_dots(M);
  float q[kSlicePanel][kSliceEPT];
#pragma unroll
  for (int k = 0; k < kSlicePanel; k++) io.load(j0 + k, q[k]);
  for (int c0 = j1; c0 < nlive; c0 += kDotBatch) {
    const int nb = min(kDotBatch, nlive - c0);
    float x[kDotBatch][kSliceEPT];
#pragma unroll
    for (int u = 0; u < kDotBatch; u++) {
      if (u < nb) {
        io.load(c0 + u, x[u]);
      } else {
#pragma unroll
        for (int e = 0; e < kSliceEPT; e++) x[u][e] = 0.f;
      }
    }
#pragma unroll
    for (int u = 0; u < kDotBatch; u++)
#pragma unroll
      for (int k = 0; k < kSlicePanel; k++) {
        float a = 0.f;
#pragma unroll
        for (int e = 0; e < kSliceEPT; e++) a += q[k][e] * x[u][e];
        a = wave_sum(a);
        if (lane == 0) red[w][u * kSlicePanel + k] = a;
      }
    __syncthreads();
    if (t < nb * kSlicePanel) {
      const int u = t / kSlicePanel, k = t % kSlicePanel;
      pd[((size_t)k * C + c0 + u) * nsl + b] = (red[0][t] + red[1][t]) + (red[2][t] + red[3][t]);
    }
    __syncthreads();
  }
}

// Totals of the panel's raw dots over the slices (slice_total's fixed
// order): one wave per (panel vector k, later vector c); blockIdx.y picks
// the matrix.
__global__ __launch_bounds__(256) void mgs_slice_reduce_kernel(const MuonMat* __restrict__ mats, int nmat, int j0) {
  const MuonMat& M = mats[blockIdx.y];
  if (M.R <= kMaxPanelR) return;
  const int C = M.C, nsl = mgs_slices(M.R), j1 = j0 + kSlicePanel, nlive = *slice_nlive(M);
  const int p = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int k = p / C, c = p % C;
  if (j1 >= nlive || k >= kSlicePanel || c < j1 || c >= nlive) return;
  const float v = slice_total(slice_dots(M) + ((size_t)k * C + c) * nsl, nsl);
  if ((threadIdx.x & 63) == 0) slice_dot_totals(M)[(size_t)k * C + c] = v;
  (void)nmat;
}

// The panel's projections applied to every later vector, v_c -= sum_k d_kc
// q_k (k ascending; every d_kc from the vector before this panel, as block
// Gram-Schmidt takes them), and the column partials of the next panel's
// first step (v_j1 . v_c for the next panel's vectors) into buffer j1 & 1.
__global__ __launch_bounds__(kSliceThreads) void mgs_slice_update_kernel(const MuonMat* __restrict__ mats, int nmat,
                                                                         int j0) {
  static_assert(kSliceBatch == kSlicePanel, "the first batch is the next panel");
  __shared__ float red[4][kSliceBatch];
  int mi, b;
  if (!slice_of(mats, nmat, mi, b)) return;
  const MuonMat& M = mats[mi];
  const int C = M.C, nsl = mgs_slices(M.R), j1 = j0 + kSlicePanel, nlive = *slice_nlive(M);
  if (j1 >= nlive) return;
  const int t = threadIdx.x, w = t >> 6, lane = t & 63;
  const SliceIO io(M, b, slice_list(M));
  const float* __restrict__ dd = slice_dot_totals(M);
  float* __restrict__ Pout = M.red + (size_t)(j1 & 1) * C * nsl;
  float q[kSlicePanel][kSliceEPT];
#pragma unroll
  for (int k = 0; k < kSlicePanel; k++) io.load(j0 + k, q[k]);
  for (int c0 = j1; c0 < nlive; c0 += kSliceBatch) {
    const int nb = min(kSliceBatch, nlive - c0);
    float x[kSliceBatch][kSliceEPT];
#pragma unroll
    for (int u = 0; u < kSliceBatch; u++) {
      if (u < nb) {
        io.load(c0 + u, x[u]);
      } else {
#pragma unroll
        for (int e = 0; e < kSliceEPT; e++) x[u][e] = 0.f;
      }
    }
#pragma unroll
    for (int u = 0; u < kSliceBatch; u++) {
      if (u >= nb) break;
#pragma unroll
      for (int k = 0; k < kSlicePanel; k++) {
        const float d = dd[(size_t)k * C + c0 + u];
#pragma unroll
        for (int e = 0; e < kSliceEPT; e++) x[u][e] -= d * q[k][e];
      }
      io.store(c0 + u, x[u]);
    }
    if (c0 != j1) continue;
    // the next panel's first column partials: v_j1 . v_c, j1 <= c < j1 + kSlicePanel
#pragma unroll
    for (int u = 0; u < kSliceBatch; u++) {
      float a = 0.f;
#pragma unroll
      for (int e = 0; e < kSliceEPT; e++) a += x[0][e] * x[u][e];
      a = wave_sum(a);
      if (lane == 0) red[w][u] = a;
    }
    __syncthreads();
    if (t < nb) Pout[(size_t)(c0 + t) * nsl + b] = (red[0][t] + red[1][t]) + (red[2][t] + red[3][t]);
    __syncthreads();
  }
}

// Sums NV values over the kPanelThreads threads of a workgroup; every thread
// gets the totals as wave-uniform values.  Each 16-lane row sums through DPP
// and stores one partial per value (P = 4 kPanelWaves partials); after the
// barrier every wave re-reduces them, G = 64 / NV lanes per value reading
// P / G partials each (one or none when G > P), a DPP tree over the G lanes,
// and the totals are read out of fixed lanes.  The order is fixed, so every workgroup and every call sums
// the same way.  `red` alternates between two buffers in consecutive calls,
// so one barrier per call suffices: a thread reads buffer b only before it
// reaches the barrier of the next call, and buffer b is written again only
// after it.
// Eight values reduce-scattered over each 16-lane row by DPP exchanges with
// the mirror lane (15 - i), the half-row mirror (7 - i) and the quad
// partners (i ^ 2, i ^ 1), each step keeping half of the values: lane i ends
// with the row total of value 4 [i >= 8] + 2 [(i & 7) >= 4] + [(i & 3) >= 2]
// (22 instructions instead of eight full row sums and the selects).
__device__ __forceinline__ float row16_reduce_scatter8(const float (&v)[8], int i) {
  const bool hi = i >= 8, h2 = (i & 7) >= 4, h1 = (i & 3) >= 2;
  float a[4], b[2];
#pragma unroll
  for (int k = 0; k < 4; k++) a[k] = (hi ? v[k + 4] : v[k]) + dpp_mov<0x140>(hi ? v[k] : v[k + 4]);
#pragma unroll
  for (int k = 0; k < 2; k++) b[k] = (h2 ? a[k + 2] : a[k]) + dpp_mov<0x141>(h2 ? a[k] : a[k + 2]);
  const float c = (h1 ? b[1] : b[0]) + dpp_mov<0x4E>(h1 ? b[0] : b[1]);
  return c + dpp_mov<0xB1>(c);
}

template <int NV>
__device__ __forceinline__ void panel_sum(float (&v)[NV], float* red) {
  constexpr int P = 4 * kPanelWaves, G = 64 / NV, GL = G < P ? G : P;  // GL: lanes holding partials
  static_assert(P <= 64 && 64 % P == 0 && (NV == 1 || NV == 2 || NV == 4 || NV == 8), "P | 64, NV | 8");
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int i = lane & 15;
  if constexpr (NV == 8) {
    const float s = row16_reduce_scatter8(v, i);
    if ((i & 1) == 0) red[(4 * w + (lane >> 4)) * NV + 4 * (i >= 8) + 2 * ((i & 7) >= 4) + ((i & 3) >= 2)] = s;
  } else {
#pragma unroll
    for (int k = 0; k < NV; k++) v[k] = row16_sum(v[k]);
    float s = v[0];
#pragma unroll
    for (int k = 1; k < NV; k++)
      if (i == k) s = v[k];
    if (i < NV) red[(4 * w + (lane >> 4)) * NV + i] = s;
  }
  __syncthreads();
  const int k = lane / G, u = lane % G;
  float p = 0.f;
#pragma unroll
  for (int j = 0; j * G < P; j++)
    if (u + G * j < P) p += red[(u + G * j) * NV + k];
  p = group8_sum(p);
  if constexpr (GL >= 16) p += dpp_mov<0x140>(p);
#pragma unroll
  for (int kk = 0; kk < NV; kk++) {
    float t = read_lane(p, kk * G);
#pragma unroll
    for (int r = 1; r < GL / 16; r++) t += read_lane(p, kk * G + 16 * r);
    v[kk] = t;
  }
}

// Elements of a vector held by thread t: VEC (R % 4 == 0, rows 16-byte
// aligned): float4 chunks t + kPanelThreads * i, i < EPT / 4; otherwise
// elements t + kPanelThreads * e.  Either way a wave's access is contiguous.
template <int EPT, bool VEC>
__device__ __forceinline__ void row_load(const gfloat* __restrict__ row, int R, int t, bool valid,
                                         float (&x)[EPT]) {
  if constexpr (VEC) {
#pragma unroll
    for (int i = 0; i < EPT / 4; i++) {
      const int c = 4 * (t + kPanelThreads * i);
      fvec4 v = {0.f, 0.f, 0.f, 0.f};
      if (valid && c < R) v = *reinterpret_cast<const gfloat4*>(row + c);
      x[4 * i] = v.x; x[4 * i + 1] = v.y; x[4 * i + 2] = v.z; x[4 * i + 3] = v.w;
    }
  } else {
#pragma unroll
    for (int e = 0; e < EPT; e++) {
      const int k = t + kPanelThreads * e;
      x[e] = (valid && k < R) ? row[k] : 0.f;
    }
  }
}

template <int EPT, bool VEC>
__device__ __forceinline__ void row_store(gfloat* __restrict__ row, int R, int t, const float (&x)[EPT]) {
  if constexpr (VEC) {
#pragma unroll
    for (int i = 0; i < EPT / 4; i++) {
      const int c = 4 * (t + kPanelThreads * i);
      if (c < R) *reinterpret_cast<gfloat4*>(row + c) = fvec4{x[4 * i], x[4 * i + 1], x[4 * i + 2], x[4 * i + 3]};
    }
  } else {
#pragma unroll
    for (int e = 0; e < EPT; e++) {
      const int k = t + kPanelThreads * e;
      if (k < R) row[k] = x[e];
    }
  }
}

// Applies the kPB projections of the panel starting at vector q0 to the NV
// vectors held in x, in order; q_{jj+1} and q_{jj+2} are in flight while
// q_jj's projections reduce.
template <int EPT, bool VEC, int NV>
__device__ __forceinline__ void mgs_project(const gfloat* __restrict__ T, int R, int ld, int q0,
                                            float (&x)[NV][EPT], float (*red)[64 * kPB], int& par) {
  const int t = threadIdx.x;
  float qn[EPT], qn2[EPT];
  row_load<EPT, VEC>(T + (int64_t)q0 * ld, R, t, true, qn);
  row_load<EPT, VEC>(T + (int64_t)(q0 + 1) * ld, R, t, true, qn2);
#pragma unroll 1
  for (int jj = 0; jj < kPB; jj++) {
    float qv[EPT];
#pragma unroll
    for (int e = 0; e < EPT; e++) {
      qv[e] = qn[e];
      qn[e] = qn2[e];
    }
    row_load<EPT, VEC>(T + (int64_t)(q0 + jj + 2) * ld, R, t, jj + 2 < kPB, qn2);
    float d[NV];
#pragma unroll
    for (int v = 0; v < NV; v++) {
      d[v] = 0.f;
#pragma unroll
      for (int e = 0; e < EPT; e++) d[v] += qv[e] * x[v][e];
    }
    panel_sum<NV>(d, red[par]);
    par ^= 1;
#pragma unroll
    for (int v = 0; v < NV; v++)
#pragma unroll
      for (int e = 0; e < EPT; e++) x[v][e] -= d[v] * qv[e];
  }
}

// MGS inside a panel of nv vectors held in x that already carry every
// earlier projection: normalise v_jj, project it out of the later vectors of
// the panel, in order.  Each q vector is stored (to vector c0 + jj of T) as
// soon as it is final, so the stores drain while the later steps run.
template <int EPT, bool VEC>
__device__ __forceinline__ void mgs_factor(float (&x)[kPB][EPT], int nv, float (*red)[64 * kPB], int& par,
                                           gfloat* __restrict__ T, int R, int ld, int c0) {
#pragma unroll
  for (int jj = 0; jj < kPB; jj++) {
    if (jj >= nv) break;
    float s[1] = {0.f};
#pragma unroll
    for (int e = 0; e < EPT; e++) s[0] += x[jj][e] * x[jj][e];
    panel_sum<1>(s, red[par]);
    par ^= 1;
    const float nrm = sqrtf(s[0]) + 1e-30f, rn = 1.f / nrm;
#pragma unroll
    for (int e = 0; e < EPT; e++) x[jj][e] = div_shared(x[jj][e], nrm, rn);
    row_store<EPT, VEC>(T + (int64_t)(c0 + jj) * ld, R, threadIdx.x, x[jj]);
    if (jj + 1 >= nv) break;
    float d[kPB];
#pragma unroll
    for (int v = 0; v < kPB; v++) {
      d[v] = 0.f;
      if (v > jj) {
#pragma unroll
        for (int e = 0; e < EPT; e++) d[v] += x[jj][e] * x[v][e];
      }
    }
    panel_sum<kPB>(d, red[par]);
    par ^= 1;
#pragma unroll
    for (int v = 0; v < kPB; v++)
      if (v > jj) {
#pragma unroll
        for (int e = 0; e < EPT; e++) x[v][e] -= d[v] * x[jj][e];
      }
  }
}

// Elements per thread for a vector of length R (R <= kMaxPanelR).
__host__ __device__ __forceinline__ int panel_ept(int R) {
  return R <= kPanelThreads ? 1 : R <= 2 * kPanelThreads ? 2 : R <= 4 * kPanelThreads ? 4
         : R <= 8 * kPanelThreads ? 8 : 16;
}

// Runs CALL with constexpr E (elements per thread) and V (float4 rows) set
// for matrix M's vector length and alignment.
#define NSH_WITH_LAYOUT(M, CALL)                                                             \
  do {                                                                                       \
    const bool vec_ = (M).R % 4 == 0 && (M).ldT % 4 == 0 &&                                   \
                      (reinterpret_cast<uintptr_t>((M).T) & 15) == 0;                          \
    switch (panel_ept((M).R)) {                                                              \
      case 1: { constexpr int E = 1; constexpr bool V = false; CALL; } break;               \
      case 2: { constexpr int E = 2; constexpr bool V = false; CALL; } break;               \
      case 4:                                                                                \
        if (vec_) { constexpr int E = 4; constexpr bool V = true; CALL; }                   \
        else { constexpr int E = 4; constexpr bool V = false; CALL; }                       \
        break;                                                                               \
      case 8:                                                                                \
        if (vec_) { constexpr int E = 8; constexpr bool V = true; CALL; }                   \
        else { constexpr int E = 8; constexpr bool V = false; CALL; }                       \
        break;                                                                               \
      default:                                                                               \
        if (vec_) { constexpr int E = 16; constexpr bool V = true; CALL; }                  \
        else { constexpr int E = 16; constexpr bool V = false; CALL; }                      \
        break;                                                                               \
    }                                                                                        \
  } while (0)

// One workgroup's share of launch jp: project panel jp (jp >= 0) out of the
// nv vectors c0 ..., and, for the lead workgroup (whose vectors are panel
// jp + 1), factorize them.
template <int EPT, bool VEC>
__device__ __forceinline__ void mgs_panel_body(gfloat* __restrict__ T, int R, int ld, int jp, int c0, int nv,
                                               bool lead, float (*red)[64 * kPB]) {
  const int t = threadIdx.x;
  float x[kPB][EPT];
#pragma unroll
  for (int v = 0; v < kPB; v++) row_load<EPT, VEC>(T + (int64_t)(c0 + v) * ld, R, t, v < nv, x[v]);
  int par = 0;
  if (jp >= 0) mgs_project<EPT, VEC, kPB>(T, R, ld, jp, x, red, par);
  if (lead) {
    mgs_factor<EPT, VEC>(x, nv, red, par, T, R, ld, c0);
    return;
  }
#pragma unroll
  for (int v = 0; v < kPB; v++)
    if (v < nv) row_store<EPT, VEC>(T + (int64_t)(c0 + v) * ld, R, t, x[v]);
}

// Launch for panel jp (jp < 0: the first launch, no projections): vectors
// c >= jp + kPB, kPB per workgroup; workgroup 0 of each matrix owns the next
// panel and factorizes it.  Each workgroup uses its own matrix's layout.
__global__ __launch_bounds__(kPanelThreads) void mgs_panel_kernel(const MuonMat* __restrict__ mats, int nmat, int jp) {
  __shared__ float red[2][64 * kPB];
  const int first = jp + kPB;
  int b = blockIdx.x, mi = 0;
  for (; mi < nmat; mi++) {
    const int nvec = mats[mi].R > kMaxPanelR ? 0 : mats[mi].C - first;
    const int cnt = nvec <= 0 ? 0 : (jp < 0 ? 1 : (nvec + kPB - 1) / kPB);
    if (b < cnt) break;
    b -= cnt;
  }
  if (mi >= nmat) return;
  const MuonMat& M = mats[mi];
  const int c0 = first + b * kPB;
  const int nv = min(kPB, M.C - c0);
  gfloat* T = as_global(M.T);
  const int R = M.R;
  const int ld = M.ldT;
  NSH_WITH_LAYOUT(M, (mgs_panel_body<E, V>(T, R, ld, jp, c0, nv, b == 0, red)));
}

// ---- zero rows of the panel path ----------------------------------------------
// Element k of every vector is zero when row k of the gradient is (an
// embedding row that no token of the step used), and stays zero through
// MGS: q_j[k] = v_j[k] / |v_j| = 0 and every projection subtracts d * 0 from
// it.  When dropping those rows moves the vectors into a smaller register
// layout (panel_ept), each vector is compacted in place to its live rows
// (padded with zeros to a multiple of 4; the stride ldT stays), MGS runs
// with R set to that length, and the q vectors are scattered back with
// zeros in the dropped rows.  Only the order in which the block sums add
// the elements changes.  MuonMat::red of a panel matrix (R > 512) holds, as
// ints: [0] the compacted length (0: not compacted), [1] the live rows,
// then rank[ldT] (flag, then compacted index or -1) and rows[ldT] (row of
// each compacted index).
constexpr int kRowHdr = 2;
__device__ __forceinline__ bool rows_compactable(const MuonMat& M) {
  return M.red && M.ldT <= kMaxPanelR && M.ldT > kPanelThreads;
}

// rank[k] = 1 if row k is nonzero in some vector, else 0: 64 rows x 16
// groups of vectors per 1024-thread workgroup; blockIdx.y = matrix.
__global__ __launch_bounds__(1024) void mgs_rows_live_kernel(const MuonMat* __restrict__ mats, int nmat) {
  __shared__ int any[16][64];
  const MuonMat& M = mats[blockIdx.y];
  if (!rows_compactable(M)) return;
  const int ld = M.ldT, C = M.C;
  const int k = blockIdx.x * 64 + (threadIdx.x & 63), grp = threadIdx.x >> 6;
  if (blockIdx.x * 64 >= ld) return;
  const gfloat* __restrict__ T = as_global(M.T);
  bool nz = false;
  if (k < ld) {
    int c = grp;
    for (; c + 16 * 7 < C; c += 16 * 8) {
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; u++) v[u] = T[(int64_t)(c + 16 * u) * ld + k];
#pragma unroll
      for (int u = 0; u < 8; u++) nz |= v[u] != 0.f;
    }
    for (; c < C; c += 16) nz |= T[(int64_t)c * ld + k] != 0.f;
  }
  any[grp][threadIdx.x & 63] = nz;
  __syncthreads();
  if (grp == 0 && k < ld) {
    int a = 0;
#pragma unroll
    for (int g = 0; g < 16; g++) a |= any[g][threadIdx.x];
    reinterpret_cast<int*>(M.red)[kRowHdr + k] = a;
  }
  (void)nmat;
}

// Per matrix (blockIdx.x), one workgroup: the live rows' compacted indices
// (a prefix sum over the flags), the compacted length, and whether to
// compact; if so, the matrix's R becomes that length until
// mgs_rows_scatter_kernel restores it.
__global__ __launch_bounds__(1024) void mgs_rows_plan_kernel(MuonMat* __restrict__ mats, int nmat) {
  __shared__ int wsum[16];
  MuonMat& M = mats[blockIdx.x];
  if (!rows_compactable(M)) return;
  int* __restrict__ hdr = reinterpret_cast<int*>(M.red);
  int* __restrict__ rank = hdr + kRowHdr;
  int* __restrict__ rows = rank + M.ldT;
  const int ld = M.ldT, t = threadIdx.x, lane = t & 63, w = t >> 6;
  constexpr int kPer = kMaxPanelR / 1024;  // rows per thread, contiguous
  int f[kPer], cnt = 0;
#pragma unroll
  for (int i = 0; i < kPer; i++) {
    const int k = t * kPer + i;
    f[i] = k < ld ? rank[k] : 0;
    cnt += f[i];
  }
  int incl = cnt;  // inclusive prefix over the wave, then over the waves
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int u = __shfl_up(incl, o, 64);
    if (lane >= o) incl += u;
  }
  if (lane == 63) wsum[w] = incl;
  __syncthreads();
  int off = incl - cnt;
  for (int i = 0; i < w; i++) off += wsum[i];
  int total = 0;
  for (int i = 0; i < 16; i++) total += wsum[i];
#pragma unroll
  for (int i = 0; i < kPer; i++) {
    const int k = t * kPer + i;
    if (k < ld) {
      rank[k] = f[i] ? off : -1;
      if (f[i]) rows[off++] = k;
    }
  }
  const int rc = (total + 3) & ~3;
  // worth it only when the vectors move into a smaller register layout
  // (an all-zero matrix is left as it is: its q vectors are zero either way)
  const bool compact = total > 0 && panel_ept(rc) < panel_ept(ld);
  if (t == 0) {
    hdr[0] = compact ? rc : 0;
    hdr[1] = total;
    if (compact) M.R = rc;
  }
  (void)nmat;
}

// Vector c = blockIdx.x of matrix blockIdx.y through LDS: its live rows to
// the front (then zeros up to the compacted length), or back.
constexpr int kRowVecThreads = 512;
__global__ __launch_bounds__(kRowVecThreads) void mgs_rows_compact_kernel(const MuonMat* __restrict__ mats, int nmat) {
  __shared__ float v[kMaxPanelR];
  const MuonMat& M = mats[blockIdx.y];
  if (!rows_compactable(M) || (int)blockIdx.x >= M.C) return;
  const int* __restrict__ hdr = reinterpret_cast<const int*>(M.red);
  const int rc = hdr[0], live = hdr[1];
  if (rc == 0) return;
  const int* __restrict__ rows = hdr + kRowHdr + M.ldT;
  const int ld = M.ldT;
  gfloat* __restrict__ x = as_global(M.T) + (int64_t)blockIdx.x * ld;
  for (int k = threadIdx.x; k < ld; k += kRowVecThreads) v[k] = x[k];
  __syncthreads();
  for (int i = threadIdx.x; i < rc; i += kRowVecThreads) x[i] = i < live ? v[rows[i]] : 0.f;
  (void)nmat;
}

__global__ __launch_bounds__(kRowVecThreads) void mgs_rows_scatter_kernel(MuonMat* __restrict__ mats, int nmat) {
  __shared__ float v[kMaxPanelR / 2];
  MuonMat& M = mats[blockIdx.y];
  if (!rows_compactable(M) || (int)blockIdx.x >= M.C) return;
  const int* __restrict__ hdr = reinterpret_cast<const int*>(M.red);
  const int rc = hdr[0];
  if (rc == 0) return;
  const int* __restrict__ rank = hdr + kRowHdr;
  const int ld = M.ldT;
  gfloat* __restrict__ x = as_global(M.T) + (int64_t)blockIdx.x * ld;
  for (int i = threadIdx.x; i < rc; i += kRowVecThreads) v[i] = x[i];
  __syncthreads();
  for (int k = threadIdx.x; k < ld; k += kRowVecThreads) {
    const int r = rank[k];
    x[k] = r >= 0 ? v[r] : 0.f;
  }
  if (blockIdx.x == 0 && threadIdx.x == 0) M.R = ld;
  (void)nmat;
}

// w -= le * q + (0.01 lr) * w, q = T (normalised vectors): element [k][j]
// of w takes q_j[k] (r >= c, through LDS tiles laid out as in the gather) or
// q_k[j] (r < c).
__global__ __launch_bounds__(256) void muon_update_kernel(const MuonMat* __restrict__ mats, int nmat) {
#pragma clang fp contract(off)
  __shared__ float tile[64 * 65];
  const MuonMat& M = mats[blockIdx.y];
  const gfloat* __restrict__ T = as_global(M.T);
  gfloat* __restrict__ w = as_global(M.w);
  const int64_t R = M.R, C = M.C;
  const float le = M.le, decay = M.decay;
  const bool vec = vec4_ok(R, C, M.w, M.T);
  if (M.transposed) {
    if (vec) {
      const gfloat4* T4 = (const gfloat4*)T;
      gfloat4* w4 = (gfloat4*)w;
      for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < R * C / 4; i += (int64_t)gridDim.x * 256) {
        const fvec4 wi = w4[i], ti = T4[i];
        fvec4 o;
        o.x = wi.x - (le * ti.x + decay * wi.x);
        o.y = wi.y - (le * ti.y + decay * wi.y);
        o.z = wi.z - (le * ti.z + decay * wi.z);
        o.w = wi.w - (le * ti.w + decay * wi.w);
        w4[i] = o;
      }
    } else {
      for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < R * C; i += (int64_t)gridDim.x * 256) {
        const float wi = w[i];
        w[i] = wi - (le * T[i] + decay * wi);
      }
    }
    return;
  }
  if (vec) {
    const int q = threadIdx.x & 15, rr = threadIdx.x >> 4;
    const int64_t tr = (R + 63) / 64, tiles = tr * ((C + 63) / 64);
    for (int64_t b = blockIdx.x; b < tiles; b += gridDim.x) {
      const int64_t j0 = (b / tr) * 64, k0 = (b % tr) * 64;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int jj = rr + 16 * i;
        if (j0 + jj < C && k0 + 4 * q < R) {
          const fvec4 x = *(const gfloat4*)(T + (j0 + jj) * R + k0 + 4 * q);
          float* t = tile + jj * 65 + 4 * q;
          t[0] = x.x, t[1] = x.y, t[2] = x.z, t[3] = x.w;
        }
      }
      __syncthreads();
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int r = rr + 16 * i;
        if (k0 + r < R && j0 + 4 * q < C) {
          const float* t = tile + 4 * q * 65 + r;
          gfloat4* wp = (gfloat4*)(w + (k0 + r) * C + j0 + 4 * q);
          const fvec4 wi = *wp;
          fvec4 o;
          o.x = wi.x - (le * t[0] + decay * wi.x);
          o.y = wi.y - (le * t[65] + decay * wi.y);
          o.z = wi.z - (le * t[130] + decay * wi.z);
          o.w = wi.w - (le * t[195] + decay * wi.w);
          *wp = o;
        }
      }
      __syncthreads();
    }
    return;
  }
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
  const int64_t tr = (R + 31) / 32, tiles = tr * ((C + 31) / 32);
  for (int64_t b = blockIdx.x; b < tiles; b += gridDim.x) {
    const int64_t j0 = (b / tr) * 32, k0 = (b % tr) * 32;
    for (int r = ty; r < 32; r += 8)
      if (j0 + r < C && k0 + tx < R) tile[r * 33 + tx] = T[(j0 + r) * R + k0 + tx];
    __syncthreads();
    for (int r = ty; r < 32; r += 8)
      if (k0 + r < R && j0 + tx < C) {
        const int64_t i = (k0 + r) * C + j0 + tx;
        const float wi = w[i];
        w[i] = wi - (le * tile[tx * 33 + r] + decay * wi);
      }
    __syncthreads();
  }
  (void)nmat;
}

}  // namespace

int launch_adamw(float* w, const float* g, float* m, float* v, int64_t n, float lr, float b1t, float b2t,
                 hipStream_t s) {
  if (n <= 0) return 0;
  if ((((uintptr_t)w | (uintptr_t)g | (uintptr_t)m | (uintptr_t)v) & 15) == 0 && n >= 4)
    hipLaunchKernelGGL(adamw_kernel<true>, dim3((unsigned)ceil_div(n / 4, 256)), dim3(256), 0, s, w, g, m, v, n, lr,
                       b1t, b2t);
  else
    hipLaunchKernelGGL(adamw_kernel<false>, dim3((unsigned)ceil_div(n, 256)), dim3(256), 0, s, w, g, m, v, n, lr,
                       b1t, b2t);
  NSH_LAUNCHED();
  return 0;
}

int64_t mgs_max_panel_len() { return kMaxPanelR; }

bool mgs_rows_may_compact(int64_t R, int64_t live_bound) {
  if (R > kMaxPanelR || R <= kPanelThreads || live_bound <= 0) return false;
  return panel_ept((int)((std::min(R, live_bound) + 3) & ~3)) < panel_ept((int)R);
}

size_t mgs_red_floats(int64_t R, int64_t C) {
  // panel path: the row-compaction tables (header, rank, rows; ints)
  if (R <= kMaxPanelR) return R > kPanelThreads ? (size_t)(kRowHdr + 2 * R) : 0;
  // column partials [2][C][nsl], panel dots [kSlicePanel][C][nsl], their
  // totals [kSlicePanel][C], each slice's mask of nonzero vectors
  // [nsl][ceil(C / 32)], their count and list [1 + C] (ints)
  const int64_t nsl = mgs_slices(R);
  return (size_t)((2 + kSlicePanel) * C * nsl + kSlicePanel * C + nsl * ((C + 31) / 32) + 1 + C);
}

int launch_muon_gather(const MuonMat* d_mats, int nmat, int64_t max_elems, hipStream_t s) {
  if (nmat <= 0) return 0;
  // one workgroup per 64 x 128 tile of the largest matrix
  const unsigned gx = (unsigned)std::min<int64_t>(ceil_div(max_elems, 8192), 4096);
  hipLaunchKernelGGL(muon_gather_kernel, dim3(gx, nmat), dim3(256), 0, s, d_mats, nmat);
  NSH_LAUNCHED();
  return 0;
}

int launch_mgs(const MuonMat* d_mats, const MuonMat* h_mats, int nmat, hipStream_t s, const MgsSide* side) {
  if (nmat <= 0) return 0;
  // panel path for vectors up to kMaxPanelR long, sliced path beyond
  int max_c = 0, max_c_long = 0, slices = 0;
  for (int i = 0; i < nmat; i++) {
    const MuonMat& M = h_mats[i];
    if (M.R > kMaxPanelR) {
      if (!M.red) {
        set_error("muon: vectors longer than " + std::to_string(kMaxPanelR) + " need the partial-sum buffer");
        return -1;
      }
      max_c_long = std::max(max_c_long, M.C);
      slices += mgs_slices(M.R);
    } else {
      max_c = std::max(max_c, M.C);
    }
  }
  // The two paths touch disjoint matrices.  With both present and a side
  // stream given, the sliced launches (bound by HBM) run on the side stream
  // beside the panel launches (bound by one workgroup's chain), forked from
  // and joined back to s by events.
  // panel-path matrices whose zero rows may be dropped (mgs_rows_*)
  int rows_r = 0, rows_c = 0;
  for (int i = 0; i < nmat; i++) {
    const MuonMat& M = h_mats[i];
    if (M.red && M.R <= kMaxPanelR && M.R > kPanelThreads) {
      rows_r = std::max(rows_r, M.R);
      rows_c = std::max(rows_c, M.C);
    }
  }
  MuonMat* dm = const_cast<MuonMat*>(d_mats);
  if (rows_r > 0) {
    hipLaunchKernelGGL(mgs_rows_live_kernel, dim3((unsigned)ceil_div(rows_r, 64), nmat), dim3(1024), 0, s, d_mats,
                       nmat);
    NSH_LAUNCHED();
    hipLaunchKernelGGL(mgs_rows_plan_kernel, dim3(nmat), dim3(1024), 0, s, dm, nmat);
    NSH_LAUNCHED();
    hipLaunchKernelGGL(mgs_rows_compact_kernel, dim3(rows_c, nmat), dim3(kRowVecThreads), 0, s, d_mats, nmat);
    NSH_LAUNCHED();
  }
  const bool fork = side && side->stream && slices > 0 && max_c > 0;
  hipStream_t ss = fork ? side->stream : s;
  if (fork) {
    NSH_CHECK(hipEventRecord(side->fork, s));
    NSH_CHECK(hipStreamWaitEvent(ss, side->fork, 0));
  }
  // Sliced path, in panels of kSlicePanel columns: MGS inside the panel (one
  // launch per column, touching only the panel's vectors), then the
  // panel's raw dots with every later vector, their totals, and the
  // projections of every later vector (which also start the next panel).
  if (slices > 0) {
    hipLaunchKernelGGL(mgs_slice_live_kernel, dim3(slices), dim3(kSliceThreads), 0, ss, d_mats, nmat);
    NSH_LAUNCHED();
    hipLaunchKernelGGL(mgs_slice_list_kernel, dim3(nmat), dim3(256), 0, ss, d_mats, nmat);
    NSH_LAUNCHED();
    hipLaunchKernelGGL(mgs_slice_kernel, dim3(slices), dim3(kSliceThreads), 0, ss, d_mats, nmat, -1, kSlicePanel);
    NSH_LAUNCHED();
  }
  for (int j0 = 0; slices > 0 && j0 < max_c_long; j0 += kSlicePanel) {
    const int j1 = j0 + kSlicePanel;
    for (int j = j0; j < j1 && j < max_c_long; j++) {
      hipLaunchKernelGGL(mgs_slice_kernel, dim3(slices), dim3(kSliceThreads), 0, ss, d_mats, nmat, j, j1);
      NSH_LAUNCHED();
    }
    if (j1 >= max_c_long) break;
    hipLaunchKernelGGL(mgs_slice_dots_kernel, dim3(slices), dim3(kSliceThreads), 0, ss, d_mats, nmat, j0);
    NSH_LAUNCHED();
    hipLaunchKernelGGL(mgs_slice_reduce_kernel, dim3((unsigned)ceil_div(kSlicePanel * max_c_long, 4), nmat),
                       dim3(256), 0, ss, d_mats, nmat, j0);
    NSH_LAUNCHED();
    hipLaunchKernelGGL(mgs_slice_update_kernel, dim3(slices), dim3(kSliceThreads), 0, ss, d_mats, nmat, j0);
    NSH_LAUNCHED();
  }
  if (fork) NSH_CHECK(hipEventRecord(side->join, ss));
  for (int jp = -kPB; jp + kPB < max_c; jp += kPB) {
    int grid = 0;
    for (int i = 0; i < nmat; i++) {
      const int nvec = h_mats[i].R > kMaxPanelR ? 0 : h_mats[i].C - (jp + kPB);
      if (nvec > 0) grid += jp < 0 ? 1 : (int)ceil_div(nvec, kPB);
    }
    hipLaunchKernelGGL(mgs_panel_kernel, dim3(grid), dim3(kPanelThreads), 0, s, d_mats, nmat, jp);
    NSH_LAUNCHED();
  }
  if (fork) NSH_CHECK(hipStreamWaitEvent(s, side->join, 0));
  if (rows_r > 0) {
    hipLaunchKernelGGL(mgs_rows_scatter_kernel, dim3(rows_c, nmat), dim3(kRowVecThreads), 0, s, dm, nmat);
    NSH_LAUNCHED();
  }
  return 0;
}

int launch_muon_update(const MuonMat* d_mats, int nmat, int64_t max_elems, hipStream_t s) {
  if (nmat <= 0) return 0;
  // one workgroup per 64 x 64 tile of the largest matrix
  const unsigned gx = (unsigned)std::min<int64_t>(ceil_div(max_elems, 4096), 4096);
  hipLaunchKernelGGL(muon_update_kernel, dim3(gx, nmat), dim3(256), 0, s, d_mats, nmat);
  NSH_LAUNCHED();
  return 0;
}

}  // namespace nship
