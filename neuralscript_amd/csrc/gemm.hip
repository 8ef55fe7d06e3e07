// fp32 MFMA GEMM for gfx950 (CDNA4):  C[M,N] = act( opA(A) . opB(B) ).
//
// Replaces the reference's dense products and their activation passes:
//   ns_matmul + ns_act2          /root/reference/src/codegen/codegen.cpp:1257-1265, 1244-1255
//   ns_matmul_grad_a  (transB)   codegen.cpp:1318-1326
//   ns_matmul_grad_w  (transA)   codegen.cpp:1329-1337
// (CUDA counterparts ns_gemm_kernel / ns_grad_a_kernel / ns_grad_w_kernel,
// /root/reference/src/codegen/cuda_backend.cpp:58-79, 446-467.)
//
// Design (wave64, MFMA 32x32x2 fp32, true fp32 products and sums):
//  * 256-thread workgroup = 4 waves in a 2x2 grid; workgroup tile 128x128,
//    wave tile 64x64 = 2x2 MFMA blocks of 32x32 (64 accumulators per lane).
//  * K advances in 16-wide slabs staged in LDS, double buffered: the next
//    slab's global loads are in flight while the current slab feeds the
//    MFMAs; one barrier per slab.
//  * Each operand keeps its global memory order in LDS (no transposing
//    stores): k-contiguous operands are read back as float4 along k,
//    row-contiguous operands as four scalars.  Within a 16-slab, lane half h
//    of MFMA step q of group g consumes k = 8g + 4h + q for BOTH operands, a
//    fixed bijection, so the contraction is unchanged.
//  * Workgroup ids are remapped so each XCD (ids are dealt round-robin over
//    the 8 XCDs) owns a contiguous run of tiles, grouped 8 tile-rows at a
//    time for L2 reuse of the B panel.
//  * The activation is applied to the accumulators before the single store.
#include "common.h"
#include "kernels.h"

namespace nship {

typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int BM = 128, BN = 128, BK = 16;  // one 2x2-wave tile; the M side doubles with 4x2 waves
constexpr int KPAD = 4;    // pitch of k-contiguous rows: 20 floats
constexpr int RPAD = 4;    // pitch of row-contiguous k rows: ROWS + 4 floats
constexpr int NT = 256;

// LDS layout of one ROWS x 16 operand tile.
template <bool KC, int ROWS>
struct TileLayout;
template <int ROWS>
struct TileLayout<true, ROWS> {  // [rows][k], k contiguous
  static constexpr int kSize = ROWS * (BK + KPAD);
  __device__ static int at(int row, int k) { return row * (BK + KPAD) + k; }
};
template <int ROWS>
struct TileLayout<false, ROWS> {  // [k][rows], rows contiguous
  static constexpr int kSize = BK * (ROWS + RPAD);
  __device__ static int at(int row, int k) { return k * (ROWS + RPAD) + row; }
};

// Global -> register staging of one ROWS x 16 operand tile by NTH threads.
//  KC: element (row, k) at base[row*ld + k]   (k contiguous)
//  MC: element (row, k) at base[k*ld + row]   (row contiguous)
// `rows` = extent of the row dimension (M or N), `K` = contraction extent.
// init() resolves what stays fixed over the K loop: with VEC, each thread's
// load addresses at k = 0 (row maps looked up once), so a slab's load is one
// add per float4; load<CHK = false> is for tiles whose rows and K slabs are
// all in range (no per-element checks).
template <bool KC, bool VEC, int ROWS, int NTH>
struct Stage {
  static constexpr int kVec = ROWS * BK / 4 / NTH;  // float4 per thread (VEC)
  static constexpr int kSca = ROWS * BK / NTH;      // floats per thread
  static constexpr int kPtr = VEC ? kVec : 1;
  float v[kSca];
  const float* p[kPtr];
  unsigned rin;  // VEC: bit i set = the rows of load i are in range
  // the arguments (the scalar path resolves them per element)
  const float* base_;
  const int* rmap_;
  int row0_, rows_;

  __device__ __forceinline__ static void vec_pos(int idx, int& r, int& k) {
    if (KC) { r = idx / (BK / 4); k = (idx % (BK / 4)) * 4; } else { k = idx / (ROWS / 4); r = (idx % (ROWS / 4)) * 4; }
  }
  // rmap (optional): row r of the operand is row rmap[r] of `base`.
  __device__ __forceinline__ void init(const float* __restrict__ base, int64_t ld, int row0, int rows, int t,
                       const int* __restrict__ rmap = nullptr) {
    base_ = base, rmap_ = rmap, row0_ = row0, rows_ = rows;
    if (VEC) {
      rin = 0;
#pragma unroll
      for (int i = 0; i < kPtr; i++) {
        int r, k;
        vec_pos(t + NTH * i, r, k);
        const int gr = row0 + r;
        const bool in = gr < rows;
        rin |= in ? 1u << i : 0u;  // whole float4 in or out: the contiguous extent is a multiple of 4
        const int64_t rr = !in ? 0 : rmap ? (int64_t)rmap[gr] : (int64_t)gr;
        p[i] = KC ? base + rr * ld + k : base + (int64_t)k * ld + (in ? gr : 0);
      }
    }
  }
  // K-blocked operand (kblk_ > 0, VEC only): slab k0 lies in block k0 / kblk_
  int kblk_ = 0;
  int64_t sk_ = 0;
  template <bool CHK = true>
  __device__ __forceinline__ void load(int64_t ld, int k0, int K, int t) {
    if (VEC) {
      int64_t kb = 0;
      int kl = k0;
      if (kblk_) {
        kb = (int64_t)(k0 / kblk_) * sk_;
        kl = k0 % kblk_;
      }
      const int64_t off = kb + (KC ? (int64_t)kl : (int64_t)kl * ld);
#pragma unroll
      for (int i = 0; i < kVec; i++) {
        float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
        bool ok = true;
        if (CHK) {
          int r, k;
          vec_pos(t + NTH * i, r, k);
          ok = ((rin >> i) & 1) && k0 + k < K;
        }
        if (ok) x = *reinterpret_cast<const float4*>(p[i] + off);
        v[4 * i + 0] = x.x; v[4 * i + 1] = x.y; v[4 * i + 2] = x.z; v[4 * i + 3] = x.w;
      }
    } else {
#pragma unroll
      for (int i = 0; i < kSca; i++) {
        const int idx = t + NTH * i;
        int r, k;
        if (KC) { r = idx / BK; k = idx % BK; } else { k = idx / ROWS; r = idx % ROWS; }
        const int gr = row0_ + r, gk = k0 + k;
        float x = 0.f;
        if (!CHK || (gr < rows_ && gk < K)) {
          const int64_t rr = rmap_ ? (int64_t)rmap_[gr] : (int64_t)gr;
          x = KC ? base_[rr * ld + gk] : base_[(int64_t)gk * ld + gr];
        }
        v[i] = x;
      }
    }
  }
  __device__ __forceinline__ void store(float* __restrict__ lds, int t) const {
    if (VEC) {
#pragma unroll
      for (int i = 0; i < kVec; i++) {
        const int idx = t + NTH * i;
        int r, k;
        if (KC) { r = idx / (BK / 4); k = (idx % (BK / 4)) * 4; } else { k = idx / (ROWS / 4); r = (idx % (ROWS / 4)) * 4; }
        float* p = lds + TileLayout<KC, ROWS>::at(r, k);
        *reinterpret_cast<float4*>(p) = make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
      }
    } else {
#pragma unroll
      for (int i = 0; i < kSca; i++) {
        const int idx = t + NTH * i;
        int r, k;
        if (KC) { r = idx / BK; k = idx % BK; } else { k = idx / ROWS; r = idx % ROWS; }
        lds[TileLayout<KC, ROWS>::at(r, k)] = v[i];
      }
    }
  }
};

// Four operand values of one lane for MFMA steps q = 0..3 of group g.
template <bool KC, int ROWS>
__device__ __forceinline__ void read_frag(const float* __restrict__ lds, int row, int kb, float f[4]) {
  if (KC) {
    const float4 x = *reinterpret_cast<const float4*>(lds + TileLayout<true, ROWS>::at(row, kb));
    f[0] = x.x; f[1] = x.y; f[2] = x.z; f[3] = x.w;
  } else {
#pragma unroll
    for (int q = 0; q < 4; q++) f[q] = lds[TileLayout<false, ROWS>::at(row, kb + q)];
  }
}

// Workgroup b of T -> a linear index such that each XCD (ids are dealt
// round-robin over the 8 XCDs) owns one contiguous run; a bijection on [0, T).
__device__ __forceinline__ int xcd_linear(int b, int T) {
  const int per = T >> 3, rem = T & 7;
  const int x = b & 7, i = b >> 3;
  return x * per + (x < rem ? x : rem) + i;
}

// Logical tile of workgroup b: XCD-contiguous runs, then 8-row groups.
__device__ __forceinline__ void tile_of(int b, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int L = xcd_linear(b, tiles_m * tiles_n);
  const int group = 8 * tiles_n;
  const int first_m = (L / group) * 8;
  const int gsize = min(tiles_m - first_m, 8);
  const int in = L % group;
  tm = first_m + in % gsize;
  tn = in / gsize;
}

// Plain epilogue C = acc * act'(aux) for one wave's 64x64 block (aux with
// C's row and column indices, pitch ldaux): the four 32x32 blocks' aux
// values are loaded one block ahead of that block's stores (the loads of
// block b + 1 are in flight while block b is stored).  Its own loop nest, so
// that the main epilogue's loops stay fully unrolled and the accumulators in
// registers.
template <int CODE>
__device__ __forceinline__ void store_act_grad(const floatx16 (&acc)[2][2], const GemmArgs& g, float* __restrict__ C,
                                               int m0, int n0, int wm, int wn, int l32, int kh, int m_end) {
  if (g.mask_in) {
    // relu' from the sign bits: one 16-bit load per lane and 32x32 block,
    // bit v for the lane's accumulator v (the layout the forward wrote)
    unsigned bits[4];
#pragma unroll
    for (int blk = 0; blk < 4; blk++) {
      const int col = n0 + wn * 64 + (blk & 1) * 32 + l32;
      const int rb = m0 + wm * 64 + (blk >> 1) * 32;
      bits[blk] = col < g.N && rb < m_end ? g.mask_in[(int64_t)(2 * (rb / 32) + kh) * g.ldmask + col] : 0u;
    }
#pragma unroll
    for (int blk = 0; blk < 4; blk++) {
      const int r = blk >> 1, c = blk & 1;
      const int col = n0 + wn * 64 + c * 32 + l32;
      const int row0 = m0 + wm * 64 + r * 32 + 4 * kh;
      const bool cin = col < g.N;
      float* cp = C + (int64_t)row0 * g.ldc + col;
#pragma unroll
      for (int v = 0; v < 16; v++) {
        const int dr = 8 * (v >> 2) + (v & 3);
        if (cin && row0 + dr < m_end) cp[(int64_t)dr * g.ldc] = acc[r][c][v] * ((bits[blk] >> v) & 1u ? 1.f : 0.f);
      }
    }
    return;
  }
  float au[2][16];
  auto load = [&](int blk, float(&dst)[16]) {
    const int col = n0 + wn * 64 + (blk & 1) * 32 + l32;
    const int row0 = m0 + wm * 64 + (blk >> 1) * 32 + 4 * kh;
    const bool cin = col < g.N;
    const float* ap = g.aux + (int64_t)row0 * g.ldaux + col;
#pragma unroll
    for (int v = 0; v < 16; v++) {
      const int dr = 8 * (v >> 2) + (v & 3);
      dst[v] = cin && row0 + dr < m_end ? ap[(int64_t)dr * g.ldaux] : 0.f;
    }
  };
  load(0, au[0]);
#pragma unroll
  for (int blk = 0; blk < 4; blk++) {
    if (blk + 1 < 4) load(blk + 1, au[(blk + 1) & 1]);
    const int r = blk >> 1, c = blk & 1;
    const int col = n0 + wn * 64 + c * 32 + l32;
    const int row0 = m0 + wm * 64 + r * 32 + 4 * kh;
    const bool cin = col < g.N;
    float* cp = C + (int64_t)row0 * g.ldc + col;
#pragma unroll
    for (int v = 0; v < 16; v++) {
      const int dr = 8 * (v >> 2) + (v & 3);
      if (cin && row0 + dr < m_end) cp[(int64_t)dr * g.ldc] = acc[r][c][v] * act_deriv(au[blk & 1][v], CODE);
    }
  }
}

// Sign bits of the pre-activation for a relu gradient later (the layout of
// GemmArgs::mask_out): each lane's 16 rows of a 32x32 block in one 16-bit
// value.  Its own loop nest, as store_act_grad.
__device__ __forceinline__ void store_relu_bits(const floatx16 (&acc)[2][2], const GemmArgs& g, int m0, int n0, int wm,
                                                int wn, int l32, int kh, int m_end) {
#pragma unroll
  for (int r = 0; r < 2; r++)
#pragma unroll
    for (int c = 0; c < 2; c++) {
      const int col = n0 + wn * 64 + c * 32 + l32;
      const int rb = m0 + wm * 64 + r * 32;
      unsigned bits = 0u;
#pragma unroll
      for (int v = 0; v < 16; v++) bits |= (acc[r][c][v] > 0.f ? 1u : 0u) << v;
      if (col < g.N && rb < m_end) g.mask_out[(int64_t)(2 * (rb / 32) + kh) * g.ldmask + col] = (uint16_t)bits;
    }
}

// opA(A)[m,k]: TA ? A[k*lda+m] : A[m*lda+k]   (KC for A <=> !TA)
// opB(B)[k,n]: TB ? B[n*ldb+k] : B[k*ldb+n]   (KC for B <=>  TB)
// PLAIN: no row scatter, no row scale; epilogue kEpiAct (with the
// pre-activation / activation pair when C2 is set), kEpiActGrad or kEpiAccum.
// WMW = 2 / WNW = 2: 4x2 / 2x4 waves (512 threads), workgroup tile
// 256 x 128 / 128 x 256: a quarter fewer operand loads and LDS stores per FLOP.
template <bool TA, bool TB, bool VEC, bool PLAIN, int WMW, int WNW>
__global__ __launch_bounds__(NT * WMW * WNW, VEC ? 4 / (WMW * WNW) : 1) void gemm_f32_kernel(GemmArgs g) {
  constexpr int BMT = BM * WMW, BNT = BN * WNW, NTT = NT * WMW * WNW;
  const int M = g.M, N = g.N, K = g.K;
  const int64_t lda = g.lda, ldb = g.ldb, ldc = g.ldc;
  const int tiles_m = g.tiles_m, tiles_n = g.tiles_n;
  const float* __restrict__ A = g.A + (int64_t)blockIdx.y * g.sA;
  const float* __restrict__ B = g.B + (int64_t)blockIdx.y * g.sB;
  float* __restrict__ C = g.C + (int64_t)blockIdx.y * g.sC;
  int m_end = M;
  // K-grouped: group blockIdx.y contracts over k in [kseg[y], kseg[y+1]).
  int kbeg = 0, kend = K;
  if (g.kseg) {
    kbeg = g.kseg[blockIdx.y];
    kend = g.kseg[blockIdx.y + 1];
  }
  if (g.kitems) {
    if ((int)blockIdx.y >= *g.nkitems) return;
    const int* it = g.kitems + 4 * blockIdx.y;
    kbeg = it[1];
    kend = it[2];
    A = g.A;
    B = g.B;
    C = it[3] < 0 ? g.C + (int64_t)it[0] * g.sC : g.kpart + (int64_t)it[3] * g.sC;
  }
  if (g.kchunk) {
    kbeg = (int)blockIdx.z * g.kchunk;
    kend = min(K, kbeg + g.kchunk);
    C += (int64_t)blockIdx.z * g.sCk;
  }
  constexpr bool AKC = !TA, BKC = TB;
  constexpr int ASZ = TileLayout<AKC, BMT>::kSize, BSZ = TileLayout<BKC, BNT>::kSize;
  __shared__ __attribute__((aligned(16))) float smem[2 * (ASZ + BSZ)];
  // buffer b: A tile at smem + b*(ASZ+BSZ), B tile right after it

  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  const int wm = wave / (2 * WNW), wn = wave % (2 * WNW);
  const int l32 = lane & 31, kh = lane >> 5;

  int m0, n0;
  if (g.groups) {
    // Grouped: tile entry -> (group, m tile); rows [seg[e], seg[e+1]) of the
    // group, B advanced by e * sBg.  Entries run XCD-contiguously with all
    // their n tiles, so a gathered A tile is fetched into one XCD's L2 only.
    // The grid is an upper bound: the workgroups past the device-side tile
    // count exit (uniformly), and the rest are spread over the 8 XCDs by
    // that count, not by the grid size, so each XCD gets an equal share.
    const int T = *g.ntiles * tiles_n;
    if ((int)blockIdx.x >= T) return;
    const int L = xcd_linear(blockIdx.x, T);
    const int entry = L / tiles_n;
    const int e = g.tiles[2 * entry], mt = g.tiles[2 * entry + 1];
    m0 = g.seg[e] + mt * BMT;
    m_end = g.seg[e + 1];
    n0 = (L % tiles_n) * BNT;
    B += (int64_t)e * g.sBg;
  } else {
    int tm, tn;
    tile_of(blockIdx.x, tiles_m, tiles_n, tm, tn);
    m0 = tm * BMT;
    n0 = tn * BNT;
  }

  floatx16 acc[2][2];
#pragma unroll
  for (int r = 0; r < 2; r++)
#pragma unroll
    for (int c = 0; c < 2; c++)
#pragma unroll
      for (int v = 0; v < 16; v++) acc[r][c][v] = 0.f;

  Stage<AKC, VEC, BMT, NTT> sa;
  Stage<BKC, VEC, BNT, NTT> sb;
  const int nk = (kend - kbeg + BK - 1) / BK;
  // (the 256-row tiles never gather rows)
  sa.init(A, lda, m0, m_end, t, WMW == 2 ? nullptr : g.a_rows);
  sb.init(B, ldb, n0, N, t);
  sa.kblk_ = g.kblk;
  sa.sk_ = g.sAk;
  sb.kblk_ = g.kblk;
  sb.sk_ = g.sBk;
  sa.load(lda, kbeg, kend, t);
  sb.load(ldb, kbeg, kend, t);
  sa.store(smem, t);
  sb.store(smem + ASZ, t);
  __syncthreads();
  // every row and K slab of the tile in range: loads without checks
  const bool full = m0 + BMT <= m_end && n0 + BNT <= N && (kend - kbeg) % BK == 0;

  for (int kt = 0; kt < nk; kt++) {
    const int cur = kt & 1;
    const bool more = kt + 1 < nk;
    if (more) {
      if (full) {
        sa.template load<false>(lda, kbeg + (kt + 1) * BK, kend, t);
        sb.template load<false>(ldb, kbeg + (kt + 1) * BK, kend, t);
      } else {
        sa.load(lda, kbeg + (kt + 1) * BK, kend, t);
        sb.load(ldb, kbeg + (kt + 1) * BK, kend, t);
      }
    }
    const float* as = smem + cur * (ASZ + BSZ);
    const float* bs = as + ASZ;
    __builtin_amdgcn_s_setprio(1);
    // the scheduler's MFMA / LDS-read interleaving for GEMM loops: +0.5-0.9%
    // on the 256-row tiles, slower on the others (c5's 128x128 products -21%)
    if constexpr (WMW == 2) __builtin_amdgcn_iglp_opt(1);
#pragma unroll
    for (int g = 0; g < 2; g++) {
      const int kb = 8 * g + 4 * kh;
      float fa[2][4], fb[2][4];
#pragma unroll
      for (int r = 0; r < 2; r++) read_frag<AKC, BMT>(as, wm * 64 + r * 32 + l32, kb, fa[r]);
#pragma unroll
      for (int c = 0; c < 2; c++) read_frag<BKC, BNT>(bs, wn * 64 + c * 32 + l32, kb, fb[c]);
#pragma unroll
      for (int q = 0; q < 4; q++)
#pragma unroll
        for (int r = 0; r < 2; r++)
#pragma unroll
          for (int c = 0; c < 2; c++)
            acc[r][c] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[r][q], fb[c][q], acc[r][c], 0, 0, 0);
    }
    __builtin_amdgcn_s_setprio(0);
    if (more) {
      float* nxt = smem + (cur ^ 1) * (ASZ + BSZ);
      sa.store(nxt, t);
      sb.store(nxt + ASZ, t);
    }
    __syncthreads();
  }

  // Accumulator v of lane (l32, kh) in a 32x32 block sits at
  // row 8*(v/4) + 4*kh + v%4, column l32.
  if constexpr (PLAIN) {
    if (g.mode == kEpiActGrad) {
      // C = acc * relu'(aux): the only activation gradient the plain path
      // takes (plain_act_grad)
      store_act_grad<kActRelu>(acc, g, C, m0, n0, wm, wn, l32, kh, m_end);
      return;
    }
    if (g.mask_out) store_relu_bits(acc, g, m0, n0, wm, wn, l32, kh, m_end);
    // plain stores, the activation resolved once per 32x32 block
#pragma unroll
    for (int r = 0; r < 2; r++)
#pragma unroll
      for (int c = 0; c < 2; c++) {
        const int col = n0 + wn * 64 + c * 32 + l32;
        const int row0 = m0 + wm * 64 + r * 32 + 4 * kh;
        float* cp = C + (int64_t)row0 * ldc + col;
        const bool cin = col < N;
#define NSH_STORE16(CODE)                                                          \
  _Pragma("unroll") for (int v = 0; v < 16; v++) {                                 \
    const int dr = 8 * (v >> 2) + (v & 3);                                         \
    if (cin && row0 + dr < m_end) cp[(int64_t)dr * ldc] = act_apply(acc[r][c][v], CODE); \
  }
        if (g.mode == kEpiAccum) {
#pragma unroll
          for (int v = 0; v < 16; v++) {
            const int dr = 8 * (v >> 2) + (v & 3);
            if (cin && row0 + dr < m_end) cp[(int64_t)dr * ldc] += acc[r][c][v];
          }
          continue;
        }
        if (g.C2) {
          // pre-activation to C, then the activation to C2 below
#pragma unroll
          for (int v = 0; v < 16; v++) {
            const int dr = 8 * (v >> 2) + (v & 3);
            if (cin && row0 + dr < m_end) cp[(int64_t)dr * ldc] = acc[r][c][v];
          }
          cp = g.C2 + (int64_t)blockIdx.y * g.sC + (int64_t)row0 * ldc + col;
        }
        switch (g.act) {
          case kActRelu: NSH_STORE16(kActRelu); break;
          case kActLeaky: NSH_STORE16(kActLeaky); break;
          case kActSigmoid: NSH_STORE16(kActSigmoid); break;
          case kActTanh: NSH_STORE16(kActTanh); break;
          case kActSilu: NSH_STORE16(kActSilu); break;
          case kActGelu: NSH_STORE16(kActGelu); break;
          case kActGeluMoe: NSH_STORE16(kActGeluMoe); break;
          default: NSH_STORE16(kActId); break;
        }
#undef NSH_STORE16
      }
    return;
  }
  // General epilogue (row scatter, row scale, activation gradient or
  // accumulate).  The rows a lane holds in a 32-row block share their output
  // row and scale between the two column blocks: they are looked up once,
  // eight rows at a time with all eight loads in flight together.
#pragma unroll
  for (int r = 0; r < 2; r++)
#pragma unroll
    for (int h = 0; h < 2; h++) {
      const int rbase = m0 + wm * 64 + r * 32 + 16 * h + 4 * kh;
      int crow[8];
      float rs[8];
      // rows past m_end read row m_end - 1's entries (m0 < m_end) and are
      // then marked -1: the loads carry no branch and issue together
#pragma unroll
      for (int u = 0; u < 8; u++) crow[u] = min(rbase + 8 * (u >> 2) + (u & 3), m_end - 1);
      if (g.c_rows) {
#pragma unroll
        for (int u = 0; u < 8; u++) crow[u] = g.c_rows[crow[u]];
      }
#pragma unroll
      for (int u = 0; u < 8; u++) rs[u] = g.row_scale ? g.row_scale[crow[u]] : 1.f;
#pragma unroll
      for (int u = 0; u < 8; u++)
        if (rbase + 8 * (u >> 2) + (u & 3) >= m_end) crow[u] = -1;
#pragma unroll
      for (int c = 0; c < 2; c++) {
        const int col = n0 + wn * 64 + c * 32 + l32;
        if (col >= N) continue;
#pragma unroll
        for (int u = 0; u < 8; u++) {
          if (crow[u] < 0) continue;
          const int row = rbase + 8 * (u >> 2) + (u & 3);
          float* dst = C + (int64_t)crow[u] * ldc + col;
          const float x = acc[r][c][8 * h + u];
          const float a = g.row_scale ? x * rs[u] : x;
          if (g.mode == kEpiAct) *dst = act_apply(a, g.act);
          else if (g.mode == kEpiActGrad) *dst = a * act_deriv(g.aux[(int64_t)row * g.ldaux + col], g.act);
          else *dst = *dst + a;
        }
      }
    }
}

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// Activation gradients the plain epilogue applies itself: ReLU's (the
// training MLPs'); the others take the general epilogue.
static bool plain_act_grad(const GemmArgs& g) { return g.mode == kEpiActGrad && g.aux && g.act == kActRelu; }

// Compute units of the current device (cached per device).
static int device_cus() {
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cus[dev]) {
    int n = 0;
    cus[dev] = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0 ? n : 256;
  }
  return cus[dev];
}

int launch_gemm_ex(const GemmArgs& in, bool tA, bool tB, int batch, hipStream_t s) {
  if (in.M <= 0 || in.N <= 0 || batch <= 0) return 0;
  GemmArgs g = in;
  if (g.kitems && (g.kseg || g.groups || g.kchunk || g.a_rows || g.c_rows || !g.nkitems)) {
    set_error("gemm: K-chunked groups exclude the other grouping modes and row maps");
    return -1;
  }
  if (g.kblk && (g.kblk % BK != 0 || g.kseg || g.kitems || g.groups)) {
    set_error("gemm: K blocks must be a multiple of 16 and exclude K-grouped and grouped modes");
    return -1;
  }
  // float4 staging needs each operand's contiguous extent, leading dimension,
  // batch stride and base to be 4-float aligned.
  // (K-grouped segments start anywhere, so a k-contiguous operand needs the
  // scalar path there.)
  const bool va = aligned16(g.A) && g.lda % 4 == 0 && g.sA % 4 == 0 && ((tA ? g.M : g.K) % 4 == 0) &&
                  (tA || !(g.kseg || g.kitems));
  const bool vb = aligned16(g.B) && g.ldb % 4 == 0 && g.sB % 4 == 0 && ((tB ? g.K : g.N) % 4 == 0) &&
                  (!tB || !(g.kseg || g.kitems));
  const bool vec = va && vb && (!g.kblk || (g.sAk % 4 == 0 && g.sBk % 4 == 0));
  if (g.kblk && !vec) {
    set_error("gemm: K-blocked operands need 16-byte aligned, 4-float strided operands");
    return -1;
  }
  // plain epilogue: no row maps or scaling; activation, activation gradient,
  // accumulate or the pre-activation / activation pair (kchunk partials are
  // always kEpiAct)
  const bool plain = !g.c_rows && !g.row_scale &&
                     (g.mode == kEpiAct || g.mode == kEpiAccum || plain_act_grad(g));
  if (g.C2 && !(plain && g.mode == kEpiAct)) {
    set_error("gemm: the pre-activation / activation pair needs the plain activation epilogue");
    return -1;
  }
  if ((g.mask_out && !(g.C2 && g.act == kActRelu && batch == 1)) || (g.mask_in && !plain_act_grad(g)) ||
      ((g.mask_out || g.mask_in) && g.ldmask < g.N)) {
    set_error("gemm: sign bits need a relu pre-activation / activation pair or a relu gradient, ldmask >= N");
    return -1;
  }
  // 256-row tiles for large dense plain NN products; 256-column tiles for
  // the grouped (per-expert) NN products, whose row ranges are short
  const bool wide = !tA && !tB && vec && plain && !g.groups && !g.kseg && !g.kitems && !g.kchunk && !g.a_rows &&
                    g.M >= 2048;
  const bool tallg = !tA && !tB && vec && g.groups && !g.kseg && !g.kitems && !g.kchunk && g.N >= 1024;
  const int bm = wide ? 2 * BM : BM, bn = tallg ? 2 * BN : BN;
  g.tiles_m = (int)ceil_div(g.M, bm);
  g.tiles_n = (int)ceil_div(g.N, bn);
  // grouped: an upper bound on tile entries, sum_e ceil(n_e / BM) <= M/BM + E
  const int entries = g.groups ? g.tiles_m + g.groups : g.tiles_m;
  const int zs = g.kchunk ? (int)ceil_div(g.K, g.kchunk) : 1;
  const dim3 grid(entries * g.tiles_n, batch, zs), block(NT);
#define NSH_GEMM(TA_, TB_, V_)                                                                        \
  do {                                                                                               \
    if (plain) hipLaunchKernelGGL((gemm_f32_kernel<TA_, TB_, V_, true, 1, 1>), grid, block, 0, s, g);  \
    else hipLaunchKernelGGL((gemm_f32_kernel<TA_, TB_, V_, false, 1, 1>), grid, block, 0, s, g);       \
  } while (0)
  // The 256-row tiles run two workgroups per CU.  When that leaves a
  // half-full last round but one per CU gives whole rounds (tiles = 256 mod
  // 512 on 256 CUs, e.g. c5's batched Q/K/V projection: 768 tiles), extra
  // dynamic LDS holds the kernel to one workgroup per CU (its static 57 KB +
  // 32 KB > half of the CU's 160 KB): 260 -> 220 us on that projection.
  // Otherwise two per CU are faster (c5's output layer: 1046 vs 1181 us).
  const int64_t wide_tiles = (int64_t)entries * g.tiles_n * batch * zs;
  const int cus = device_cus();
  const size_t wide_dyn = wide && wide_tiles % (2 * cus) != 0 && wide_tiles % cus == 0 ? 32768 : 0;
  if (wide) hipLaunchKernelGGL((gemm_f32_kernel<false, false, true, true, 2, 1>), grid, dim3(2 * NT), wide_dyn, s, g);
  else if (tallg && plain) hipLaunchKernelGGL((gemm_f32_kernel<false, false, true, true, 1, 2>), grid, dim3(2 * NT), 0, s, g);
  else if (tallg) hipLaunchKernelGGL((gemm_f32_kernel<false, false, true, false, 1, 2>), grid, dim3(2 * NT), 0, s, g);
  else if (!tA && !tB) { if (vec) NSH_GEMM(false, false, true); else NSH_GEMM(false, false, false); }
  else if (!tA && tB) { if (vec) NSH_GEMM(false, true, true); else NSH_GEMM(false, true, false); }
  else if (tA && !tB) { if (vec) NSH_GEMM(true, false, true); else NSH_GEMM(true, false, false); }
  else { if (vec) NSH_GEMM(true, true, true); else NSH_GEMM(true, true, false); }
#undef NSH_GEMM
  NSH_LAUNCHED();
  return 0;
}

// Sum of the K-chunk partials in chunk order, then the GEMM's epilogue.
// ws holds [splits][batch][M][N]; thread per output element.
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* __restrict__ ws, int splits, int64_t zstride,
                                                            GemmArgs g) {
  const int64_t n_out = (int64_t)g.M * g.N;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n_out) return;
  const int y = blockIdx.y;
  const int64_t off = (int64_t)y * n_out + i;
  float a = 0.f;
  for (int z = 0; z < splits; z++) a += ws[(int64_t)z * zstride + off];
  const int row = (int)(i / g.N), col = (int)(i % g.N);
  float* dst = g.C + (int64_t)y * g.sC + (int64_t)row * g.ldc + col;
  if (g.mode == kEpiAct) *dst = act_apply(a, g.act);
  else if (g.mode == kEpiActGrad) *dst = a * act_deriv(g.aux[(int64_t)row * g.ldaux + col], g.act);
  else *dst = *dst + a;
}

static bool splittable(const GemmArgs& g) {
  return !g.groups && !g.kseg && !g.kitems && !g.a_rows && !g.c_rows && !g.row_scale && !g.C2 && g.kchunk == 0;
}

// Chunk length for `splits` chunks: a multiple of BK (and so of 4, keeping
// float4 staging aligned).
static int split_chunk(int K, int splits) { return (int)(ceil_div(ceil_div(K, splits), BK) * BK); }

int gemm_split_count(const GemmArgs& g, int batch) {
  if (!splittable(g) || g.M <= 0 || g.N <= 0 || batch <= 0) return 1;
  const int64_t tiles = ceil_div(g.M, BM) * ceil_div(g.N, BN) * batch;
  if (tiles >= 384) return 1;
  // The largest split (chunks of at least 512) whose workgroups fill whole
  // rounds of the CUs at up to 4 per CU (c5's output-layer weight gradient,
  // 256 tiles: 4 chunks, 1016 us against 1032 for 3; its 512 x 512 ones: 32
  // and 16), else enough chunks for ~768 workgroups.
  const int cus = device_cus();
  for (int64_t s = std::min<int64_t>(32, g.K / 512); s >= 2; s--)
    if (tiles * s <= 4 * cus && (tiles * s) % cus == 0) return (int)ceil_div(g.K, split_chunk(g.K, (int)s));
  int64_t sp = std::min<int64_t>(ceil_div(768, tiles), g.K / 512);
  sp = std::min<int64_t>(sp, 32);
  if (sp < 2) return 1;
  return (int)ceil_div(g.K, split_chunk(g.K, (int)sp));
}

size_t gemm_split_workspace(const GemmArgs& g, int batch, int splits) {
  return splits <= 1 ? 0 : (size_t)splits * batch * g.M * g.N;
}

int launch_gemm_split(const GemmArgs& in, bool tA, bool tB, int batch, int splits, float* ws, hipStream_t s) {
  if (splits <= 1 || !ws || !splittable(in) || in.K < 2 * BK) return launch_gemm_ex(in, tA, tB, batch, s);
  if (in.M <= 0 || in.N <= 0 || batch <= 0) return 0;
  const int chunk = split_chunk(in.K, splits);
  const int zs = (int)ceil_div(in.K, chunk);
  const int64_t n_out = (int64_t)in.M * in.N;
  GemmArgs p = in;
  p.C = ws;
  p.ldc = in.N;
  p.sC = n_out;
  p.mode = kEpiAct;
  p.act = 0;
  p.aux = nullptr;
  p.mask_in = nullptr;  // the reduction applies relu' from aux
  p.kchunk = chunk;
  p.sCk = n_out * batch;
  if (launch_gemm_ex(p, tA, tB, batch, s) != 0) return -1;
  const dim3 grid((unsigned)ceil_div(n_out, 256), batch);
  hipLaunchKernelGGL(splitk_reduce_kernel, grid, dim3(256), 0, s, ws, zs, n_out * batch, in);
  NSH_LAUNCHED();
  return 0;
}

int launch_gemm(const float* A, const float* B, float* C, int64_t M, int64_t N, int64_t K,
                int64_t lda, int64_t ldb, int64_t ldc, bool tA, bool tB, int act, hipStream_t s) {
  if (M > INT32_MAX || N > INT32_MAX || K > INT32_MAX) {
    set_error("gemm: dimension exceeds int32");
    return -1;
  }
  GemmArgs g;
  g.A = A; g.B = B; g.C = C;
  g.M = (int)M; g.N = (int)N; g.K = (int)K;
  g.lda = lda; g.ldb = ldb; g.ldc = ldc;
  g.act = act;
  return launch_gemm_ex(g, tA, tB, 1, s);
}

}  // namespace nship
