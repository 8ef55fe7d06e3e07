// Top-1 mixture of experts forward: router, dispatch, grouped expert GEMMs.
//
//   reference arithmetic: ns_moe_fwd, codegen.cpp:1915-1945
//     lg_e = sum_k x_k Wg[k,e]    (one fp32 accumulator, k ascending, no FMA)
//     mx = max over live e; lg_e = expf(lg_e - mx); sum over live e (ascending)
//     best = first live e with a strictly larger exp'd value; p = lg_best / sum
//     out = p * ( GELU(x We1[best]) We2[best] ),  GELU = 0.5 a (1 + erf(a/sqrt2))
//
// gfx950 design:
//  * Router: the expert choice is an integer decision, so it must be
//    bit-exact.  The logits are computed exactly as the reference does them
//    (sequential k, separate multiply and add: contraction is switched off in
//    this kernel), and exp is evaluated in double precision and rounded once
//    to float, i.e. correctly rounded, which glibc's expf also is except
//    within ~0.002 ulp of a rounding boundary.  x and Wg slabs are staged in
//    LDS; each thread owns 16 tokens x E/64 experts.
//  * Dispatch: per 256-token block, each token's rank among the block's
//    tokens of the same expert and the block's per-expert counts; one scan
//    turns those into expert segments and a STABLE permutation (tokens stay
//    in order within their expert), plus the (expert, m-tile) list of the
//    grouped GEMM -- all on the device, no host round trip.
//  * Experts: two grouped fp32-MFMA GEMMs over the expert-sorted rows: the
//    first gathers x rows through the permutation and applies GELU in its
//    epilogue, the second scatters rows back to token order scaled by p.
#include <type_traits>

#include "common.h"
#include "kernels.h"

namespace nship {
namespace {

constexpr int kTok = 64;   // tokens per router workgroup
constexpr int kKS = 32;    // k slab
constexpr int kBlk = 256;  // tokens per dispatch block
// Experts whose scan tables (3 E + 2 ints) sit in 64 KB of dynamic LDS;
// beyond, the tables live in the ints workspace (moe_work_ints reserves
// them after ntiles).
constexpr int kLdsExperts = 4096;

// exp(x) correctly rounded to float (double evaluation, one rounding).
__device__ __forceinline__ float exp_rn(float x) { return (float)exp((double)x); }

template <int EPT>  // experts per thread / 64 (E <= 64 * EPT)
__global__ __launch_bounds__(256) void moe_router_kernel(const float* __restrict__ x, const float* __restrict__ Wg,
                                                         const uint8_t* __restrict__ active, float* __restrict__ logits,
                                                         int* __restrict__ best, float* __restrict__ prob, int M,
                                                         int D, int E) {
#pragma clang fp contract(off)
  __shared__ float xs[kTok][kKS + 1];
  __shared__ float ws[kKS][64 * EPT];
  __shared__ float lg[kTok][64 * EPT + 1];
  const int t = threadIdx.x;
  const int e0 = t & 63, tg = t >> 6;  // expert lane, token group (16 tokens)
  const int tok0 = blockIdx.x * kTok;
  float acc[16][EPT];
#pragma unroll
  for (int i = 0; i < 16; i++)
#pragma unroll
    for (int j = 0; j < EPT; j++) acc[i][j] = 0.f;

  for (int k0 = 0; k0 < D; k0 += kKS) {
    for (int i = t; i < kTok * kKS; i += 256) {
      const int r = i / kKS, c = i % kKS;
      const int tok = tok0 + r, k = k0 + c;
      xs[r][c] = (tok < M && k < D) ? x[(int64_t)tok * D + k] : 0.f;
    }
    for (int i = t; i < kKS * 64 * EPT; i += 256) {
      const int r = i / (64 * EPT), c = i % (64 * EPT);
      const int k = k0 + r;
      ws[r][c] = (k < D && c < E) ? Wg[(int64_t)k * E + c] : 0.f;
    }
    __syncthreads();
    const int kn = min(kKS, D - k0);
    for (int kk = 0; kk < kn; kk++) {
#pragma unroll
      for (int j = 0; j < EPT; j++) {
        const float w = ws[kk][e0 + 64 * j];
#pragma unroll
        for (int i = 0; i < 16; i++) {
          const float prod = xs[tg * 16 + i][kk] * w;
          acc[i][j] = acc[i][j] + prod;
        }
      }
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 16; i++)
#pragma unroll
    for (int j = 0; j < EPT; j++) lg[tg * 16 + i][e0 + 64 * j] = acc[i][j];
  __syncthreads();

  // Routing: one thread per token, experts in ascending order.
  if (t < kTok && tok0 + t < M) {
    const int tok = tok0 + t;
    float* l = lg[t];
    if (logits)
      for (int e = 0; e < E; e++) logits[(int64_t)tok * E + e] = l[e];
    float mx = -1.0e30f, sum = 0.f;
    for (int e = 0; e < E; e++)
      if ((!active || active[e]) && l[e] > mx) mx = l[e];
    int b = -1;
    for (int e = 0; e < E; e++) {
      if (active && !active[e]) continue;
      l[e] = exp_rn(l[e] - mx);
      sum = sum + l[e];
      if (b < 0 || l[e] > l[b]) b = e;
    }
    best[tok] = b;
    prob[tok] = (sum > 0.f && b >= 0) ? l[b] / sum : 0.f;
  }
}

// Router with one lane per token: a workgroup holds 64 tokens, and each of
// its 4 waves accumulates EG = E/4 experts of all 64 tokens in registers
// (E <= 64, D % 4 == 0, 16-byte aligned x).  The gate weights a wave needs
// are wave-uniform, so they come through scalar loads and feed the
// multiplies as scalar operands: two vector instructions per multiply-add,
// the unfused sequential-k arithmetic of the reference.  x goes through LDS
// in coalesced 32-wide k slabs (register prefetch of the next slab); the
// logits meet in LDS for the routing of each token by wave 0.
constexpr int kRT = 64;       // tokens per workgroup (one per lane)
constexpr int kRK = 32;       // k slab
constexpr int kRP = kRK + 4;  // LDS row pitch of the x slab

template <int EG, bool EXACT>  // EXACT: E == 4 * EG (no per-expert guards)
__global__ __launch_bounds__(256) void moe_router_tok_kernel(const float* __restrict__ x, const float* __restrict__ Wg,
                                                             const uint8_t* __restrict__ active,
                                                             float* __restrict__ logits, int* __restrict__ best,
                                                             float* __restrict__ prob, int M, int D, int E) {
#pragma clang fp contract(off)
  __shared__ __attribute__((aligned(16))) float xs[kRT * kRP];
  __shared__ float lg[kRT][4 * EG + 1];
  const int t = threadIdx.x, lane = t & 63;
  const int wv = __builtin_amdgcn_readfirstlane(t >> 6);  // wave-uniform, so weights load as scalars
  const int tok0 = blockIdx.x * kRT;
  const int e0 = wv * EG;  // first expert of this wave
  float acc[EG];
#pragma unroll
  for (int j = 0; j < EG; j++) acc[j] = 0.f;
  // slab staging: float4 i of thread t is token (t + 256 i) / 8, k offset 4 ((t + 256 i) % 8)
  float4 st[2];
#pragma unroll
  for (int i = 0; i < 2; i++) {
    const int f = t + 256 * i, r = f >> 3, c = (f & 7) * 4;
    st[i] = (tok0 + r < M && c < D) ? *reinterpret_cast<const float4*>(x + (int64_t)(tok0 + r) * D + c)
                                    : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  for (int k0 = 0; k0 < D; k0 += kRK) {
    __syncthreads();  // previous slab consumed
#pragma unroll
    for (int i = 0; i < 2; i++) {
      const int f = t + 256 * i, r = f >> 3, c = (f & 7) * 4;
      *reinterpret_cast<float4*>(xs + r * kRP + c) = st[i];
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 2; i++) {
      const int f = t + 256 * i, r = f >> 3, c = (f & 7) * 4;
      const int k = k0 + kRK + c;
      st[i] = (tok0 + r < M && k < D) ? *reinterpret_cast<const float4*>(x + (int64_t)(tok0 + r) * D + k)
                                      : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    const int kn = min(kRK, D - k0);  // a multiple of 4
    for (int kq = 0; kq < kn; kq += 4) {
      const float4 xv = *reinterpret_cast<const float4*>(xs + lane * kRP + kq);
      const float xk[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
      for (int u = 0; u < 4; u++) {
        const float* __restrict__ wr = Wg + (int64_t)(k0 + kq + u) * (EXACT ? 4 * EG : E) + e0;
#pragma unroll
        for (int j = 0; j < EG; j++)
          if (EXACT || e0 + j < E) {
            const float prod = xk[u] * wr[j];
            acc[j] = acc[j] + prod;
          }
      }
    }
  }
  const int tok = tok0 + lane;
#pragma unroll
  for (int j = 0; j < EG; j++) {
    lg[lane][e0 + j] = acc[j];
    if (logits && tok < M && (EXACT || e0 + j < E)) logits[(int64_t)tok * E + e0 + j] = acc[j];
  }
  __syncthreads();
  if (wv != 0 || tok >= M) return;
  // Routing, experts in ascending order (first strict maximum wins).
  const float* l = lg[lane];
  float mx = -1.0e30f;
  for (int e = 0; e < E; e++)
    if ((!active || active[e]) && l[e] > mx) mx = l[e];
  float sum = 0.f, bv = 0.f;
  int b = -1;
  for (int e = 0; e < E; e++) {
    if (active && !active[e]) continue;
    const float v = exp_rn(l[e] - mx);
    sum = sum + v;
    if (b < 0 || v > bv) {
      b = e;
      bv = v;
    }
  }
  best[tok] = b;
  prob[tok] = (sum > 0.f && b >= 0) ? bv / sum : 0.f;
}

// Router logits for any number of experts: workgroup (token tile, expert
// tile) computes 64 tokens x 64 experts, each logit a sequential-k fp32 sum
// with contraction off (the arithmetic of moe_router_kernel), into logits.
__global__ __launch_bounds__(256) void moe_logits_kernel(const float* __restrict__ x, const float* __restrict__ Wg,
                                                         float* __restrict__ logits, int M, int D, int E) {
#pragma clang fp contract(off)
  __shared__ float xs[kTok][kKS + 1];
  __shared__ float ws[kKS][64];
  const int t = threadIdx.x;
  const int el = t & 63, tg = t >> 6;  // expert lane, token group (16 tokens)
  const int tok0 = blockIdx.x * kTok, eb = blockIdx.y * 64;
  float acc[16];
#pragma unroll
  for (int i = 0; i < 16; i++) acc[i] = 0.f;
  for (int k0 = 0; k0 < D; k0 += kKS) {
    for (int i = t; i < kTok * kKS; i += 256) {
      const int r = i / kKS, c = i % kKS;
      const int tok = tok0 + r, k = k0 + c;
      xs[r][c] = (tok < M && k < D) ? x[(int64_t)tok * D + k] : 0.f;
    }
    for (int i = t; i < kKS * 64; i += 256) {
      const int r = i / 64, c = i % 64;
      const int k = k0 + r;
      ws[r][c] = (k < D && eb + c < E) ? Wg[(int64_t)k * E + eb + c] : 0.f;
    }
    __syncthreads();
    const int kn = min(kKS, D - k0);
    for (int kk = 0; kk < kn; kk++) {
      const float w = ws[kk][el];
#pragma unroll
      for (int i = 0; i < 16; i++) {
        const float prod = xs[tg * 16 + i][kk] * w;
        acc[i] = acc[i] + prod;
      }
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 16; i++) {
    const int tok = tok0 + tg * 16 + i;
    if (tok < M && eb + el < E) logits[(int64_t)tok * E + eb + el] = acc[i];
  }
}

// Routing from stored logits, one thread per token, experts in ascending
// order (first strict maximum of the exp'd values wins), as the router
// kernels route.
__global__ __launch_bounds__(256) void moe_route_logits_kernel(const float* __restrict__ logits,
                                                               const uint8_t* __restrict__ active,
                                                               int* __restrict__ best, float* __restrict__ prob, int M,
                                                               int E) {
  const int tok = blockIdx.x * 256 + threadIdx.x;
  if (tok >= M) return;
  const float* l = logits + (int64_t)tok * E;
  float mx = -1.0e30f;
  for (int e = 0; e < E; e++)
    if ((!active || active[e]) && l[e] > mx) mx = l[e];
  float sum = 0.f, bv = 0.f;
  int b = -1;
  for (int e = 0; e < E; e++) {
    if (active && !active[e]) continue;
    const float v = exp_rn(l[e] - mx);
    sum = sum + v;
    if (b < 0 || v > bv) {
      b = e;
      bv = v;
    }
  }
  best[tok] = b;
  prob[tok] = (sum > 0.f && b >= 0) ? bv / sum : 0.f;
}

// In-block rank of each token among same-expert tokens, and block counts.
__global__ __launch_bounds__(kBlk) void moe_rank_kernel(const int* __restrict__ best, int* __restrict__ rank,
                                                        int* __restrict__ bcount, int M, int E) {
  __shared__ int b[kBlk];
  const int t = threadIdx.x, tok = blockIdx.x * kBlk + t;
  b[t] = tok < M ? best[tok] : -1;
  __syncthreads();
  const int mine = b[t];
  int r = 0;
  for (int j = 0; j < t; j++) r += b[j] == mine;
  if (tok < M) rank[tok] = r;
  for (int e = t; e < E; e += kBlk) {
    int c = 0;
    for (int j = 0; j < kBlk; j++) c += b[j] == e;
    bcount[(int64_t)blockIdx.x * E + e] = c;
  }
}

// moe_scan_kernel with the block counts staged in LDS (nblk * E <= 16384),
// transposed to [expert][block] with an odd row pitch (conflict-free when
// staged from and written back to the [block][expert] global layout).
// Staging keeps 16 loads in flight per lane.  One wave per expert at a
// time, lane l owning the run of blocks [l c, (l + 1) c): the expert's total
// and each block's offset come from one wave scan of the 64 run sums (DPP
// row shifts plus three lane reads: no LDS round trips), and the expert
// prefix from one wave scan per 64 experts.
constexpr int kScanLds = 16384;
template <int CTRL>
__device__ __forceinline__ int dpp_shr_int(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, true);  // 0 where the source is outside the row
}
__device__ __forceinline__ int wave_incl_scan(int v) {
  const int lane = threadIdx.x & 63;
  v += dpp_shr_int<0x111>(v);  // row_shr:1
  v += dpp_shr_int<0x112>(v);  // row_shr:2
  v += dpp_shr_int<0x114>(v);  // row_shr:4
  v += dpp_shr_int<0x118>(v);  // row_shr:8
  const int r0 = __builtin_amdgcn_readlane(v, 15), r1 = __builtin_amdgcn_readlane(v, 31);
  const int r2 = __builtin_amdgcn_readlane(v, 47);
  return v + (lane >= 16 ? r0 : 0) + (lane >= 32 ? r1 : 0) + (lane >= 48 ? r2 : 0);
}
__global__ __launch_bounds__(256) void moe_scan_lds_kernel(int* __restrict__ bcount, int* __restrict__ seg,
                                                           int* __restrict__ tiles, int* __restrict__ ntiles,
                                                           int nblk, int E, int bm) {
  __shared__ int cnt[kScanLds + 256];
  __shared__ int base[257], tb[257];
  const int t = threadIdx.x, w = t >> 6, lane = t & 63;
  const int P = nblk | 1;  // odd pitch
  constexpr int kB = 16;   // rows per batch and wave
  for (int e0 = 0; e0 < E; e0 += 64) {
    const int e = e0 + lane;
    for (int k0 = w; k0 < nblk; k0 += 4 * kB) {
      int v[kB];
#pragma unroll
      for (int j = 0; j < kB; j++) {
        const int k = k0 + 4 * j;
        v[j] = (k < nblk && e < E) ? bcount[(int64_t)k * E + e] : 0;
      }
#pragma unroll
      for (int j = 0; j < kB; j++) {
        const int k = k0 + 4 * j;
        if (k < nblk && e < E) cnt[e * P + k] = v[j];
      }
    }
  }
  __syncthreads();
  // this lane's run of blocks [kb, ke)
  const int run = (nblk + 63) / 64;
  const int kb = min(nblk, lane * run), ke = min(nblk, kb + run);
  for (int e = w; e < E; e += 4) {
    int c = 0;
    for (int k = kb; k < ke; k++) c += cnt[e * P + k];
    const int tot = __builtin_amdgcn_readlane(wave_incl_scan(c), 63);
    if (lane == 0) base[e + 1] = tot;  // total of expert e, turned into the prefix below
  }
  __syncthreads();
  if (w == 0) {
    int carry = 0, tcarry = 0;
    for (int e0 = 0; e0 < E; e0 += 64) {
      const int e = e0 + lane;
      const int tot = e < E ? base[e + 1] : 0, nt = (tot + bm - 1) / bm;
      const int inc = wave_incl_scan(tot), tinc = wave_incl_scan(nt);
      if (e < E) {
        base[e + 1] = carry + inc;
        tb[e + 1] = tcarry + tinc;
      }
      carry += __builtin_amdgcn_readlane(inc, 63);
      tcarry += __builtin_amdgcn_readlane(tinc, 63);
    }
    if (lane == 0) {
      base[0] = 0;
      tb[0] = 0;
      *ntiles = tcarry;
      seg[E] = carry;
    }
  }
  __syncthreads();
  for (int e = w; e < E; e += 4) {
    int c = 0;
    for (int k = kb; k < ke; k++) c += cnt[e * P + k];
    int off = base[e] + wave_incl_scan(c) - c;
    for (int k = kb; k < ke; k++) {
      const int v = cnt[e * P + k];
      cnt[e * P + k] = off;
      off += v;
    }
    if (lane == 0) seg[e] = base[e];
    for (int i = lane; i < tb[e + 1] - tb[e]; i += 64) {
      tiles[2 * (tb[e] + i)] = e;
      tiles[2 * (tb[e] + i) + 1] = i;
    }
  }
  __syncthreads();
  for (int e0 = 0; e0 < E; e0 += 64) {
    const int e = e0 + lane;
    for (int k0 = w; k0 < nblk; k0 += 4 * kB) {
      int v[kB];
#pragma unroll
      for (int j = 0; j < kB; j++) {
        const int k = k0 + 4 * j;
        v[j] = (k < nblk && e < E) ? cnt[e * P + k] : 0;
      }
#pragma unroll
      for (int j = 0; j < kB; j++) {
        const int k = k0 + 4 * j;
        if (k < nblk && e < E) bcount[(int64_t)k * E + e] = v[j];
      }
    }
  }
}

// Expert segments, per-block offsets (in place over bcount) and the
// (expert, m-tile) list.  One workgroup; thread t owns experts t, t + 256,
// ...; the per-expert tables (3 E + 2 ints) live in dynamic LDS, or in gtab
// (global memory) above kLdsExperts.
__global__ __launch_bounds__(256) void moe_scan_kernel(int* __restrict__ bcount, int* __restrict__ seg,
                                                       int* __restrict__ tiles, int* __restrict__ ntiles, int nblk,
                                                       int E, int bm, int* __restrict__ gtab) {
  extern __shared__ int scan_tab[];
  int* tot = gtab ? gtab : scan_tab;  // gtab: the tables in global memory (E > kLdsExperts)
  int* base = tot + E;
  int* tb = base + E + 1;
  const int t = threadIdx.x;
  for (int e = t; e < E; e += 256) {
    int c = 0;
    for (int k = 0; k < nblk; k++) c += bcount[(int64_t)k * E + e];
    tot[e] = c;
  }
  __syncthreads();
  if (t == 0) {
    base[0] = 0;
    tb[0] = 0;
    for (int e = 0; e < E; e++) {
      base[e + 1] = base[e] + tot[e];
      tb[e + 1] = tb[e] + (tot[e] + bm - 1) / bm;
    }
    *ntiles = tb[E];
  }
  __syncthreads();
  for (int e = t; e < E; e += 256) {
    seg[e] = base[e];
    int run = base[e];
    for (int k = 0; k < nblk; k++) {
      const int c = bcount[(int64_t)k * E + e];
      bcount[(int64_t)k * E + e] = run;
      run += c;
    }
    for (int i = 0; i < tb[e + 1] - tb[e]; i++) {
      tiles[2 * (tb[e] + i)] = e;
      tiles[2 * (tb[e] + i) + 1] = i;
    }
  }
  if (t == 0) seg[E] = base[E];
}

__global__ __launch_bounds__(kBlk) void moe_place_kernel(const int* __restrict__ best, const int* __restrict__ rank,
                                                         const int* __restrict__ boff, int* __restrict__ perm, int M,
                                                         int E) {
  const int tok = blockIdx.x * kBlk + threadIdx.x;
  if (tok >= M) return;
  const int e = best[tok];
  if (e < 0) return;
  perm[boff[(int64_t)blockIdx.x * E + e] + rank[tok]] = tok;
}

// hidden = GELU(pre) over the routed rows [0, *nrows) of [*, H].
__global__ void gelu_rows_kernel(const float* __restrict__ pre, float* __restrict__ hid, const int* __restrict__ nrows,
                                 int64_t H) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)(*nrows) * H) return;
  hid[i] = act_apply(pre[i], kActGeluMoe);
}

// Rows of tokens routed nowhere (no live expert) are zero; one thread per token.
__global__ void zero_rows_kernel(const int* __restrict__ best, float* __restrict__ out, int M, int D) {
  const int tok = blockIdx.x * blockDim.x + threadIdx.x;
  if (tok >= M || best[tok] >= 0) return;
  for (int c = 0; c < D; c++) out[(int64_t)tok * D + c] = 0.f;
}

}  // namespace

size_t moe_work_ints(int64_t M, int64_t E) {
  const int64_t nblk = ceil_div(M, kBlk);
  // best, rank, perm: 3M; bcount: nblk*E; seg: E+1; tiles: 2*(M/128+E+1); ntiles: 1;
  // above kLdsExperts the scan's tables: 3E+2
  return (size_t)(3 * M + nblk * E + (E + 1) + 2 * (ceil_div(M, 128) + E + 1) + 1 +
                  (E > kLdsExperts ? 3 * E + 2 : 0));
}

int launch_moe_route(const float* x, const float* Wg, const uint8_t* active, const MoeWork& w, int64_t M, int64_t D,
                     int64_t E, hipStream_t s) {
  if (M <= 0) return 0;
  if (M > INT32_MAX / 2 || E > INT32_MAX / 4 || (int64_t)ceil_div(M, kBlk) * E > INT32_MAX) {
    set_error("moe: too many tokens or experts");
    return -1;
  }
  const int m = (int)M, d = (int)D, e = (int)E;
  const bool tok_path = E <= 64 && D % 4 == 0 && ((uintptr_t)x & 15) == 0;
  if (E > 256) {  // logits by expert tiles, then routing from them
    hipLaunchKernelGGL(moe_logits_kernel, dim3((unsigned)ceil_div(M, kTok), (unsigned)ceil_div(E, 64)), dim3(256), 0,
                       s, x, Wg, w.logits, m, d, e);
    NSH_LAUNCHED();
    hipLaunchKernelGGL(moe_route_logits_kernel, dim3((unsigned)ceil_div(M, 256)), dim3(256), 0, s, w.logits, active,
                       w.best, w.prob, m, e);
  } else if (tok_path) {
    const dim3 g((unsigned)ceil_div(M, kRT));
#define NSH_ROUTER(EG_)                                                                                      \
  if (E == 4 * EG_)                                                                                          \
    hipLaunchKernelGGL((moe_router_tok_kernel<EG_, true>), g, dim3(256), 0, s, x, Wg, active, w.logits, w.best, \
                       w.prob, m, d, e);                                                                     \
  else                                                                                                       \
    hipLaunchKernelGGL((moe_router_tok_kernel<EG_, false>), g, dim3(256), 0, s, x, Wg, active, w.logits,       \
                       w.best, w.prob, m, d, e)
    if (E <= 8) { NSH_ROUTER(2); }
    else if (E <= 16) { NSH_ROUTER(4); }
    else if (E <= 32) { NSH_ROUTER(8); }
    else { NSH_ROUTER(16); }
#undef NSH_ROUTER
  } else {
    const dim3 g1((unsigned)ceil_div(M, kTok));
    if (E <= 64) hipLaunchKernelGGL(moe_router_kernel<1>, g1, dim3(256), 0, s, x, Wg, active, w.logits, w.best, w.prob, m, d, e);
    else if (E <= 128) hipLaunchKernelGGL(moe_router_kernel<2>, g1, dim3(256), 0, s, x, Wg, active, w.logits, w.best, w.prob, m, d, e);
    else hipLaunchKernelGGL(moe_router_kernel<4>, g1, dim3(256), 0, s, x, Wg, active, w.logits, w.best, w.prob, m, d, e);
  }
  NSH_LAUNCHED();
  const int nblk = (int)ceil_div(M, kBlk);
  hipLaunchKernelGGL(moe_rank_kernel, dim3(nblk), dim3(kBlk), 0, s, w.best, w.rank, w.bcount, m, e);
  NSH_LAUNCHED();
  if ((int64_t)nblk * E <= kScanLds && E <= 256)
    hipLaunchKernelGGL(moe_scan_lds_kernel, dim3(1), dim3(256), 0, s, w.bcount, w.seg, w.tiles, w.ntiles, nblk, e, 128);
  else if (E <= kLdsExperts)
    hipLaunchKernelGGL(moe_scan_kernel, dim3(1), dim3(256), (3 * E + 2) * sizeof(int), s, w.bcount, w.seg, w.tiles,
                       w.ntiles, nblk, e, 128, nullptr);
  else
    hipLaunchKernelGGL(moe_scan_kernel, dim3(1), dim3(256), 0, s, w.bcount, w.seg, w.tiles, w.ntiles, nblk, e, 128,
                       w.ntiles + 1);
  NSH_LAUNCHED();
  hipLaunchKernelGGL(moe_place_kernel, dim3(nblk), dim3(kBlk), 0, s, w.best, w.rank, w.bcount, w.perm, m, e);
  NSH_LAUNCHED();
  return 0;
}

int launch_moe_experts(const float* x, const float* We1, const float* We2, const MoeWork& w, float* out, int64_t M,
                       int64_t D, int64_t H, int64_t E, hipStream_t s) {
  if (M <= 0) return 0;
  // hidden[pos] = GELU(x[perm[pos]] . We1[e])   (expert-sorted rows)
  GemmArgs g;
  g.A = x; g.B = We1; g.C = w.hidden;
  g.M = (int)M; g.N = (int)H; g.K = (int)D;
  g.lda = D; g.ldb = H; g.ldc = H;
  g.act = w.pre ? kActId : kActGeluMoe;
  g.a_rows = w.perm;
  g.groups = (int)E; g.seg = w.seg; g.tiles = w.tiles; g.ntiles = w.ntiles; g.sBg = D * H;
  if (w.pre) {  // training keeps the pre-activation for the backward pass
    g.C = w.pre;
    if (launch_gemm_ex(g, false, false, 1, s) != 0) return -1;
    hipLaunchKernelGGL(gelu_rows_kernel, dim3((unsigned)ceil_div(M * H, 256)), dim3(256), 0, s, w.pre, w.hidden,
                       w.seg + E, H);
    NSH_LAUNCHED();
  } else if (launch_gemm_ex(g, false, false, 1, s) != 0) {
    return -1;
  }
  // out[perm[pos]] = p[perm[pos]] * (hidden[pos] . We2[e])
  GemmArgs g2 = g;
  g2.A = w.hidden; g2.B = We2; g2.C = out;
  g2.N = (int)D; g2.K = (int)H;
  g2.lda = H; g2.ldb = D; g2.ldc = D;
  g2.act = kActId;
  g2.a_rows = nullptr;
  g2.c_rows = w.perm;
  g2.row_scale = w.prob;
  g2.sBg = H * D;
  if (launch_gemm_ex(g2, false, false, 1, s) != 0) return -1;
  // tokens without a live expert
  hipLaunchKernelGGL(zero_rows_kernel, dim3((unsigned)ceil_div(M, 256)), dim3(256), 0, s, w.best, out, (int)M,
                     (int)D);
  NSH_LAUNCHED();
  return 0;
}


// ============================================================================
// Backward (MOE_GRAD_X / _WG / _WE1 / _WE2, codegen.cpp:1388-1579), from the
// forward's routing and expert-sorted rows:
//   dpre2 = dout We2[b]^T;  dpb = sum_a gelu(u_a) dpre2_a;  sd = dpb p_b
//   dH = dpre2 p_b gelu'(u);  dg_e = p_e ((e == b ? dpb : 0) - sd)
//   dx = dg Wg^T + dH We1[b]^T;  dWg = x^T dg
//   dWe1[e] = sum over e's tokens of x^T dH;  dWe2[e] = sum of (gelu(u) p_b)^T dout
// Every product is an fp32-MFMA GEMM: grouped by expert over the sorted rows
// (dpre2, the expert part of dx), or grouped over each expert's token
// segment as the contraction (dWe1, dWe2).
// ============================================================================

// One wave per routed (expert-sorted) row; the routing probabilities are
// recomputed from the logits where each is used (p_b by every lane, p_e by
// the lane writing dg_e), all by the same expression.
__global__ __launch_bounds__(256) void moe_bwd_rows_kernel(const float* __restrict__ pre, const float* __restrict__ dpre2,
                                                           const float* __restrict__ logits,
                                                           const uint8_t* __restrict__ active,
                                                           const int* __restrict__ perm, const int* __restrict__ best,
                                                           const int* __restrict__ nrows, float* __restrict__ dH,
                                                           float* __restrict__ hp, float* __restrict__ dg, int H, int E) {
  const int lane = threadIdx.x & 63;
  const int64_t pos = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (pos >= *nrows) return;
  const int tok = perm[pos];
  const int b = best[tok];
  const float* l = logits + (int64_t)tok * E;
  // routing probabilities, as in the forward (sequential over experts)
  float mx = -1.0e30f, sum = 0.f;
  if (lane == 0) {
    for (int e = 0; e < E; e++)
      if ((!active || active[e]) && l[e] > mx) mx = l[e];
    for (int e = 0; e < E; e++)
      if (!active || active[e]) sum = sum + exp_rn(l[e] - mx);
  }
  mx = __shfl(mx, 0, 64);
  sum = __shfl(sum, 0, 64);
  auto prob_of = [&](int e) {
    const bool live = e >= 0 && e < E && (!active || active[e]);
    return (live && sum > 0.f) ? exp_rn(l[e] - mx) / sum : 0.f;
  };
  const float pb = prob_of(b);
  const float* u = pre + pos * H;
  const float* d2 = dpre2 + pos * H;
  float* dh = dH + pos * H;
  float* h2 = hp + pos * H;
  float dpb = 0.f;
  for (int a = lane; a < H; a += 64) {
    const float ua = u[a];
    const float ga = act_apply(ua, kActGeluMoe);
    const float gd = act_deriv(ua, kActGeluMoe);
    dpb += ga * d2[a];
    dh[a] = d2[a] * pb * gd;
    h2[a] = ga * pb;
  }
  dpb = wave_sum(dpb);
  const float sd = dpb * pb;
  for (int e = lane; e < E; e += 64) dg[(int64_t)tok * E + e] = prob_of(e) * ((e == b ? dpb : 0.f) - sd);
}

// Two [M, D] arrays gathered by the same rows in one launch, W floats per
// thread (float4 when D % 4 == 0 and the bases are 16-byte aligned):
// dst_j[r] = src_j[perm[r]] for r < *nrows.
template <int W>
__global__ __launch_bounds__(256) void gather2_rows_kernel(const float* __restrict__ s1, const float* __restrict__ s2,
                                                           const int* __restrict__ perm, const int* __restrict__ nrows,
                                                           float* __restrict__ d1, float* __restrict__ d2, int64_t DW) {
  typedef typename std::conditional<W == 4, float4, float>::type T;
  const int64_t n = (int64_t)(*nrows) * DW;
  const T* __restrict__ a = reinterpret_cast<const T*>(s1);
  const T* __restrict__ b = reinterpret_cast<const T*>(s2);
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const int64_t r = i / DW, c = i - r * DW;
    const int64_t src = (int64_t)perm[r] * DW + c;
    reinterpret_cast<T*>(d1)[i] = a[src];
    reinterpret_cast<T*>(d2)[i] = b[src];
  }
}

__global__ void fill_zero_kernel(float* __restrict__ p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0.f;
}

// ---- expert weight gradients in token chunks ---------------------------------
// dWe1[e] = xs[seg e]^T dH[seg e] (and dWe2 alike) contract over the expert's
// tokens.  Under Zipf routing one expert holds a quarter of the tokens: as one
// K range per expert its 64 output tiles ran 4-5x longer than the rest and
// held the launch (moep: 222 us per product against 78 us for that expert's
// tiles alone).  Every expert's range is therefore cut into chunks of at most
// kchunk_of(M) tokens, one GEMM work item each; an expert with one chunk writes its
// gradient directly, one with several writes partials that
// moe_kpart_sum_kernel adds in chunk order (deterministic).  moep's two
// products with the partial sums: chunks of 128 tokens 0.40 ms, 256: 0.32,
// 512: 0.29 (one range per expert: 0.49).  The chunk grows with M beyond
// 16384 tokens so that the partial-sum buffer (its size must cover any
// routing: 2 * ceil(M / chunk) expert gradients) stays at 64 of them.
static int64_t kchunk_of(int64_t M) { return std::max<int64_t>(512, ceil_div(ceil_div(M, 32), 16) * 16); }
static int64_t kitems_max(int64_t M, int64_t E) { return E + ceil_div(M, kchunk_of(M)); }
static int64_t kreduce_max(int64_t M) { return M / (kchunk_of(M) + 1); }
static int64_t kslots_max(int64_t M) { return 2 * ceil_div(M, kchunk_of(M)); }

size_t moe_bwd_kitem_ints(int64_t M, int64_t E) {
  return (size_t)(2 + 4 * kitems_max(M, E) + 3 * kreduce_max(M));
}
size_t moe_bwd_kpart_floats(int64_t M, int64_t D, int64_t H) {
  return kreduce_max(M) > 0 ? (size_t)(kslots_max(M) * D * H) : 0;
}

// kit[0] = items, kit[1] = experts with several chunks; then maxitems items
// (expert, k begin, k end, partial slot or -1) in expert order, then those
// experts' (expert, first slot, chunks).  One workgroup: each thread counts
// a run of experts; wave prefix sums (wave_incl_scan) and one LDS exchange of
// the four wave totals turn the counts into offsets.

__global__ __launch_bounds__(256) void moe_kitems_kernel(const int* __restrict__ seg, int E, int kc, int maxitems,
                                                         int* __restrict__ kit, int* __restrict__ dirty) {
  __shared__ int wtot[3][4];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6, per = (E + 255) / 256;
  const int e0 = min(E, t * per), e1 = min(E, e0 + per);
  // an expert without tokens: one empty item (its zero gradients), or none
  // when its slices are known to be zero already
  auto chunks = [&](int e) {
    const int n = seg[e + 1] - seg[e];
    return n > kc ? (n + kc - 1) / kc : n > 0 || !dirty || dirty[e] ? 1 : 0;
  };
  int cnt[3] = {0, 0, 0};  // items, partial slots, experts with several chunks
  for (int e = e0; e < e1; e++) {
    const int c = chunks(e);
    cnt[0] += c;
    if (c > 1) {
      cnt[1] += c;
      cnt[2]++;
    }
  }
  int incl[3];
#pragma unroll
  for (int j = 0; j < 3; j++) {
    incl[j] = wave_incl_scan(cnt[j]);
    if (lane == 63) wtot[j][w] = incl[j];
  }
  __syncthreads();
  int off[3];
#pragma unroll
  for (int j = 0; j < 3; j++) {
    int before = 0;
    for (int u = 0; u < w; u++) before += wtot[j][u];
    off[j] = before + incl[j] - cnt[j];
  }
  if (t == 255) {
    kit[0] = off[0] + cnt[0];
    kit[1] = off[2] + cnt[2];
  }
  int io = off[0], so = off[1], ro = off[2];
  int* items = kit + 2;
  int* red = kit + 2 + 4 * maxitems;
  for (int e = e0; e < e1; e++) {
    const int c = chunks(e), b0 = seg[e], b1 = seg[e + 1];
    for (int z = 0; z < c; z++, io++) {
      items[4 * io] = e;
      items[4 * io + 1] = b0 + z * kc;
      items[4 * io + 2] = min(b1, b0 + (z + 1) * kc);
      items[4 * io + 3] = c > 1 ? so + z : -1;
    }
    if (c > 1) {
      red[3 * ro] = e;
      red[3 * ro + 1] = so;
      red[3 * ro + 2] = c;
      ro++;
      so += c;
    }
  }
  // after both passes over this thread's experts: which slices the launch
  // leaves nonzero (only this thread touches its experts' flags)
  if (dirty)
    for (int e = e0; e < e1; e++) dirty[e] = seg[e + 1] > seg[e] ? 1 : 0;
}

// C[e] = sum over its chunks z (in order) of kpart[first slot + z]; blockIdx.y
// = entry of an expert with several chunks (entries past kit[1] exit).  VEC:
// float4 elements (DH % 4 == 0; the buffers are 16-byte aligned).
template <bool VEC>
__global__ __launch_bounds__(256) void moe_kpart_sum_kernel(const int* __restrict__ kit, int maxitems,
                                                            const float* __restrict__ kpart, float* __restrict__ C,
                                                            int64_t DH) {
  const int r = blockIdx.y;
  if (r >= kit[1]) return;
  const int* red = kit + 2 + 4 * maxitems + 3 * r;
  const int e = red[0], s0 = red[1], c = red[2];
  const float* __restrict__ src = kpart + (int64_t)s0 * DH;
  float* __restrict__ dst = C + (int64_t)e * DH;
  if (VEC) {
    const int64_t n4 = DH / 4;
    const float4* __restrict__ s4 = reinterpret_cast<const float4*>(src);
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += (int64_t)gridDim.x * 256) {
      float4 a = s4[i];
      for (int z = 1; z < c; z++) {
        const float4 b = s4[(int64_t)z * n4 + i];
        a.x += b.x; a.y += b.y; a.z += b.z; a.w += b.w;
      }
      reinterpret_cast<float4*>(dst)[i] = a;
    }
  } else {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < DH; i += (int64_t)gridDim.x * 256) {
      float a = src[i];
      for (int z = 1; z < c; z++) a += src[(int64_t)z * DH + i];
      dst[i] = a;
    }
  }
}

// dWg[D, E] = x[M, D]^T dg[M, E]
static GemmArgs dwg_args(const float* x, const float* dg, float* dWg, int64_t M, int64_t D, int64_t E) {
  GemmArgs g;
  g.A = x; g.B = dg; g.C = dWg;
  g.M = (int)D; g.N = (int)E; g.K = (int)M;
  g.lda = D; g.ldb = E; g.ldc = E;
  return g;
}

size_t moe_bwd_splitk_floats(int64_t M, int64_t D, int64_t E) {
  if (M <= 0 || M > INT32_MAX) return 0;
  const GemmArgs g = dwg_args(nullptr, nullptr, nullptr, M, D, E);
  return gemm_split_workspace(g, 1, gemm_split_count(g, 1));
}

int launch_moe_backward(const float* x, const float* dout, const float* Wg, const float* We1, const float* We2,
                        const uint8_t* active, const MoeWork& w, const MoeBwdWork& b, float* dx, float* dWg,
                        float* dWe1, float* dWe2, int64_t M, int64_t D, int64_t H, int64_t E, hipStream_t s,
                        int phases) {
  if (M <= 0) {  // no tokens: the weight gradients are empty sums
    if (dWg && launch_fill(dWg, D * E, 0.f, s) != 0) return -1;
    if (dWe1 && launch_fill(dWe1, E * D * H, 0.f, s) != 0) return -1;
    if (dWe2 && launch_fill(dWe2, E * H * D, 0.f, s) != 0) return -1;
    return 0;
  }
  const int* nrows = w.seg + E;
  if (phases & kMoeBwdGrouped) {
  // dpre2[pos] = dout[perm[pos]] . We2[e]^T
  GemmArgs g;
  g.A = dout; g.B = We2; g.C = b.dpre2;
  g.M = (int)M; g.N = (int)H; g.K = (int)D;
  g.lda = D; g.ldb = D; g.ldc = H;
  g.a_rows = w.perm;
  g.groups = (int)E; g.seg = w.seg; g.tiles = w.tiles; g.ntiles = w.ntiles; g.sBg = H * D;
  if (launch_gemm_ex(g, false, true, 1, s) != 0) return -1;
  hipLaunchKernelGGL(fill_zero_kernel, dim3((unsigned)ceil_div(M * E, 256)), dim3(256), 0, s, b.dg, M * E);
  NSH_LAUNCHED();
  const dim3 rg((unsigned)ceil_div(M, 4));
  hipLaunchKernelGGL(moe_bwd_rows_kernel, rg, dim3(256), 0, s, w.pre, b.dpre2, w.logits, active, w.perm, w.best,
                     nrows, b.dH, b.hp, b.dg, (int)H, (int)E);
  NSH_LAUNCHED();
  // dx = dg Wg^T, then += dH We1[e]^T scattered back to token order
  if (dx) {
    if (launch_gemm(b.dg, Wg, dx, M, D, E, E, E, D, false, true, 0, s) != 0) return -1;
    GemmArgs h;
    h.A = b.dH; h.B = We1; h.C = dx;
    h.M = (int)M; h.N = (int)D; h.K = (int)H;
    h.lda = H; h.ldb = H; h.ldc = D;
    h.c_rows = w.perm;
    h.mode = kEpiAccum;
    h.groups = (int)E; h.seg = w.seg; h.tiles = w.tiles; h.ntiles = w.ntiles; h.sBg = D * H;
    if (launch_gemm_ex(h, false, true, 1, s) != 0) return -1;
  }
  }
  // dWg = x^T dg: D x E outputs (a handful of tiles) over K = M tokens, split
  // over K when the caller brought the workspace
  if ((phases & kMoeBwdGate) && dWg) {
    const GemmArgs g = dwg_args(x, b.dg, dWg, M, D, E);
    const int sp = gemm_split_count(g, 1);
    const bool split = sp > 1 && b.splitk && gemm_split_workspace(g, 1, sp) <= b.splitk_floats;
    if ((split ? launch_gemm_split(g, true, false, 1, sp, b.splitk, s) : launch_gemm_ex(g, true, false, 1, s)) != 0)
      return -1;
  }
  if (!(phases & kMoeBwdKGrouped)) return 0;
  // expert-sorted copies of x and dout for the K-grouped products
  const bool gvec = D % 4 == 0 &&
                    ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(dout) |
                      reinterpret_cast<uintptr_t>(b.xs) | reinterpret_cast<uintptr_t>(b.ds)) & 15) == 0;
  const int64_t DW = gvec ? D / 4 : D;
  const dim3 gd((unsigned)std::min<int64_t>(ceil_div(M * DW, 256), 8192));
  if (gvec)
    hipLaunchKernelGGL(gather2_rows_kernel<4>, gd, dim3(256), 0, s, x, dout, w.perm, nrows, b.xs, b.ds, DW);
  else
    hipLaunchKernelGGL(gather2_rows_kernel<1>, gd, dim3(256), 0, s, x, dout, w.perm, nrows, b.xs, b.ds, DW);
  NSH_LAUNCHED();
  // token chunks of each expert (without the work buffers: one K range per
  // expert)
  const bool chunked = b.kitems && (b.kpart || kreduce_max(M) == 0);
  const int maxitems = (int)kitems_max(M, E), maxred = (int)kreduce_max(M);
  if (chunked) {
    hipLaunchKernelGGL(moe_kitems_kernel, dim3(1), dim3(256), 0, s, w.seg, (int)E, (int)kchunk_of(M), maxitems,
                       b.kitems, b.dirty);
    NSH_LAUNCHED();
  }
  auto weight_grad = [&](const float* A, const float* B, float* C, int64_t R, int64_t Cc) -> int {
    GemmArgs k;
    k.A = A; k.B = B; k.C = C;
    k.M = (int)R; k.N = (int)Cc; k.K = (int)M;
    k.lda = R; k.ldb = Cc; k.ldc = Cc;
    k.sC = R * Cc;
    if (!chunked) {
      k.kseg = w.seg;
      return launch_gemm_ex(k, true, false, (int)E, s);
    }
    k.kitems = b.kitems + 2; k.nkitems = b.kitems; k.kpart = b.kpart;
    if (launch_gemm_ex(k, true, false, maxitems, s) != 0) return -1;
    if (maxred > 0) {
      const int64_t DH = R * Cc;
      const bool vec = DH % 4 == 0 && ((reinterpret_cast<uintptr_t>(C) | reinterpret_cast<uintptr_t>(b.kpart)) & 15) == 0;
      // one element (float4) per thread: each entry's sum is a few MB, and
      // fewer threads looping over it left the pass latency-bound
      const unsigned gx = (unsigned)std::min<int64_t>(ceil_div(vec ? DH / 4 : DH, 256), 4096);
      if (vec)
        hipLaunchKernelGGL(moe_kpart_sum_kernel<true>, dim3(gx, maxred), dim3(256), 0, s, b.kitems, maxitems, b.kpart,
                           C, DH);
      else
        hipLaunchKernelGGL(moe_kpart_sum_kernel<false>, dim3(gx, maxred), dim3(256), 0, s, b.kitems, maxitems, b.kpart,
                           C, DH);
      NSH_LAUNCHED();
    }
    return 0;
  };
  // dWe1[e] [D, H] = xs[seg e]^T dH[seg e]
  if (dWe1 && weight_grad(b.xs, b.dH, dWe1, D, H) != 0) return -1;
  // dWe2[e] [H, D] = hp[seg e]^T ds[seg e]
  if (dWe2 && weight_grad(b.hp, b.ds, dWe2, H, D) != 0) return -1;
  return 0;
}

}  // namespace nship
