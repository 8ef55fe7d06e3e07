// Host-side launchers of the hand-written gfx950 kernels.  All take device
// pointers and a stream, enqueue asynchronously, and return 0 / -1.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>

namespace nship {

// gemm.hip -------------------------------------------------------------------
enum GemmEpilogue : int {
  kEpiAct = 0,      // C = act(acc)
  kEpiActGrad = 1,  // C = acc * act'(aux)      (matmul_grad_a fused with ACTIVATION_GRAD)
  kEpiAccum = 2,    // C = C + acc
};

struct GemmArgs {
  const float* A = nullptr;
  const float* B = nullptr;
  float* C = nullptr;
  int M = 0, N = 0, K = 0;
  int64_t lda = 0, ldb = 0, ldc = 0;
  int64_t sA = 0, sB = 0, sC = 0;  // batch strides (blockIdx.y)
  int act = 0;
  int mode = kEpiAct;
  const float* aux = nullptr;
  int64_t ldaux = 0;
  // kEpiAct with C2 set: C = acc and C2 = act(acc), same pitch (a training
  // forward keeps the pre-activation for the backward pass)
  float* C2 = nullptr;
  // Row gather / scatter (!transA only): operand-A row r is A row a_rows[r];
  // output row r goes to C row c_rows[r], scaled by row_scale[c_rows[r]].
  const int* a_rows = nullptr;
  const int* c_rows = nullptr;
  const float* row_scale = nullptr;
  // Grouped mode (groups > 0): rows [seg[e], seg[e+1]) form group e and use
  // B + e * sBg; `tiles` lists (group, m-tile) pairs, *ntiles of them.
  int groups = 0;
  const int* seg = nullptr;
  const int* tiles = nullptr;
  const int* ntiles = nullptr;
  int64_t sBg = 0;
  // K-grouped mode (kseg set): launch with batch = groups; group y contracts
  // over k in [kseg[y], kseg[y+1]) and writes C + y * sC.
  const int* kseg = nullptr;
  // K-chunked groups (kitems set, nkitems on the device): launch with batch
  // = an upper bound on the items; item y = kitems[4y .. 4y+3] = (group e,
  // k begin, k end, slot) contracts over [k begin, k end) and writes
  // C + e * sC when slot < 0, else kpart + slot * sC (a partial sum that a
  // later pass adds up); items past *nkitems exit.  A and B are not
  // advanced per item (the k range selects the group's rows).
  const int* kitems = nullptr;
  const int* nkitems = nullptr;
  float* kpart = nullptr;
  // Split K (kchunk > 0): blockIdx.z contracts over k in
  // [z * kchunk, min(K, (z+1) * kchunk)) and writes C + z * sCk.
  int kchunk = 0;
  int64_t sCk = 0;
  // ReLU sign bits, plain path only, in the MFMA accumulator layout: for
  // the 32-row block b = row / 32, half h and column col, the 16-bit value
  // at [(2 b + h) * ldmask + col] holds bit v = (pre-activation > 0) of row
  // 32 b + 4 h + 8 (v / 4) + v % 4 -- the rows one lane holds.  mask_out:
  // written by a kEpiAct GEMM with C2 set and act relu (one batch); mask_in:
  // a relu kEpiActGrad GEMM takes the derivative from these bits instead of
  // from aux (the same values, 1/32 of the bytes, one load per lane and
  // block; aux stays the fallback).  Size: 2 * ceil(rows / 32) * ldmask.
  uint16_t* mask_out = nullptr;
  const uint16_t* mask_in = nullptr;
  int64_t ldmask = 0;
  // K-blocked operands (kblk > 0, a multiple of 16, float4 staging only):
  // contraction index k lies in block k / kblk at offset k % kblk; block b of
  // A starts at A + b * sAk and of B at B + b * sBk, each block laid out as
  // the operand is (lda / ldb).  One launch then contracts over several
  // separately stored products, e.g. dX = [dQ dK dV] . [Wq Wk Wv]^T.
  int kblk = 0;
  int64_t sAk = 0, sBk = 0;
  int tiles_m = 0, tiles_n = 0;    // filled by the launcher
};

int launch_gemm_ex(const GemmArgs& g, bool tA, bool tB, int batch, hipStream_t s);
// Split-K for GEMMs with few output tiles and a long K: number of K chunks
// the heuristic picks (1 = no split) and the workspace it needs (floats).
int gemm_split_count(const GemmArgs& g, int batch);
size_t gemm_split_workspace(const GemmArgs& g, int batch, int splits);
// Runs g with `splits` K chunks through `ws` (partials, then a fixed-order
// reduction applying g's epilogue); splits <= 1 or a plan the split does not
// support (row gather/scatter, groups) runs launch_gemm_ex.
int launch_gemm_split(const GemmArgs& g, bool tA, bool tB, int batch, int splits, float* ws, hipStream_t s);
int launch_gemm(const float* A, const float* B, float* C, int64_t M, int64_t N, int64_t K,
                int64_t lda, int64_t ldb, int64_t ldc, bool tA, bool tB, int act, hipStream_t s);


// rowops.hip -----------------------------------------------------------------
int launch_embedding(const float* W, const float* idx, float* out, int64_t n, int64_t V, int64_t D, hipStream_t s);
int launch_layernorm(const float* x, float* y, int64_t rows, int64_t last, hipStream_t s);
int launch_layernorm_grad(const float* dout, const float* x, float* dx, int64_t rows, int64_t last, hipStream_t s);
int launch_softmax_xent(const float* logits, const float* labels, float* grad, float* row_loss, float* loss,
                        int64_t rows, int64_t C, bool write_grad, hipStream_t s);
int launch_act_grad(const float* din, const float* pre, float* dout, int64_t n, int code, hipStream_t s);
size_t embedding_grad_workspace(int64_t n, int64_t V);  // ints
int launch_embedding_grad(const float* dout, const float* idx, float* dW, int64_t n, int64_t V, int64_t D, int* ws,
                          hipStream_t s);

// attention.hip ----------------------------------------------------------------
// ctx[S, D] (heads concatenated) = softmax(Q_h K_h^T * scale) V_h per head,
// Q/K/V row-major [S, D] with row pitch ld.  lse (optional, [H, S]) receives
// log2(sum_j 2^(s_j * scale * log2 e)) per query, for the backward pass.
// Head sizes 32, 64 and 128 on 16-byte aligned rows (ld % 4 == 0) run in
// place (attention_in_place over the arrays read as float4 rows: Q, K, V,
// and O, dO in the backward); every other head size up to 128 runs on a copy
// padded with zero columns to the next of them, in pad_ws
// (attention_pad_floats floats).  Above 128, pad_ws (as many floats) holds
// the scores of a block of query rows, [H][rows][S], which the GEMM kernels
// produce and consume (rows: all S while H * S * S floats fit 1 GiB).
bool attention_in_place(int64_t D, int64_t H, int64_t ld, const void* const* ptrs, int n);
size_t attention_pad_floats(int64_t S, int64_t D, int64_t H, bool backward);
int launch_attention_fwd(const float* Q, const float* K, const float* V, float* ctx, float* lse, int64_t S, int64_t D,
                         int64_t H, int64_t ld, float* pad_ws, hipStream_t s);

// Backward of the core: dQ, dK, dV [S, D] (row pitch ld) from dO = d ctx, the
// forward's ctx (O) and lse; delta: [H, S] workspace.  ds_ws (optional, 16-byte
// aligned, attention_bwd_ds_floats(S, D, H) floats when that is nonzero)
// holds dS so that dQ is a product over it instead of a second pass that
// recomputes S and dP.
size_t attention_bwd_ds_floats(int64_t S, int64_t D, int64_t H);
int launch_attention_bwd(const float* Q, const float* K, const float* V, const float* O, const float* dO,
                         const float* lse, float* delta, float* dQ, float* dK, float* dV, int64_t S, int64_t D,
                         int64_t H, int64_t ld, float* ds_ws, float* pad_ws, hipStream_t s);

// optim.hip --------------------------------------------------------------------
int launch_adamw(float* w, const float* g, float* m, float* v, int64_t n, float lr, float b1t, float b2t,
                 hipStream_t s);

// One Muon matrix of an optimizer step (device-resident descriptor).
struct MuonMat {
  float* w;          // weight [r][c], updated in place
  const float* g;    // gradient [r][c]
  float* T;          // work: vectors contiguous, [C][R]; q vectors on exit
  float* red;        // mgs_red_floats(R, C): sliced path (R > 8192) partial sums; panel path (R > 512) the
                     // row-compaction tables; null when that is 0
  int R, C;          // vector length, number of vectors
  int ldT;           // stride of T's vectors: R (MGS may run on fewer, compacted rows, R set meanwhile)
  int transposed;    // r < c: the vectors are the rows of g
  float le, decay;   // lr * sqrt(min(r, c)), 0.01 * lr
};
size_t mgs_red_floats(int64_t R, int64_t C);
int launch_muon_gather(const MuonMat* d_mats, int nmat, int64_t max_elems, hipStream_t s);
// MGS of every matrix: T holds the vectors on entry, the q vectors on exit.
// Longest vector the register-panel MGS takes; longer ones go through the
// sliced path (and need MuonMat::red).
int64_t mgs_max_panel_len();
// Whether a register-panel matrix (R <= mgs_max_panel_len()) whose vectors
// have at most live_bound nonzero elements could run MGS on compacted rows
// (a smaller register layout); its MuonMat::red (mgs_red_floats) enables it.
bool mgs_rows_may_compact(int64_t R, int64_t live_bound);
// A second stream for the sliced-path launches of launch_mgs, and the two
// events (no timing) that fork it from and join it back to the main stream.
struct MgsSide {
  hipStream_t stream = nullptr;
  hipEvent_t fork = nullptr, join = nullptr;
};
int launch_mgs(const MuonMat* d_mats, const MuonMat* h_mats, int nmat, hipStream_t s,
               const MgsSide* side = nullptr);
int launch_muon_update(const MuonMat* d_mats, int nmat, int64_t max_elems, hipStream_t s);

// peak.hip -----------------------------------------------------------------------
// Attainable-peak microbenchmarks: time (ms, HIP events on the null stream) of
// one launch of `blocks` x 256 threads issuing iters x 4 fp32 MFMAs per wave,
// and of one float4 copy of n floats (mean over reps); `out` is a dummy
// buffer of 256 floats.
int bench_mfma_peak(int iters, int blocks, float* out, float* ms);
int bench_copy(const float* src, float* dst, int64_t n, int reps, float* ms);
int bench_rowops(const float* idx, const float* labels, int64_t M, int64_t D, int64_t V, int64_t C, int reps,
                 double* us);

// movement.hip -------------------------------------------------------------------
int launch_binop(const float* A, const float* B, float* C, int64_t na, int64_t nb, int code, hipStream_t s);
// out = in, then softmax over each full row of `last` (a tail shorter than a row is copied)
int launch_softmax(const float* in, float* out, int64_t n, int64_t last, hipStream_t s);
int launch_transpose(const float* in, float* out, int64_t R, int64_t C, hipStream_t s);
int launch_concat_cols(const float* a, const float* b, float* out, int64_t R, int64_t ca, int64_t cb, hipStream_t s);
int launch_slice_cols(const float* in, float* out, int64_t M, int64_t C, int64_t start, int64_t width,
                      hipStream_t s);
int launch_index(const float* in, const int64_t* idx, float* out, int64_t M, int64_t C, int64_t L, int axis,
                 hipStream_t s);
int launch_scatter(const float* in, const int64_t* idx, const float* upd, float* out, int64_t R, int64_t C,
                   int64_t L, int axis, hipStream_t s);
int launch_fill(float* out, int64_t n, float v, hipStream_t s);
// y = x * (keep[i] ? scale : 0): a dropout's forward (train mode) and its gradient
int launch_dropout(const float* x, const uint8_t* keep, float* y, int64_t n, float scale, hipStream_t s);
int launch_copy(const float* in, float* out, int64_t n, hipStream_t s);

// moe.hip ----------------------------------------------------------------------
struct MoeWork {
  float* logits;   // [M, E]  raw router logits (kept for tie reports)
  int* best;       // [M]     chosen expert, -1 if none live
  float* prob;     // [M]     routing probability of the chosen expert
  int* rank;       // [M]     rank of the token among same-expert tokens of its block
  int* bcount;     // [nblk, E]
  int* seg;        // [E + 1] segment starts of the expert-sorted order
  int* perm;       // [M]     expert-sorted position -> token
  int* tiles;      // [2 * (M/128 + E)] (expert, m-tile) pairs
  int* ntiles;     // [1]; above 4096 experts the dispatch scan's tables (3E+2 ints) follow it
  float* hidden;   // [M, H]  GELU(x We1[e]) in expert-sorted order
  float* pre;      // [M, H]  x We1[e] before GELU (training only, else null)
};
struct MoeBwdWork {
  float* dpre2;    // [M, H]
  float* dH;       // [M, H]
  float* hp;       // [M, H]  GELU(u) * p_best
  float* dg;       // [M, E]  router logit gradient (token order)
  float* xs;       // [M, D]  x in expert-sorted order
  float* ds;       // [M, D]  dout in expert-sorted order
  float* splitk = nullptr;   // optional: K-chunk partials of dWg = x^T dg (moe_bwd_splitk_floats)
  size_t splitk_floats = 0;
  // the expert weight gradients' work items and partial sums
  // (moe_bwd_kitem_ints, moe_bwd_kpart_floats)
  int* kitems = nullptr;
  float* kpart = nullptr;
  // optional, with kitems: one int per expert, nonzero when its dWe1 / dWe2
  // slices may hold nonzeros.  An expert without tokens then gets its zero
  // gradients written only when its flag is set (and the flag cleared); an
  // expert with tokens sets it.  The caller keeps the array with the two
  // gradient buffers and sets every flag when either buffer is new.
  int* dirty = nullptr;
};
// Ints of MoeBwdWork::kitems and floats of MoeBwdWork::kpart for M tokens:
// every expert's tokens are cut into chunks (512 tokens, more beyond 16384
// tokens) for the weight gradients dWe1, dWe2, and the experts with several
// chunks sum their partials in chunk order afterwards (kpart: at most 64
// expert gradients).
size_t moe_bwd_kitem_ints(int64_t M, int64_t E);
size_t moe_bwd_kpart_floats(int64_t M, int64_t D, int64_t H);
// Floats of MoeBwdWork::splitk that let dWg = x^T dg (K = M tokens, only
// D x E outputs) run split over K; 0 when it would not be split.
size_t moe_bwd_splitk_floats(int64_t M, int64_t D, int64_t E);
size_t moe_work_ints(int64_t M, int64_t E);   // int-sized words of all int arrays
int launch_moe_route(const float* x, const float* Wg, const uint8_t* active, const MoeWork& w, int64_t M, int64_t D,
                     int64_t E, hipStream_t s);
int launch_moe_experts(const float* x, const float* We1, const float* We2, const MoeWork& w, float* out, int64_t M,
                       int64_t D, int64_t H, int64_t E, hipStream_t s);
// dx / dWg / dWe1 / dWe2 (any may be null) from the forward's MoeWork (with pre).
// Phases of the MoE backward (run in this order; a caller may issue them as
// separate calls to time them): the expert-grouped products (dpre2 = dout
// We2[e]^T, the per-row routing gradients, dx), the router's dWg = x^T dg,
// and the K-grouped weight gradients dWe1, dWe2.
constexpr int kMoeBwdGrouped = 1, kMoeBwdGate = 2, kMoeBwdKGrouped = 4, kMoeBwdAll = 7;
int launch_moe_backward(const float* x, const float* dout, const float* Wg, const float* We1, const float* We2,
                        const uint8_t* active, const MoeWork& w, const MoeBwdWork& b, float* dx, float* dWg,
                        float* dWe1, float* dWe2, int64_t M, int64_t D, int64_t H, int64_t E, hipStream_t s,
                        int phases = kMoeBwdAll);

}  // namespace nship
