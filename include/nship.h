/*
 * nship.h -- C-ABI of libnship, the MI355X (gfx950) HIP backend behind the
 * NeuralScript runtime ABI.
 *
 * Three layers, all plain C types (no HIP or torch types in signatures):
 *
 *  1. Plans.  A network is described by the text the reference compiler
 *     prints for `nsc <net>.ns --mlir` (printer:
 *     /root/reference/src/mlir/mlir_compiler.cpp:949-1025).  It replaces the
 *     code the reference generates per network (gen_cpu / gen_cuda,
 *     /root/reference/src/codegen/codegen.cpp:306-1132, 1133-2657): instead
 *     of emitting kernels, the backend interprets the instruction list with
 *     fixed, hand-written gfx950 kernels.  Attributes the printer drops can be
 *     added to an instruction's trailing comment as key=value
 *     (`initial=K0` on ns.layer.moe for MoE(initial_experts: K0)).
 *
 *  2. Models.  nsh_model_* / nsh_* mirror the ns_* runtime functions one for
 *     one (ns_runtime.h); a per-network library (see neuralscript_amd/emit.py)
 *     binds one plan and exports the ns_* names as thin wrappers.
 *     nsh_*_device variants take device pointers and enqueue on the model's
 *     stream without host copies.
 *
 *  3. Kernels.  nsh_op_* run one hand-written kernel family on device
 *     pointers (synchronously), for hosts that drive the kernels directly and
 *     for per-kernel parity tests.  Each cites the reference function whose
 *     arithmetic it reproduces.
 *
 * Errors: functions return 0 / -1 (NULL for constructors) like the reference;
 * nsh_last_error() gives the calling thread's last message.
 */
#ifndef NSHIP_H
#define NSHIP_H

#include <stddef.h>
#include <stdint.h>

#include "ns_runtime.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct nsh_plan nsh_plan;

/* ---- errors and device helpers ---------------------------------------- */
const char* nsh_last_error(void);
int nsh_device_count(void);
/* Device memory for hosts (and tests) that do not own a HIP allocator. */
void* nsh_dev_alloc(size_t bytes);
int nsh_dev_free(void* p);
/* The copies wait for the whole device first (every model's stream). */
int nsh_memcpy_h2d(void* dst, const void* src, size_t bytes);
int nsh_memcpy_d2h(void* dst, const void* src, size_t bytes);
int nsh_memset_d(void* dst, int value, size_t bytes);
int nsh_device_synchronize(void);

/* ---- plans (replace the per-network generated driver tables,
 *      codegen.cpp:2438-2466 / 917-941) ------------------------------------ */
nsh_plan* nsh_plan_parse(const char* ir_text);
void nsh_plan_free(nsh_plan* p);
size_t nsh_plan_weight_count(const nsh_plan* p);              /* ns_weight_total */
const ns_weight_layout* nsh_plan_layout(const nsh_plan* p);   /* ns_layout */
size_t nsh_plan_output_numel(const nsh_plan* p, size_t input_numel); /* codegen.cpp:2481-2483 */
int nsh_plan_has_train(const nsh_plan* p);
int nsh_plan_has_moe(const nsh_plan* p);
size_t nsh_plan_in_cols(const nsh_plan* p);
size_t nsh_plan_out_cols(const nsh_plan* p);

/* ---- models: one per ns_* function ------------------------------------- */
ns_model* nsh_model_init(const nsh_plan* p, const float* weights, size_t num_floats); /* codegen.cpp:2467-2474 */
void nsh_model_free(ns_model* m);                                                    /* :2497-2499 */
int nsh_eval_infer(ns_model* m, const float* input, float* output, size_t input_numel); /* :2475-2480 */
size_t nsh_model_weight_count(const ns_model* m);
int nsh_model_get_weights(const ns_model* m, float* out, size_t n);                  /* :2490-2494 */
int nsh_save_checkpoint(const ns_model* m, const char* path);                        /* :2505-2528 */
int nsh_load_checkpoint(ns_model* m, const char* path);                              /* :2529-2557 */
size_t nsh_expert_count(const ns_model* m);                                          /* :2562-2565 */
size_t nsh_expert_birth(ns_model* m, int n);                                         /* :2567-2595 */
size_t nsh_expert_merge(ns_model* m, int a, int b);                                  /* :2597-2617 */
size_t nsh_expert_kill(ns_model* m, int k);                                          /* :2619-2626 */
int nsh_train_step(ns_model* m, const float* input, const float* labels,
                   size_t input_numel, float* loss_out, float lr);                   /* :2636-2644 */
int nsh_objective_loss(ns_model* m, const float* input, const float* labels,
                       size_t input_numel, float* loss_out);                         /* :2645-2651 */

/* The other visible symbols of the emitted TU.
 * nsh_forward: `forward(input, weights, output, n[, moe_active])`
 * (codegen.cpp:2263-2288): the weights come with the call and are read on
 * every call; moe_active (MoE plans) NULL = every expert live.  The plan
 * keeps one model for it (made on the first call, freed with the plan); like
 * the reference's static buffers it serves one call at a time.
 * nsh_train_core: `ns_train_core(ctx, x, nx, y, w, wout, loss_out, lr,
 * train_mode)` (codegen.cpp:2753-3157) over model m: weights read from w,
 * forward (+ backward and one optimizer step at lr exactly, train_mode != 0),
 * the loss to *loss_out, the updated weights to wout (train_mode, wout not
 * NULL); no LR schedule, no step counter (the wrapper's).
 * nsh_model_set_weights / nsh_model_set_expert_mask: replace the model's
 * blob (n == weight count) / liveness mask (NULL = all live) and re-sync
 * the device copies. */
int nsh_forward(const nsh_plan* p, const float* input, const float* weights, float* output, size_t input_numel,
                const uint8_t* moe_active);
int nsh_train_core(ns_model* m, const float* x, size_t nx, const float* y, const float* w, float* wout,
                   float* loss_out, float lr, int train_mode);
int nsh_model_set_weights(ns_model* m, const float* w, size_t n);
int nsh_model_set_expert_mask(ns_model* m, const uint8_t* active);
/* The wrapper's LR multiplier at step `step` (optim_params.hpp:54-62): the
 * schedule named by the IR line `// ns.lr_schedule <constant|cosine_warmup>
 * warmup=W total=T min=F`, constant when absent (the reference's default). */
float nsh_plan_lr_scale(const nsh_plan* p, int64_t step);

/* Device-resident forward: input/output are device pointers; enqueued on the
 * model's stream, returns before completion (nsh_model_sync waits). */
int nsh_eval_infer_device(ns_model* m, const float* d_input, float* d_output, size_t input_numel);
int nsh_model_sync(ns_model* m);

/* Device-resident training step (inputs and one-hot labels in device
 * memory); loss_out is a host pointer (NULL: no wait, no loss). */
int nsh_train_step_device(ns_model* m, const float* d_input, const float* d_labels, size_t input_numel,
                          float* loss_out, float lr);

/* Copy of IR value `name` (e.g. "g17", "attn8") as left by the most recent
 * forward or training call; weights give their current values.  For
 * per-instruction parity checks.  n must equal the value's element count. */
int nsh_model_read_value(ns_model* m, const char* name, float* out, size_t n);

/* Routing of the most recent MoE forward of n tokens: chosen expert (-1 if
 * none live), its probability, and the raw router logits [n, E].  Any output
 * may be NULL. */
int nsh_model_last_routing(ns_model* m, int32_t* best, float* prob, float* logits, size_t n);

/* Per-kernel timing with HIP events recorded on the model's stream around
 * every launch.  The report is one JSON object: kernel -> {calls, ms}. */
int nsh_profile_enable(ns_model* m, int on);
/* Limit the event pairs to the listed regions (comma-separated names, e.g.
 * "attention_bwd,gemm"); NULL or "" times every region.  Each event pair
 * leaves a gap of a few microseconds between launches, so a timed run that
 * needs only one region's figure selects it. */
int nsh_profile_select(ns_model* m, const char* regions);
int nsh_profile_reset(ns_model* m);
int nsh_profile_report(ns_model* m, char* buf, size_t len);

/* ---- kernels on device pointers (synchronous) --------------------------- */

/* C[M,N] = opA(A) opB(B) then activation `act` (0 id, 1 relu, 2 leaky,
 * 3 sigmoid, 4 tanh, 5 silu, 6 gelu).  opA(A)[m,k] = transA ? A[k*lda+m] :
 * A[m*lda+k]; opB(B)[k,n] = transB ? B[n*ldb+k] : B[k*ldb+n].
 * Replaces ns_matmul + ns_act2 (codegen.cpp:1257-1265, 1244-1255),
 * ns_matmul_grad_a (transB, :1318-1326) and ns_matmul_grad_w (transA,
 * :1329-1337); fp32 MFMA. */
int nsh_op_gemm(const float* A, const float* B, float* C, int64_t M, int64_t N, int64_t K,
                int64_t lda, int64_t ldb, int64_t ldc, int transA, int transB, int act);

/* nsh_op_gemm with K split into `splits` chunks (0: the runtime's heuristic,
 * the one its plans use): per-chunk partials into `workspace`, summed in
 * chunk order, then the activation; the same operation as nsh_op_gemm, with
 * the reduction over k reassociated.  The workspace holds
 * nsh_op_gemm_splitk_workspace(...) bytes. */
size_t nsh_op_gemm_splitk_workspace(int64_t M, int64_t N, int64_t K, int splits);
int nsh_op_gemm_splitk(const float* A, const float* B, float* C, int64_t M, int64_t N, int64_t K,
                       int64_t lda, int64_t ldb, int64_t ldc, int transA, int transB, int act, int splits,
                       void* workspace);

/* out[i,:] = W[row(idx[i]),:], out-of-range or non-integral-range ids -> row 0;
 * ns_embedding, codegen.cpp:1711-1718. */
int nsh_op_embedding(const float* W, const float* idx, float* out, int64_t n, int64_t V, int64_t D);

/* Row LayerNorm, no affine, eps 1e-5; ns_layernorm, codegen.cpp:1280-1291. */
int nsh_op_layernorm(const float* x, float* y, int64_t rows, int64_t last);

/* The reference's LayerNorm gradient; ns_layernorm_grad, codegen.cpp:1346-1371. */
int nsh_op_layernorm_grad(const float* dout, const float* x, float* dx, int64_t rows, int64_t last);

/* Softmax cross-entropy over rows of C: row_loss[r] = -sum_{y>0} log p,
 * *loss = mean over rows, grad = (p - y) / rows (skipped when grad is NULL);
 * ns_cross_entropy / ns_loss_grad, codegen.cpp:1582-1613.  loss and
 * row_loss are device pointers. */
int nsh_op_softmax_xent(const float* logits, const float* labels, float* grad, float* row_loss, float* loss,
                        int64_t rows, int64_t C);

/* dout = din * act'(pre); ns_act_grad, codegen.cpp:1340-1343. */
int nsh_op_act_grad(const float* din, const float* pre, float* dout, int64_t n, int act);

/* dW[V,D] = scatter-add of dout rows by index, in token order (bit-exact
 * with the reference's sequential loop); ns_embedding_grad_w,
 * codegen.cpp:1374-1383.  `workspace`: device bytes from
 * nsh_op_embedding_grad_workspace. */
size_t nsh_op_embedding_grad_workspace(int64_t n, int64_t V);
int nsh_op_embedding_grad(const float* dout, const float* idx, float* dW, int64_t n, int64_t V, int64_t D,
                          void* workspace);

/* nsh_op_embedding_grad without any allocation.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, serving loops, harnesses that forbid hipMalloc).  The
 * sort state lives in a static device array of
 * NSH_EMBEDDING_GRAD_NOALLOC_MAX_INTS ints (4 MiB, held by every GPU the
 * library runs on until the process ends); sizes with 3*V + 1 + 2*n above it
 * return -1.  The kernels are enqueued on `stream` (a hipStream_t; NULL = the
 * null stream) and the call returns without waiting.  Every call on one GPU
 * shares that array: calls that overlap on one GPU (other streams, other
 * threads) race and must be serialised by the caller.  Same result as
 * nsh_op_embedding_grad, bit for bit. */
#define NSH_EMBEDDING_GRAD_NOALLOC_MAX_INTS 1048576
int nsh_op_embedding_grad_noalloc(const float* dout, const float* idx, float* dW, int64_t n, int64_t V, int64_t D,
                                  void* stream);

/* Attention core over one sequence of S tokens: ctx[S,D] = per-head
 * softmax(Q K^T / sqrt(D/H)) V; Q, K, V are [S, D]; lse (optional, [H, S])
 * receives each query's log2-sum-exp of the log2e-scaled scores; the core
 * of ns_attention_fwd, codegen.cpp:1724-1777. */
int nsh_op_attention_fwd(const float* Q, const float* K, const float* V, float* ctx, float* lse, int64_t S,
                         int64_t D, int64_t H);

/* Backward of the attention core: dQ, dK, dV [S, D] from Q, K, V, the
 * forward's ctx (O), dO = d ctx and lse (nsh_op_attention_fwd's), i.e. per
 * head the gradient of softmax(Q K^T / sqrt(D/H)) V; the core of the
 * ATTENTION_GRAD_* kernels, codegen.cpp:1785-1907.  workspace: bytes from
 * nsh_op_attention_bwd_workspace(S, D, H, store_ds).  store_ds != 0 keeps dS
 * (H*S*S floats, when S % 64 == 0 and the head size is 32 or 64) so that dQ
 * is one product over it instead of a pass that recomputes S and dP; the
 * result is the same to fp32 rounding. */
size_t nsh_op_attention_bwd_workspace(int64_t S, int64_t D, int64_t H, int store_ds);
int nsh_op_attention_bwd(const float* Q, const float* K, const float* V, const float* O, const float* dO,
                         const float* lse, float* dQ, float* dK, float* dV, int64_t S, int64_t D, int64_t H,
                         int store_ds, void* workspace);

/* Modified Gram-Schmidt of g [r,c] over columns (r >= c) or rows (r < c),
 * q = the orthonormal result in g's layout; ns_orthonom, codegen.cpp:1617-1633.
 * workspace: device bytes from nsh_op_muon_workspace. */
size_t nsh_op_muon_workspace(int64_t r, int64_t c);
int nsh_op_orthonormalize(const float* g, float* q, int64_t r, int64_t c, void* workspace);

/* Muon step of one matrix (momentum reset every step, so m = g):
 * w -= lr sqrt(min(r,c)) MGS(g) + 0.01 lr w; codegen.cpp:3099-3107. */
int nsh_op_muon_step(float* w, const float* g, int64_t r, int64_t c, float lr, void* workspace);

/* Muon step of n matrices at once (the fused multi-tensor form the training
 * step uses): w[i] [r[i], c[i]] updated with gradient g[i]. */
size_t nsh_op_muon_multi_workspace(int n, const int64_t* r, const int64_t* c);
int nsh_op_muon_multi(int n, float* const* w, const float* const* g, const int64_t* r, const int64_t* c, float lr,
                      void* workspace);

/* AdamW step with step counter t (after increment), moments m, v updated in
 * place; codegen.cpp:3108-3119. */
int nsh_op_adamw_step(float* w, const float* g, float* m, float* v, int64_t n, int64_t t, float lr);

/* Attainable peaks of the running GPU (no reference counterpart: the
 * reference has no timing).  nsh_bench_mfma_peak: register-only fp32 MFMA
 * loop, blocks x 256 threads, iters x 4 MFMA 32x32x2 per wave (4096 FLOP
 * each); *tflops = executed rate.  nsh_bench_copy: float4 copy of n floats
 * (n % 4 == 0, 16-byte aligned), mean over reps; *gbs = (read + write)
 * bytes / time. */
int nsh_bench_mfma_peak(int iters, int blocks, double* tflops);
int nsh_bench_copy(const float* src, float* dst, int64_t n, int reps, double* gbs);
/* The row kernels of a training step at one shape (no reference
 * counterpart), each timed over `reps` back-to-back launches between one
 * pair of events: us[0..4] = microseconds per launch of the embedding
 * gather [M] ids of a [V, D] table, LayerNorm and its gradient on [M, D],
 * the embedding gradient, and softmax cross-entropy with its gradient on
 * [M, C].  idx: M float ids, labels: [M, C] (device pointers); every other
 * buffer is allocated and freed by the call. */
int nsh_bench_rowops(const float* idx, const float* labels, int64_t M, int64_t D, int64_t V, int64_t C, int reps,
                     double* us);

#ifdef __cplusplus
}
#endif

#endif /* NSHIP_H */
