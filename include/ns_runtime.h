/*
 * ns_runtime.h -- the NeuralScript AOT runtime C-ABI, as exported by every
 * per-network library built on libnship (the MI355X HIP backend).
 *
 * Same functions, argument meanings, struct layouts and 0 / -1 / NULL error
 * convention as the reference interface
 * /root/reference/include/ns/runtime/ns_runtime.h:30-129 (ABI 1.2.0), so a
 * host written against the reference links against this backend unchanged.
 * Each declaration cites the reference line it replaces.
 *
 * Backend-specific behaviour (all within the reference contract):
 *  - weights live in device memory (HBM); the host copy is synchronised
 *    lazily, so ns_model_get_weights / ns_save_checkpoint return the current
 *    trained weights and ns_load_checkpoint re-uploads them;
 *  - calls are synchronous with respect to the host; one call at a time per
 *    model (each model owns a private HIP stream);
 *  - device failures make the call return -1 (the reference's CUDA driver
 *    returns 0 silently there); the message is in nsh_last_error().
 */
#ifndef NSHIP_NS_RUNTIME_H
#define NSHIP_NS_RUNTIME_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NS_RUNTIME_VERSION_MAJOR 1
#define NS_RUNTIME_VERSION_MINOR 2
#define NS_RUNTIME_VERSION_PATCH 0
#define NS_RUNTIME_VERSION "1.2.0"

typedef struct ns_model ns_model;

/* ns_runtime.h:33-37 */
typedef struct ns_weight_desc {
    const char* name;
    size_t offset; /* in floats */
    size_t count;  /* in floats */
} ns_weight_desc;

/* ns_runtime.h:40-43 */
typedef struct ns_weight_layout {
    size_t num_weights;
    const ns_weight_desc* desc;
} ns_weight_layout;

/* ns_runtime.h:48 -- copies the blob; NULL unless num_floats matches. */
ns_model* ns_runtime_init(const float* weights, size_t num_floats);

/* ns_runtime.h:54 -- host pointers; writes the forward result. */
int ns_eval_infer(ns_model* m, const float* input, float* output, size_t input_numel);

/* ns_runtime.h:57 -- (input_numel / in_cols) * out_cols. */
size_t ns_model_output_numel(const ns_model* m, size_t input_numel);

/* ns_runtime.h:60 */
size_t ns_model_weight_count(const ns_model* m);

/* ns_runtime.h:65 */
size_t ns_weight_count_static(void);

/* ns_runtime.h:69 -- -1 on NULL arguments or n != weight count. */
int ns_model_get_weights(const ns_model* m, float* out, size_t n);

/* ns_runtime.h:72 */
const ns_weight_layout* ns_model_layout(const ns_model* m);

/* ns_runtime.h:75 -- NULL-safe. */
void ns_free(ns_model* m);

/* ns_runtime.h:81 -- NSM2 file: magic, u64 count, weights, MoE tail. */
int ns_save_checkpoint(const ns_model* m, const char* path);

/* ns_runtime.h:86 -- NSM1 / NSM2; re-syncs the device blob and mask. */
int ns_load_checkpoint(ns_model* m, const char* path);

/* ns_runtime.h:106-109 -- MoE expert lifecycle (MoE networks only). */
size_t ns_expert_count(const ns_model* m);
size_t ns_expert_birth(ns_model* m, int n);
size_t ns_expert_merge(ns_model* m, int a, int b);
size_t ns_expert_kill(ns_model* m, int k);

/* ns_runtime.h:123-124 -- forward + backward + one optimizer step. */
int ns_runtime_train_step(ns_model* m, const float* input, const float* labels,
                          size_t input_numel, float* loss_out, float lr);

/* ns_runtime.h:128-129 -- loss only; never mutates weights. */
int ns_objective_loss(ns_model* m, const float* input, const float* labels,
                      size_t input_numel, float* loss_out);

#ifdef __cplusplus
}
#endif

#endif /* NSHIP_NS_RUNTIME_H */
