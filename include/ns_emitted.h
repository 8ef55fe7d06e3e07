/*
 * ns_emitted.h -- the other visible symbols of a per-network library: the
 * emitted translation unit's entry function and training core, which the
 * reference's code generator exports beside the ns_runtime.h ABI (internal
 * in the reference, but extern "C" and so callable; its own test hosts call
 * the entry function directly, e.g. test_codegen_cpu.cpp:97,
 * test_datamove.cpp:119).  Per-network libraries built by
 * neuralscript_amd/emit.py export them with the reference's names and
 * argument meanings; the work is done by libnship (nsh_forward,
 * nsh_train_core).
 */
#ifndef NSHIP_NS_EMITTED_H
#define NSHIP_NS_EMITTED_H

#include <stddef.h>
#include <stdint.h>

#include "ns_runtime.h"

#ifdef __cplusplus
extern "C" {
#endif

/* The entry function, `forward` unless the compiler was given another
 * function name (codegen.cpp:2263-2265, CUDA :552): output = the network on
 * `input` (n floats) with the weight blob `weights`, read on every call;
 * MoE networks take `moe_active` (one byte per expert, nonzero = live; NULL
 * = every expert live, ns_moe_fwd codegen.cpp:1915-1945).  No return value,
 * as in the reference (a failure leaves the output unwritten and its
 * message in nsh_last_error()).  One call at a time, as the reference's
 * static buffers require.  A MoE network's library exports the same name
 * with one more argument, as the reference emits it:
 *   void forward(const float* input, const float* weights, float* output,
 *                size_t n, const uint8_t* moe_active);
 * (declare that prototype instead when binding such a library). */
void forward(const float* input, const float* weights, float* output, size_t n);

/* The training core (codegen.cpp:2753-2755, CUDA :3249): the context is the
 * model returned by ns_runtime_init (the reference passes its model's ctx).
 * Weights read from w; forward, then with train_mode the backward and one
 * optimizer step at lr exactly (no schedule, no step counter: the
 * wrappers' business); the mean loss to *loss_out; with train_mode and a
 * non-NULL wout the updated weights to wout. */
typedef ns_model ns_cpu_ctx;
void ns_train_core(ns_cpu_ctx* ctx, const float* x, size_t nx, const float* y, const float* w, float* wout,
                   float* loss_out, float lr, int train_mode);

#ifdef __cplusplus
}
#endif

#endif /* NSHIP_NS_EMITTED_H */
