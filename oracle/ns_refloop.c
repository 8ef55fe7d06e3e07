/*
 * ns_refloop.c -- the NeuralScript CPU runtime kernels in the REFERENCE'S OWN
 * loop order: the CPU-baseline restatement timed beside the GPU.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (libnship) links, loads or
 * calls this file; only tests/ and bench.py's cpu_baseline leg use it.
 *
 * ns_oracle.c (the checker) reorders work across independent outputs and runs
 * threaded; this file keeps the loop nests of the code the reference emits for
 * `nsc --cpp --runtime` (all in /root/reference/src/codegen/codegen.cpp, cited
 * per function): i-j-k products with the k loop innermost, the attention's
 * S x S score matrix per head, the per-token MoE loop, the left-looking
 * Gram-Schmidt over strided columns.  It is built like the reference's tests
 * build the emitted driver (gcc -O2, no -march, so no FMA; one thread) and
 * exports the checker's `or_*` interface, so the same sequencing code
 * (oracle.py) drives either library.  tests/test_oracle.py pins it bitwise to
 * the reference fixtures and to the checker.
 *
 * Sampling hooks for bounded baselines (rl_*): the same nests over a subrange
 * of query rows, and per-part timers of the attention functions, so that a
 * few rows can stand for the whole workload (rows are independent given K/V).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#define EXPORT __attribute__((visibility("default")))

static double now_s(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

/* std::max(a, b) as libstdc++ defines it: (a < b) ? b : a */
static inline float smax(float a, float b) { return (a < b) ? b : a; }

/* ns_act2 codegen.cpp:1244-1255 */
static float act2(float x, int code) {
    switch (code) {
    case 1: return x > 0 ? x : 0.f;
    case 2: return x > 0 ? x : 0.01f * x;
    case 3: return 1.f / (1.f + expf(-x));
    case 4: return tanhf(x);
    case 5: return x / (1.f + expf(-x));
    case 6: return 0.5f * x * (1.f + erff(x / 1.41421356f));
    default: return x;
    }
}

/* ns_act_deriv codegen.cpp:1305-1315 */
static float act_deriv(float x, int code) {
    switch (code) {
    case 1: return x > 0.f ? 1.f : 0.f;
    case 2: return x > 0.f ? 1.f : 0.01f;
    case 3: { float s = 1.f / (1.f + expf(-x)); return s * (1.f - s); }
    case 4: { float t = tanhf(x); return 1.f - t * t; }
    case 5: { float s = x / (1.f + expf(-x)); return s + x * (1.f - s); }
    case 6: {
        float u = x / 1.41421356f;
        float p = 0.5f * (1.f + erff(u));
        return p + x * expf(-u * u) / 2.50662827f;
    }
    default: return 1.f;
    }
}

EXPORT void or_act(const float* in, float* out, size_t n, int code) {
    for (size_t i = 0; i < n; i++) out[i] = act2(in[i], code);
}

/* ns_act_grad codegen.cpp:1340-1343 */
EXPORT void or_act_grad(const float* din, const float* pre, float* dout, size_t n, int code) {
    for (size_t i = 0; i < n; i++) dout[i] = din[i] * act_deriv(pre[i], code);
}

/* ns_matmul codegen.cpp:1257-1265 over rows [i0, i1): i, then j, then the
 * k reduction (B read with stride N). */
static void gemm_rows(const float* A, const float* B, float* C, int64_t i0, int64_t i1, int64_t K, int64_t N) {
    for (int64_t i = i0; i < i1; i++)
        for (int64_t j = 0; j < N; j++) {
            float acc = 0.f;
            for (int64_t k = 0; k < K; k++) acc += A[(size_t)i * K + k] * B[(size_t)k * N + j];
            C[(size_t)i * N + j] = acc;
        }
}

/* FUSED matmul + activation: the product, then the epilogue's elementwise
 * pass over the whole result (codegen.cpp:2034-2078). */
EXPORT void or_matmul(const float* A, const float* B, float* C, int64_t M, int64_t K, int64_t N, int act) {
    gemm_rows(A, B, C, 0, M, K, N);
    if (act)
        for (size_t i = 0; i < (size_t)M * N; i++) C[i] = act2(C[i], act);
}

EXPORT void or_matmul_rows(const float* A, const int64_t* rows, int64_t R, const float* B, float* C, int64_t K,
                           int64_t N, int act) {
    for (int64_t r = 0; r < R; r++) {
        const float* a = A + (size_t)rows[r] * K;
        for (int64_t j = 0; j < N; j++) {
            float acc = 0.f;
            for (int64_t k = 0; k < K; k++) acc += a[k] * B[(size_t)k * N + j];
            C[(size_t)r * N + j] = act ? act2(acc, act) : acc;
        }
    }
}

/* ns_matmul_grad_a codegen.cpp:1318-1326: i, k, then j */
EXPORT void or_matmul_grad_a(const float* dC, const float* B, float* dA, int64_t M, int64_t K, int64_t N) {
    for (int64_t i = 0; i < M; i++)
        for (int64_t k = 0; k < K; k++) {
            float acc = 0.f;
            for (int64_t j = 0; j < N; j++) acc += dC[(size_t)i * N + j] * B[(size_t)k * N + j];
            dA[(size_t)i * K + k] = acc;
        }
}

/* ns_matmul_grad_w codegen.cpp:1329-1337: k, j, then i */
EXPORT void or_matmul_grad_w(const float* A, const float* dC, float* dB, int64_t M, int64_t K, int64_t N) {
    for (int64_t k = 0; k < K; k++)
        for (int64_t j = 0; j < N; j++) {
            float acc = 0.f;
            for (int64_t i = 0; i < M; i++) acc += A[(size_t)i * K + k] * dC[(size_t)i * N + j];
            dB[(size_t)k * N + j] = acc;
        }
}

/* ns_layernorm codegen.cpp:1280-1291 on a copy of the input (:2020-2025) */
EXPORT void or_layernorm(const float* in, float* out, size_t numel, int64_t last) {
    if (out != in) memcpy(out, in, numel * sizeof(float));
    const int64_t rows = (int64_t)numel / last;
    for (int64_t r = 0; r < rows; r++) {
        float* m = out + (size_t)r * last;
        float mean = 0.f, var = 0.f;
        for (int64_t j = 0; j < last; j++) mean += m[j];
        mean /= last;
        for (int64_t j = 0; j < last; j++) { float d = m[j] - mean; var += d * d; }
        var /= last;
        float inv = 1.f / sqrtf(var + 1e-5f);
        for (int64_t j = 0; j < last; j++) m[j] = (m[j] - mean) * inv;
    }
}

/* ns_softmax codegen.cpp:1293-1303 on a copy of the input */
EXPORT void or_softmax(const float* in, float* out, size_t numel, int64_t last) {
    if (out != in) memcpy(out, in, numel * sizeof(float));
    const int64_t rows = (int64_t)numel / last;
    for (int64_t r = 0; r < rows; r++) {
        float* m = out + (size_t)r * last;
        float mx = m[0];
        for (int64_t j = 1; j < last; j++) mx = smax(mx, m[j]);
        float s = 0.f;
        for (int64_t j = 0; j < last; j++) { m[j] = expf(m[j] - mx); s += m[j]; }
        for (int64_t j = 0; j < last; j++) m[j] /= s;
    }
}

/* ns_layernorm_grad codegen.cpp:1346-1371 */
EXPORT void or_layernorm_grad(const float* dout, const float* x, float* dx, size_t numel, int64_t last) {
    const int64_t rows = (int64_t)numel / last;
    for (int64_t r = 0; r < rows; r++) {
        float mean_x = 0.f, mean_dout = 0.f;
        for (int64_t j = 0; j < last; j++) {
            mean_x += x[(size_t)r * last + j];
            mean_dout += dout[(size_t)r * last + j];
        }
        mean_x /= last;
        mean_dout /= last;
        float var_x = 0.f, gamma = 0.f;
        for (int64_t j = 0; j < last; j++) {
            float xj = x[(size_t)r * last + j] - mean_x;
            var_x += xj * xj;
            gamma += xj * dout[(size_t)r * last + j];
        }
        var_x /= last;
        gamma /= last;
        float inv = 1.f / sqrtf(var_x + 1e-5f);
        for (int64_t j = 0; j < last; j++) {
            float xj = x[(size_t)r * last + j] - mean_x;
            dx[(size_t)r * last + j] = (dout[(size_t)r * last + j] - mean_dout - xj * gamma) * inv;
        }
    }
}

/* The (int64_t) cast of a float index, with the cases C leaves undefined
 * (NaN, beyond int64) mapped to out of range as x86's conversion does. */
static inline int64_t emb_row(float f, int64_t V) {
    if (!(f > -1.0f) || !(f < (float)V)) return -1;
    int64_t k = (int64_t)f;
    return (k < 0 || k >= V) ? -1 : k;
}

/* ns_embedding codegen.cpp:1711-1718 */
EXPORT void or_embedding(const float* W, const float* idx, float* out, int64_t n, int64_t V, int64_t D) {
    for (int64_t i = 0; i < n; i++) {
        int64_t k = emb_row(idx[i], V);
        if (k < 0) k = 0;
        memcpy(out + (size_t)i * D, W + (size_t)k * D, (size_t)D * sizeof(float));
    }
}

EXPORT void or_embedding_rows(const float* idx, int64_t* rows, int64_t n, int64_t V) {
    for (int64_t i = 0; i < n; i++) rows[i] = emb_row(idx[i], V);
}

/* ns_embedding_grad_w codegen.cpp:1374-1383 */
EXPORT void or_embedding_grad_w(const float* dout, const float* idx, float* dW, size_t M, int64_t D, int64_t V) {
    for (int64_t k = 0; k < V * D; k++) dW[k] = 0.f;
    for (size_t i = 0; i < M; i++) {
        int64_t row = emb_row(idx[i], V);
        if (row < 0) continue;
        for (int64_t j = 0; j < D; j++) dW[(size_t)row * D + j] += dout[i * D + j];
    }
}

/* ns_cross_entropy codegen.cpp:1598-1613 */
EXPORT float or_cross_entropy(const float* preds, const float* labels, size_t numel, int64_t C) {
    const int64_t rows = (int64_t)numel / C;
    float loss = 0.f;
    for (int64_t r = 0; r < rows; r++) {
        const float* p = preds + (size_t)r * C;
        float mx = p[0];
        for (int64_t j = 1; j < C; j++) mx = smax(mx, p[j]);
        float s = 0.f;
        for (int64_t j = 0; j < C; j++) s += expf(p[j] - mx);
        for (int64_t j = 0; j < C; j++) {
            float pj = expf(p[j] - mx) / s;
            if (labels[(size_t)r * C + j] > 0.f) loss -= logf(pj);
        }
    }
    return loss / (float)rows;
}

/* ns_loss_grad codegen.cpp:1582-1595 */
EXPORT void or_loss_grad(const float* preds, const float* labels, float* d, size_t numel, int64_t C) {
    const int64_t rows = (int64_t)numel / C;
    for (int64_t r = 0; r < rows; r++) {
        const float* p = preds + (size_t)r * C;
        float mx = p[0];
        for (int64_t j = 1; j < C; j++) mx = smax(mx, p[j]);
        float s = 0.f;
        for (int64_t j = 0; j < C; j++) s += expf(p[j] - mx);
        for (int64_t j = 0; j < C; j++) {
            float pj = expf(p[j] - mx) / s;
            d[(size_t)r * C + j] = (pj - labels[(size_t)r * C + j]) / (float)rows;
        }
    }
}

/* ------------------------------------------------------------------------ */
/* attention over one sequence (S = BS), ns_attention_fwd codegen.cpp:1724-1777 */
/* ------------------------------------------------------------------------ */

/* Per-part times of the last or_attention_fwd / or_attention_bwd call (s):
 * [0] projections (the D x D products and dPre), [1] the per-head S x S
 * loops, [2..6] the backward's per-output tails (dWq, dWk, dWv, dWo, dX). */
static double g_split[8];

EXPORT void rl_last_attention_split(double* out) { memcpy(out, g_split, sizeof(g_split)); }

/* The per-head part of the forward for query rows [i0, i1): scores against
 * all S keys into sc (row i at sc[(i - i0) * S]), row softmax, then
 * ctx[i, h*Dk + d] = sum_j sc[i, j] V[j, h*Dk + d] (codegen.cpp:1747-1772). */
static void attn_core_rows(const float* Q, const float* K, const float* V, float* ctx, float* sc, int64_t S,
                           int64_t D, int64_t H, int64_t i0, int64_t i1) {
    const int64_t Dk = D / H;
    const float scale = 1.0f / sqrtf((float)Dk);
    for (int64_t h = 0; h < H; h++) {
        for (int64_t i = i0; i < i1; i++) {
            float* row = sc + (size_t)(i - i0) * S;
            for (int64_t j = 0; j < S; j++) {
                float a = 0.f;
                for (int64_t d = 0; d < Dk; d++) a += Q[(size_t)i * D + h * Dk + d] * K[(size_t)j * D + h * Dk + d];
                row[j] = a * scale;
            }
        }
        for (int64_t i = i0; i < i1; i++) {
            float* row = sc + (size_t)(i - i0) * S;
            float mx = row[0];
            for (int64_t j = 1; j < S; j++) mx = smax(mx, row[j]);
            float s = 0.f;
            for (int64_t j = 0; j < S; j++) { row[j] = expf(row[j] - mx); s += row[j]; }
            for (int64_t j = 0; j < S; j++) row[j] /= s;
        }
        for (int64_t i = i0; i < i1; i++)
            for (int64_t d = 0; d < Dk; d++) {
                float a = 0.f;
                for (int64_t j = 0; j < S; j++) a += sc[(size_t)(i - i0) * S + j] * V[(size_t)j * D + h * Dk + d];
                ctx[(size_t)i * D + h * Dk + d] = a;
            }
    }
}

EXPORT void or_attention_fwd(const float* x, const float* Wq, const float* Wk, const float* Wv, const float* Wo,
                             float* out, int64_t BS, int64_t D, int64_t H) {
    const size_t n = (size_t)BS * D;
    float* Q = (float*)malloc(n * sizeof(float));
    float* K = (float*)malloc(n * sizeof(float));
    float* V = (float*)malloc(n * sizeof(float));
    float* ctx = (float*)malloc(n * sizeof(float));
    float* sc = (float*)malloc((size_t)BS * BS * sizeof(float));
    double t0 = now_s();
    gemm_rows(x, Wq, Q, 0, BS, D, D);
    gemm_rows(x, Wk, K, 0, BS, D, D);
    gemm_rows(x, Wv, V, 0, BS, D, D);
    double t1 = now_s();
    attn_core_rows(Q, K, V, ctx, sc, BS, D, H, 0, BS);
    double t2 = now_s();
    gemm_rows(ctx, Wo, out, 0, BS, D, D);
    double t3 = now_s();
    memset(g_split, 0, sizeof(g_split));
    g_split[0] = (t1 - t0) + (t3 - t2);
    g_split[1] = t2 - t1;
    free(Q); free(K); free(V); free(ctx); free(sc);
}

/* Sampling hook: the per-head loops for query rows [i0, i1) only, given
 * full Q, K, V [S, D]; returns the seconds they took. */
EXPORT double rl_attention_core_rows(const float* Q, const float* K, const float* V, float* ctx, int64_t S,
                                     int64_t D, int64_t H, int64_t i0, int64_t i1) {
    float* sc = (float*)malloc((size_t)(i1 - i0) * S * sizeof(float));
    double t0 = now_s();
    attn_core_rows(Q, K, V, ctx, sc, S, D, H, i0, i1);
    double t = now_s() - t0;
    free(sc);
    return t;
}

/* The per-head part of ns_attention_bwd (codegen.cpp:1846-1893) for head h:
 * the loops over query rows run over [0, ni), the loops over key rows over
 * [0, nj) (the full backward uses ni = nj = S); sc and ds are S x S, dp
 * holds ni rows.  t[0] += seconds in the query-row loops, t[1] += seconds in
 * the key-row loops. */
static void attn_bwd_head(const float* Qq, const float* Kk, const float* Vv, const float* dPre, float* oh,
                          float* dQ2, float* dK2, float* dV2, float* sc, float* dp, float* ds, int64_t S, int64_t D,
                          int64_t H, int64_t h, int64_t ni, int64_t nj, double* t) {
    const int64_t Dk = D / H, o = h * Dk;
    const float scale = 1.0f / sqrtf((float)Dk);
    double t0 = now_s();
    for (int64_t i = 0; i < ni; i++) {
        for (int64_t j = 0; j < S; j++) {
            float a = 0.f;
            for (int64_t d = 0; d < Dk; d++) a += Qq[(size_t)i * D + o + d] * Kk[(size_t)j * D + o + d];
            sc[(size_t)i * S + j] = a * scale;
        }
        float mx = sc[(size_t)i * S];
        for (int64_t j = 1; j < S; j++) mx = smax(mx, sc[(size_t)i * S + j]);
        float s = 0.f;
        for (int64_t j = 0; j < S; j++) { sc[(size_t)i * S + j] = expf(sc[(size_t)i * S + j] - mx); s += sc[(size_t)i * S + j]; }
        for (int64_t j = 0; j < S; j++) sc[(size_t)i * S + j] /= s;
    }
    for (int64_t i = 0; i < ni; i++)
        for (int64_t d = 0; d < Dk; d++) {
            float a = 0.f;
            for (int64_t j = 0; j < S; j++) a += sc[(size_t)i * S + j] * Vv[(size_t)j * D + o + d];
            oh[(size_t)i * D + o + d] = a;
        }
    double t1 = now_s();
    for (int64_t j = 0; j < nj; j++)
        for (int64_t d = 0; d < Dk; d++) {
            float a = 0.f;
            for (int64_t i = 0; i < S; i++) a += sc[(size_t)i * S + j] * dPre[(size_t)i * D + o + d];
            dV2[(size_t)j * D + o + d] += a;
        }
    double t2 = now_s();
    for (int64_t i = 0; i < ni; i++) {
        for (int64_t j = 0; j < S; j++) {
            float a = 0.f;
            for (int64_t d = 0; d < Dk; d++) a += Vv[(size_t)j * D + o + d] * dPre[(size_t)i * D + o + d];
            dp[(size_t)i * S + j] = a;
        }
        float dot = 0.f;
        for (int64_t j = 0; j < S; j++) dot += sc[(size_t)i * S + j] * dp[(size_t)i * S + j];
        for (int64_t j = 0; j < S; j++) ds[(size_t)i * S + j] = sc[(size_t)i * S + j] * (dp[(size_t)i * S + j] - dot);
    }
    for (int64_t i = 0; i < ni; i++)
        for (int64_t d = 0; d < Dk; d++) {
            float a = 0.f;
            for (int64_t j = 0; j < S; j++) a += ds[(size_t)i * S + j] * Kk[(size_t)j * D + o + d];
            dQ2[(size_t)i * D + o + d] += a * scale;
        }
    double t3 = now_s();
    for (int64_t j = 0; j < nj; j++)
        for (int64_t d = 0; d < Dk; d++) {
            float a = 0.f;
            for (int64_t i = 0; i < S; i++) a += ds[(size_t)i * S + j] * Qq[(size_t)i * D + o + d];
            dK2[(size_t)j * D + o + d] += a * scale;
        }
    double t4 = now_s();
    t[0] += (t1 - t0) + (t3 - t2);
    t[1] += (t2 - t1) + (t4 - t3);
}

/* Sampling hook: one head (h = 0) of the backward's S x S loops at full
 * sequence length S with ni query rows and nj key rows; Q, K, V, dPre are
 * [S, D], sc and ds S x S buffers whose other rows hold what the caller put
 * there.  out[0] = seconds of the query-row loops, out[1] of the key-row
 * loops. */
EXPORT void rl_attention_bwd_core_sample(const float* Q, const float* K, const float* V, const float* dPre,
                                         float* sc, float* ds, int64_t S, int64_t D, int64_t H, int64_t ni,
                                         int64_t nj, double* out) {
    const size_t n = (size_t)S * D;
    float* oh = (float*)calloc(n, sizeof(float));
    float* g = (float*)calloc(3 * n, sizeof(float));
    float* dp = (float*)malloc((size_t)(ni ? ni : 1) * S * sizeof(float));
    out[0] = out[1] = 0.0;
    attn_bwd_head(Q, K, V, dPre, oh, g, g + n, g + 2 * n, sc, dp, ds, S, D, H, 0, ni, nj, out);
    free(oh); free(g); free(dp);
}

/* ns_attention_bwd codegen.cpp:1785-1907.  Any output may be NULL (the
 * emitted train core calls it once per output, :3017-3051). */
EXPORT void or_attention_bwd(const float* dout, const float* x, const float* Wq, const float* Wk, const float* Wv,
                             const float* Wo, float* dX, float* dWq, float* dWk, float* dWv, float* dWo, int64_t BS,
                             int64_t D, int64_t H) {
    const int64_t S = BS;
    const size_t n = (size_t)BS * D;
    float* Qq = (float*)malloc(n * sizeof(float));
    float* Kk = (float*)malloc(n * sizeof(float));
    float* Vv = (float*)malloc(n * sizeof(float));
    float* dQ2 = (float*)calloc(n, sizeof(float));
    float* dK2 = (float*)calloc(n, sizeof(float));
    float* dV2 = (float*)calloc(n, sizeof(float));
    float* dPre = (float*)malloc(n * sizeof(float));
    float* oh = (float*)calloc(n, sizeof(float));
    float* sc = (float*)malloc((size_t)S * S * sizeof(float));
    float* dp = (float*)malloc((size_t)S * S * sizeof(float));
    float* ds = (float*)malloc((size_t)S * S * sizeof(float));
    memset(g_split, 0, sizeof(g_split));
    double t0 = now_s();
    gemm_rows(x, Wq, Qq, 0, BS, D, D);
    gemm_rows(x, Wk, Kk, 0, BS, D, D);
    gemm_rows(x, Wv, Vv, 0, BS, D, D);
    for (int64_t i = 0; i < BS; i++)
        for (int64_t k = 0; k < D; k++) {
            float a = 0.f;
            for (int64_t m = 0; m < D; m++) a += dout[(size_t)i * D + m] * Wo[(size_t)k * D + m];
            dPre[(size_t)i * D + k] = a;
        }
    double t1 = now_s();
    double th[2] = {0.0, 0.0};
    for (int64_t h = 0; h < H; h++)
        attn_bwd_head(Qq, Kk, Vv, dPre, oh, dQ2, dK2, dV2, sc, dp, ds, S, D, H, h, S, S, th);
    double t2 = now_s();
    g_split[0] = t1 - t0;
    g_split[1] = t2 - t1;
    /* gtx: C = A^T B over the BS rows (k, n, then i) */
    const float* gtx_a[4] = {x, x, x, oh};
    const float* gtx_b[4] = {dQ2, dK2, dV2, dout};
    float* gtx_c[4] = {dWq, dWk, dWv, dWo};
    for (int q = 0; q < 4; q++) {
        if (!gtx_c[q]) continue;
        double ta = now_s();
        for (int64_t k = 0; k < D * D; k++) gtx_c[q][k] = 0.f;
        for (int64_t k = 0; k < D; k++)
            for (int64_t m = 0; m < D; m++) {
                float a = 0.f;
                for (int64_t i = 0; i < BS; i++) a += gtx_a[q][(size_t)i * D + k] * gtx_b[q][(size_t)i * D + m];
                gtx_c[q][(size_t)k * D + m] = a;
            }
        g_split[2 + q] = now_s() - ta;
    }
    if (dX) {
        double ta = now_s();
        /* gmt: C = A B^T (i, j, then k), three times, then the sum */
        float* g3 = (float*)malloc(3 * n * sizeof(float));
        const float* ga[3] = {dQ2, dK2, dV2};
        const float* gw[3] = {Wq, Wk, Wv};
        for (int q = 0; q < 3; q++)
            for (int64_t i = 0; i < BS; i++)
                for (int64_t j = 0; j < D; j++) {
                    float a = 0.f;
                    for (int64_t k = 0; k < D; k++) a += ga[q][(size_t)i * D + k] * gw[q][(size_t)j * D + k];
                    g3[q * n + (size_t)i * D + j] = a;
                }
        for (size_t i = 0; i < n; i++) dX[i] = g3[i] + g3[n + i] + g3[2 * n + i];
        free(g3);
        g_split[6] = now_s() - ta;
    }
    free(Qq); free(Kk); free(Vv); free(dQ2); free(dK2); free(dV2); free(dPre); free(oh);
    free(sc); free(dp); free(ds);
}

/* ------------------------------------------------------------------------ */
/* top-1 MoE forward, ns_moe_fwd codegen.cpp:1915-1945 (one token at a time) */
/* ------------------------------------------------------------------------ */

EXPORT void or_moe_fwd(const float* x, const float* Wg, const float* We1, const float* We2, const uint8_t* active,
                       float* out, int64_t* best_out, float* prob_out, int64_t M, int64_t D, int64_t H, int64_t E) {
    float* lg = (float*)malloc((size_t)E * sizeof(float));
    float* h = (float*)malloc((size_t)H * sizeof(float));
    for (int64_t i = 0; i < M; i++) {
        float mx = -1.0e30f, sum = 0.f;
        for (int64_t e = 0; e < E; e++) {
            float a = 0.f;
            for (int64_t k = 0; k < D; k++) a += x[(size_t)i * D + k] * Wg[(size_t)k * E + e];
            lg[e] = a;
            if ((!active || active[e]) && a > mx) mx = a;
        }
        for (int64_t e = 0; e < E; e++)
            if (!active || active[e]) { lg[e] = expf(lg[e] - mx); sum += lg[e]; }
        int64_t best = -1;
        for (int64_t e = 0; e < E; e++)
            if ((!active || active[e]) && (best < 0 || lg[e] > lg[best])) best = e;
        const float p = (sum > 0.f && best >= 0) ? lg[best] / sum : 0.f;
        if (best_out) best_out[i] = best;
        if (prob_out) prob_out[i] = p;
        if (best < 0) {  /* no live expert: the reference reads expert -1; zeros here */
            memset(out + (size_t)i * D, 0, (size_t)D * sizeof(float));
            continue;
        }
        for (int64_t a = 0; a < H; a++) {
            float acc = 0.f;
            for (int64_t k = 0; k < D; k++) acc += x[(size_t)i * D + k] * We1[(size_t)best * D * H + (size_t)k * H + a];
            h[a] = 0.5f * acc * (1.f + erff(acc * 0.7071067811865476f));
        }
        for (int64_t j = 0; j < D; j++) {
            float a = 0.f;
            for (int64_t b = 0; b < H; b++) a += h[b] * We2[(size_t)best * H * D + (size_t)b * D + j];
            out[(size_t)i * D + j] = p * a;
        }
    }
    free(lg);
    free(h);
}

/* ------------------------------------------------------------------------ */
/* optimizer, codegen.cpp:3088-3124                                          */
/* ------------------------------------------------------------------------ */

/* ns_orthonom codegen.cpp:1617-1633: left-looking MGS over the columns of
 * G[M,N] (M >= N, column k-th element at G[k*N + j]) or its rows (M < N). */
EXPORT void or_orthonom(float* G, int64_t M, int64_t N) {
    const int tr = M < N;
    const size_t R = tr ? (size_t)N : (size_t)M;
    const size_t C = tr ? (size_t)M : (size_t)N;
#define AT(k, j) (*(tr ? &G[(j) * R + (k)] : &G[(k) * (size_t)N + (j)]))
    for (size_t j = 0; j < C; j++) {
        for (size_t i = 0; i < j; i++) {
            float dot = 0.f;
            for (size_t k = 0; k < R; k++) dot += AT(k, i) * AT(k, j);
            for (size_t k = 0; k < R; k++) AT(k, j) -= dot * AT(k, i);
        }
        float nrm = 0.f;
        for (size_t k = 0; k < R; k++) nrm += AT(k, j) * AT(k, j);
        nrm = sqrtf(nrm) + 1e-30f;
        for (size_t k = 0; k < R; k++) AT(k, j) /= nrm;
    }
#undef AT
}

/* Muon with a momentum buffer that is zero at every apply (codegen.cpp:
 * 3099-3107); g becomes the momentum, then its orthonormalisation. */
EXPORT void or_muon_step(float* w, float* g, int64_t r, int64_t c, float lr) {
    const size_t n = (size_t)r * c;
    for (size_t i = 0; i < n; i++) g[i] = 0.95f * 0.f + g[i];
    or_orthonom(g, r, c);
    const float rank = sqrtf((float)(r < c ? r : c));
    const float le = lr * rank;
    for (size_t i = 0; i < n; i++) w[i] -= le * g[i] + (0.01f * lr) * w[i];
}

/* codegen.cpp:3108-3119; t is the step count after its increment */
EXPORT void or_adamw_step(float* w, const float* g, float* m, float* v, size_t n, int64_t t, float lr) {
    const float b1t = 1.f - powf(0.9f, (float)t), b2t = 1.f - powf(0.999f, (float)t);
    for (size_t i = 0; i < n; i++) {
        const float gg = g[i];
        m[i] = 0.9f * m[i] + 0.1f * gg;
        v[i] = 0.999f * v[i] + 0.001f * gg * gg;
        const float mh = m[i] / b1t, vh = v[i] / b2t;
        w[i] -= (lr * mh / (sqrtf(vh) + 1e-8f)) + (0.01f * lr) * w[i];
    }
}

/* codegen.cpp:3097 */
EXPORT int or_use_muon(int64_t r, int64_t c) { return r > 1 && c > 1 && (r < c ? r : c) >= 8; }
