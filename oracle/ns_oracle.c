/*
 * ns_oracle.c -- CPU restatement of the NeuralScript CPU code generator's
 * runtime kernels (the `nsc --cpp --runtime` output).
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (libnship) links, loads or
 * calls this file; only tests/, __graft_entry__.smoke() and bench.py's CPU
 * baseline leg use it, and only as the checker.
 *
 * Every function reproduces, element by element, the arithmetic of the kernel
 * text the reference emits (cited per function, all in
 * /root/reference/src/codegen/codegen.cpp): the same fp32 operations in the
 * same order for every output element -- single accumulator, ascending
 * reduction index, multiply then add (built with -ffp-contract=off so no FMA
 * is formed), the same libm calls.  Work is reordered only ACROSS independent
 * output elements (loop interchange, row blocking, threads), which leaves
 * every result bit-identical to the emitted scalar code.  The reference's own
 * emitted code, compiled from its sources into oracle/_ref/, pins this
 * bitwise (tests/test_oracle.py).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define EXPORT __attribute__((visibility("default")))

/* ---------------------------------------------------------------------- */
/* activations: ns_act2 codegen.cpp:1244-1255, ns_act_deriv :1305-1315     */
/* ---------------------------------------------------------------------- */
static inline float act_fwd(float x, int code) {
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

static inline float act_deriv(float x, int code) {
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
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < n; i++) out[i] = act_fwd(in[i], code);
}

/* ns_act_grad codegen.cpp:1340-1343 */
EXPORT void or_act_grad(const float* din, const float* pre, float* dout, size_t n, int code) {
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < n; i++) dout[i] = din[i] * act_deriv(pre[i], code);
}

/* ---------------------------------------------------------------------- */
/* dense products                                                          */
/* ---------------------------------------------------------------------- */

/* C[M,N] = A[M,K] B[K,N]; ns_matmul codegen.cpp:1257-1265.  Per element the
 * sum runs k = 0..K-1 into one float starting at 0.f; the i-k-j order below
 * performs exactly that sequence for every (i,j).  `act` applies the fused
 * epilogue the forward body runs afterwards (codegen.cpp:2057-2075). */
EXPORT void or_matmul(const float* A, const float* B, float* C,
                      int64_t M, int64_t K, int64_t N, int act) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < M; i++) {
        float* c = C + (size_t)i * N;
        for (int64_t j = 0; j < N; j++) c[j] = 0.f;
        const float* a = A + (size_t)i * K;
        for (int64_t k = 0; k < K; k++) {
            const float av = a[k];
            const float* b = B + (size_t)k * N;
            for (int64_t j = 0; j < N; j++) c[j] += av * b[j];
        }
        if (act)
            for (int64_t j = 0; j < N; j++) c[j] = act_fwd(c[j], act);
    }
}

/* The same product for a subset of rows of A (rows[r] -> C row r). */
EXPORT void or_matmul_rows(const float* A, const int64_t* rows, int64_t R, const float* B,
                           float* C, int64_t K, int64_t N, int act) {
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < R; r++) {
        float* c = C + (size_t)r * N;
        for (int64_t j = 0; j < N; j++) c[j] = 0.f;
        const float* a = A + (size_t)rows[r] * K;
        for (int64_t k = 0; k < K; k++) {
            const float av = a[k];
            const float* b = B + (size_t)k * N;
            for (int64_t j = 0; j < N; j++) c[j] += av * b[j];
        }
        if (act)
            for (int64_t j = 0; j < N; j++) c[j] = act_fwd(c[j], act);
    }
}

static float* transpose_copy(const float* B, int64_t R, int64_t C) {
    float* t = (float*)malloc((size_t)R * C * sizeof(float));
#pragma omp parallel for schedule(static)
    for (int64_t c = 0; c < C; c++)
        for (int64_t r = 0; r < R; r++) t[(size_t)c * R + r] = B[(size_t)r * C + c];
    return t;
}

/* dA[M,K] = dC[M,N] B[K,N]^T, sum over j ascending; ns_matmul_grad_a
 * codegen.cpp:1318-1326.  B is transposed once so the j-outer / k-inner
 * accumulation reads contiguous memory. */
EXPORT void or_matmul_grad_a(const float* dC, const float* B, float* dA,
                             int64_t M, int64_t K, int64_t N) {
    float* Bt = transpose_copy(B, K, N); /* [N,K] */
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < M; i++) {
        float* a = dA + (size_t)i * K;
        for (int64_t k = 0; k < K; k++) a[k] = 0.f;
        const float* d = dC + (size_t)i * N;
        for (int64_t j = 0; j < N; j++) {
            const float dv = d[j];
            const float* b = Bt + (size_t)j * K;
            for (int64_t k = 0; k < K; k++) a[k] += dv * b[k];
        }
    }
    free(Bt);
}

/* dB[K,N] = A[M,K]^T dC[M,N], sum over i ascending; ns_matmul_grad_w
 * codegen.cpp:1329-1337 (also the attention backward's `gtx`, :1815-1822). */
EXPORT void or_matmul_grad_w(const float* A, const float* dC, float* dB,
                             int64_t M, int64_t K, int64_t N) {
#pragma omp parallel for schedule(static)
    for (int64_t k = 0; k < K; k++) {
        float* b = dB + (size_t)k * N;
        for (int64_t j = 0; j < N; j++) b[j] = 0.f;
        for (int64_t i = 0; i < M; i++) {
            const float av = A[(size_t)i * K + k];
            const float* d = dC + (size_t)i * N;
            for (int64_t j = 0; j < N; j++) b[j] += av * d[j];
        }
    }
}

/* ---------------------------------------------------------------------- */
/* row-wise normalisation                                                  */
/* ---------------------------------------------------------------------- */

/* out = LayerNorm(in) over rows of `last`; ns_layernorm codegen.cpp:1280-1291
 * (the forward copies the input then normalises in place, :2020-2025). */
EXPORT void or_layernorm(const float* in, float* out, size_t numel, int64_t last) {
    const int64_t rows = (int64_t)numel / last;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; r++) {
        const float* x = in + (size_t)r * last;
        float* y = out + (size_t)r * last;
        float mean = 0.f, var = 0.f;
        for (int64_t j = 0; j < last; j++) mean += x[j];
        mean /= last;
        for (int64_t j = 0; j < last; j++) { float d = x[j] - mean; var += d * d; }
        var /= last;
        const float inv = 1.f / sqrtf(var + 1e-5f);
        for (int64_t j = 0; j < last; j++) y[j] = (x[j] - mean) * inv;
    }
}

/* ns_softmax codegen.cpp:1293-1303: out = copy of in, then every full row
 * of `last` values: max (std::max order), expf(x - max) summed in order,
 * then divided by the sum. */
EXPORT void or_softmax(const float* in, float* out, size_t numel, int64_t last) {
    if (out != in) memcpy(out, in, numel * sizeof(float));
    const int64_t rows = (int64_t)numel / last;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; r++) {
        float* m = out + (size_t)r * last;
        float mx = m[0];
        for (int64_t j = 1; j < last; j++) mx = (mx < m[j]) ? m[j] : mx;
        float s = 0.f;
        for (int64_t j = 0; j < last; j++) { m[j] = expf(m[j] - mx); s += m[j]; }
        for (int64_t j = 0; j < last; j++) m[j] /= s;
    }
}

/* ns_layernorm_grad codegen.cpp:1346-1371 */
EXPORT void or_layernorm_grad(const float* dout, const float* x, float* dx,
                              size_t numel, int64_t last) {
    const int64_t rows = (int64_t)numel / last;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; r++) {
        const float* xr = x + (size_t)r * last;
        const float* dr = dout + (size_t)r * last;
        float mean_x = 0.f, mean_d = 0.f;
        for (int64_t j = 0; j < last; j++) { mean_x += xr[j]; mean_d += dr[j]; }
        mean_x /= last;
        mean_d /= last;
        float var_x = 0.f, gamma = 0.f;
        for (int64_t j = 0; j < last; j++) {
            float xj = xr[j] - mean_x;
            var_x += xj * xj;
            gamma += xj * dr[j];
        }
        var_x /= last;
        gamma /= last;
        const float inv = 1.f / sqrtf(var_x + 1e-5f);
        for (int64_t j = 0; j < last; j++) {
            float xj = xr[j] - mean_x;
            dx[(size_t)r * last + j] = (dr[j] - mean_d - xj * gamma) * inv;
        }
    }
}

/* ---------------------------------------------------------------------- */
/* embedding                                                               */
/* ---------------------------------------------------------------------- */

/* out[i,:] = W[(int64)idx[i], :], out-of-range -> row 0; ns_embedding
 * codegen.cpp:1711-1718.  The float->int64 conversion is C truncation; the
 * test below is the same predicate written so it is defined for NaN and
 * magnitudes beyond int64 (x86 converts those to INT64_MIN, i.e. out of
 * range). */
static inline int64_t emb_row(float f, int64_t V) {
    if (!(f > -1.0f) || !(f < (float)V)) return -1;
    int64_t k = (int64_t)f;
    return (k < 0 || k >= V) ? -1 : k;
}

EXPORT void or_embedding(const float* W, const float* idx, float* out,
                         int64_t n, int64_t V, int64_t D) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; i++) {
        int64_t k = emb_row(idx[i], V);
        if (k < 0) k = 0;
        memcpy(out + (size_t)i * D, W + (size_t)k * D, (size_t)D * sizeof(float));
    }
}

/* Resolved row per index (-1 = out of range), for bit-exact index checks. */
EXPORT void or_embedding_rows(const float* idx, int64_t* rows, int64_t n, int64_t V) {
    for (int64_t i = 0; i < n; i++) rows[i] = emb_row(idx[i], V);
}

/* dW[V,D] = scatter-add of dout rows in token order, skipping out-of-range
 * indices; ns_embedding_grad_w codegen.cpp:1374-1383.  Columns are
 * independent, so threads split columns and keep token order per element. */
EXPORT void or_embedding_grad_w(const float* dout, const float* idx, float* dW,
                                size_t M, int64_t D, int64_t V) {
    int64_t* rows = (int64_t*)malloc((M ? M : 1) * sizeof(int64_t));
    for (size_t i = 0; i < M; i++) rows[i] = emb_row(idx[i], V);
    memset(dW, 0, (size_t)V * D * sizeof(float));
    const int64_t CB = 64;
#pragma omp parallel for schedule(static)
    for (int64_t c0 = 0; c0 < D; c0 += CB) {
        const int64_t c1 = c0 + CB < D ? c0 + CB : D;
        for (size_t i = 0; i < M; i++) {
            const int64_t r = rows[i];
            if (r < 0) continue;
            float* w = dW + (size_t)r * D;
            const float* d = dout + i * D;
            for (int64_t j = c0; j < c1; j++) w[j] += d[j];
        }
    }
    free(rows);
}

/* ---------------------------------------------------------------------- */
/* softmax cross-entropy                                                   */
/* ---------------------------------------------------------------------- */

static inline float row_max(const float* p, int64_t C) {
    float mx = p[0];
    for (int64_t j = 1; j < C; j++) mx = (mx < p[j]) ? p[j] : mx; /* std::max */
    return mx;
}

/* mean over rows of -sum_{y>0} log softmax; ns_cross_entropy
 * codegen.cpp:1598-1613.  The single float accumulator runs over rows then
 * columns in order, so the per-row (max, sum) pass is threaded and the
 * accumulation pass is sequential. */
EXPORT float or_cross_entropy(const float* preds, const float* labels, size_t numel, int64_t C) {
    const int64_t rows = (int64_t)numel / C;
    float* mx = (float*)malloc((rows ? rows : 1) * sizeof(float));
    float* sm = (float*)malloc((rows ? rows : 1) * sizeof(float));
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; r++) {
        const float* p = preds + (size_t)r * C;
        const float m = row_max(p, C);
        float s = 0.f;
        for (int64_t j = 0; j < C; j++) s += expf(p[j] - m);
        mx[r] = m;
        sm[r] = s;
    }
    float loss = 0.f;
    for (int64_t r = 0; r < rows; r++) {
        const float* p = preds + (size_t)r * C;
        const float* y = labels + (size_t)r * C;
        for (int64_t j = 0; j < C; j++) {
            if (y[j] > 0.f) {
                float pj = expf(p[j] - mx[r]) / sm[r];
                loss -= logf(pj);
            }
        }
    }
    free(mx);
    free(sm);
    return loss / (float)rows;
}

/* d = (softmax(preds) - labels) / rows; ns_loss_grad codegen.cpp:1582-1595 */
EXPORT void or_loss_grad(const float* preds, const float* labels, float* d, size_t numel, int64_t C) {
    const int64_t rows = (int64_t)numel / C;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; r++) {
        const float* p = preds + (size_t)r * C;
        const float m = row_max(p, C);
        float s = 0.f;
        for (int64_t j = 0; j < C; j++) s += expf(p[j] - m);
        for (int64_t j = 0; j < C; j++) {
            float pj = expf(p[j] - m) / s;
            d[(size_t)r * C + j] = (pj - labels[(size_t)r * C + j]) / (float)rows;
        }
    }
}

/* ---------------------------------------------------------------------- */
/* multi-head self-attention over ONE sequence of BS tokens (S = BS)       */
/* ---------------------------------------------------------------------- */

/* Scores of query row i against all S keys for head h, softmaxed in place:
 * the per-row part of ns_attention_fwd codegen.cpp:1747-1763 (identical in
 * the backward's recomputation, :1846-1857). */
static void attn_prob_row(const float* Q, const float* K, float* p, int64_t i, int64_t S,
                          int64_t D, int64_t h, int64_t Dk, float scale) {
    const float* q = Q + (size_t)i * D + h * Dk;
    for (int64_t j = 0; j < S; j++) {
        const float* k = K + (size_t)j * D + h * Dk;
        float a = 0.f;
        for (int64_t d = 0; d < Dk; d++) a += q[d] * k[d];
        p[j] = a * scale;
    }
    const float mx = row_max(p, S);
    float s = 0.f;
    for (int64_t j = 0; j < S; j++) { p[j] = expf(p[j] - mx); s += p[j]; }
    for (int64_t j = 0; j < S; j++) p[j] /= s;
}

/* Per-head context rows ctx[i, h*Dk+d] = sum_j P[i,j] V[j, h*Dk+d] (j
 * ascending) for the query rows listed in `qrows` (all rows when NULL). */
static void attn_context(const float* Q, const float* K, const float* V, float* ctx,
                         const int64_t* qrows, int64_t nq, int64_t S, int64_t D, int64_t H) {
    const int64_t Dk = D / H;
    const float scale = 1.0f / sqrtf((float)Dk);
#pragma omp parallel
    {
        float* p = (float*)malloc((size_t)S * sizeof(float));
        float* acc = (float*)malloc((size_t)Dk * sizeof(float));
#pragma omp for schedule(static) collapse(2)
        for (int64_t h = 0; h < H; h++)
            for (int64_t r = 0; r < nq; r++) {
                const int64_t i = qrows ? qrows[r] : r;
                attn_prob_row(Q, K, p, i, S, D, h, Dk, scale);
                for (int64_t d = 0; d < Dk; d++) acc[d] = 0.f;
                for (int64_t j = 0; j < S; j++) {
                    const float pj = p[j];
                    const float* v = V + (size_t)j * D + h * Dk;
                    for (int64_t d = 0; d < Dk; d++) acc[d] += pj * v[d];
                }
                memcpy(ctx + (size_t)r * D + h * Dk, acc, (size_t)Dk * sizeof(float));
            }
        free(p);
        free(acc);
    }
}

/* out = MHA(x) with S = BS (one sequence); ns_attention_fwd
 * codegen.cpp:1724-1777, called with S = BS at :2224-2235. */
EXPORT void or_attention_fwd(const float* x, const float* Wq, const float* Wk, const float* Wv,
                             const float* Wo, float* out, int64_t BS, int64_t D, int64_t H) {
    const size_t n = (size_t)BS * D;
    float* Q = (float*)malloc(n * sizeof(float));
    float* K = (float*)malloc(n * sizeof(float));
    float* V = (float*)malloc(n * sizeof(float));
    float* ctx = (float*)malloc(n * sizeof(float));
    or_matmul(x, Wq, Q, BS, D, D, 0);
    or_matmul(x, Wk, K, BS, D, D, 0);
    or_matmul(x, Wv, V, BS, D, D, 0);
    attn_context(Q, K, V, ctx, NULL, BS, BS, D, H);
    or_matmul(ctx, Wo, out, BS, D, D, 0);
    free(Q); free(K); free(V); free(ctx);
}

/* The same forward for a subset of query rows (rows are independent given
 * the full K and V), for checks at full sequence length. */
EXPORT void or_attention_fwd_rows(const float* x, const float* Wq, const float* Wk,
                                  const float* Wv, const float* Wo, const int64_t* qrows,
                                  int64_t nq, float* out, int64_t BS, int64_t D, int64_t H) {
    const size_t n = (size_t)BS * D;
    float* Q = (float*)malloc((size_t)nq * D * sizeof(float));
    float* K = (float*)malloc(n * sizeof(float));
    float* V = (float*)malloc(n * sizeof(float));
    float* ctx = (float*)malloc((size_t)nq * D * sizeof(float));
    or_matmul_rows(x, qrows, nq, Wq, Q, D, D, 0);
    or_matmul(x, Wk, K, BS, D, D, 0);
    or_matmul(x, Wv, V, BS, D, D, 0);
    /* Q holds only the selected rows: index it densely. */
    int64_t* dense = (int64_t*)malloc((size_t)(nq ? nq : 1) * sizeof(int64_t));
    for (int64_t r = 0; r < nq; r++) dense[r] = r;
    /* attn_context indexes Q by row id; pass the dense Q with dense ids and
     * the full K/V (row ids of K/V are the sequence positions). */
    {
        const int64_t Dk = D / H;
        const float scale = 1.0f / sqrtf((float)Dk);
#pragma omp parallel
        {
            float* p = (float*)malloc((size_t)BS * sizeof(float));
            float* acc = (float*)malloc((size_t)Dk * sizeof(float));
#pragma omp for schedule(static) collapse(2)
            for (int64_t h = 0; h < H; h++)
                for (int64_t r = 0; r < nq; r++) {
                    const float* q = Q + (size_t)r * D + h * Dk;
                    for (int64_t j = 0; j < BS; j++) {
                        const float* k = K + (size_t)j * D + h * Dk;
                        float a = 0.f;
                        for (int64_t d = 0; d < Dk; d++) a += q[d] * k[d];
                        p[j] = a * scale;
                    }
                    const float mx = row_max(p, BS);
                    float s = 0.f;
                    for (int64_t j = 0; j < BS; j++) { p[j] = expf(p[j] - mx); s += p[j]; }
                    for (int64_t j = 0; j < BS; j++) p[j] /= s;
                    for (int64_t d = 0; d < Dk; d++) acc[d] = 0.f;
                    for (int64_t j = 0; j < BS; j++) {
                        const float pj = p[j];
                        const float* v = V + (size_t)j * D + h * Dk;
                        for (int64_t d = 0; d < Dk; d++) acc[d] += pj * v[d];
                    }
                    memcpy(ctx + (size_t)r * D + h * Dk, acc, (size_t)Dk * sizeof(float));
                }
            free(p);
            free(acc);
        }
    }
    or_matmul(ctx, Wo, out, nq, D, D, 0);
    free(dense);
    free(Q); free(K); free(V); free(ctx);
}

/* Attention backward for S = BS; ns_attention_bwd codegen.cpp:1785-1907
 * (emitted once per output at :3017-3051; its recomputation is deterministic,
 * so producing all five outputs from one recomputation gives the same bits).
 * Any output pointer may be NULL.  Memory: two S*S float planes per head. */
EXPORT void or_attention_bwd(const float* dout, const float* x, const float* Wq, const float* Wk,
                             const float* Wv, const float* Wo, float* dX, float* dWq, float* dWk,
                             float* dWv, float* dWo, int64_t BS, int64_t D, int64_t H) {
    if (D <= 0 || H <= 0 || BS <= 0) return;
    const int64_t S = BS, Dk = D / H;
    const float scale = 1.0f / sqrtf((float)Dk);
    const size_t n = (size_t)BS * D;
    float* Q = (float*)malloc(n * sizeof(float));
    float* K = (float*)malloc(n * sizeof(float));
    float* V = (float*)malloc(n * sizeof(float));
    float* dPre = (float*)malloc(n * sizeof(float));
    float* oh = (float*)calloc(n, sizeof(float));
    float* dQ = (float*)calloc(n, sizeof(float));
    float* dK = (float*)calloc(n, sizeof(float));
    float* dV = (float*)calloc(n, sizeof(float));
    float* P = (float*)malloc((size_t)S * S * sizeof(float));
    float* dS = (float*)malloc((size_t)S * S * sizeof(float));
    or_matmul(x, Wq, Q, BS, D, D, 0);
    or_matmul(x, Wk, K, BS, D, D, 0);
    or_matmul(x, Wv, V, BS, D, D, 0);
    /* dPre[i,k] = sum_n dout[i,n] Wo[k,n]  (n ascending) */
    or_matmul_grad_a(dout, Wo, dPre, BS, D, D);
    for (int64_t h = 0; h < H; h++) {
        /* rows: P, oh, dp -> dS, dQ */
#pragma omp parallel
        {
            float* dp = (float*)malloc((size_t)S * sizeof(float));
            float* acc = (float*)malloc((size_t)Dk * sizeof(float));
#pragma omp for schedule(static)
            for (int64_t i = 0; i < S; i++) {
                float* p = P + (size_t)i * S;
                attn_prob_row(Q, K, p, i, S, D, h, Dk, scale);
                for (int64_t d = 0; d < Dk; d++) acc[d] = 0.f;
                for (int64_t j = 0; j < S; j++) {
                    const float* v = V + (size_t)j * D + h * Dk;
                    for (int64_t d = 0; d < Dk; d++) acc[d] += p[j] * v[d];
                }
                for (int64_t d = 0; d < Dk; d++) oh[(size_t)i * D + h * Dk + d] = acc[d];
                const float* g = dPre + (size_t)i * D + h * Dk;
                for (int64_t j = 0; j < S; j++) {
                    const float* v = V + (size_t)j * D + h * Dk;
                    float a = 0.f;
                    for (int64_t d = 0; d < Dk; d++) a += v[d] * g[d];
                    dp[j] = a;
                }
                float dot = 0.f;
                for (int64_t j = 0; j < S; j++) dot += p[j] * dp[j];
                float* ds = dS + (size_t)i * S;
                for (int64_t j = 0; j < S; j++) ds[j] = p[j] * (dp[j] - dot);
                for (int64_t d = 0; d < Dk; d++) acc[d] = 0.f;
                for (int64_t j = 0; j < S; j++) {
                    const float* k = K + (size_t)j * D + h * Dk;
                    for (int64_t d = 0; d < Dk; d++) acc[d] += ds[j] * k[d];
                }
                for (int64_t d = 0; d < Dk; d++) dQ[(size_t)i * D + h * Dk + d] += acc[d] * scale;
            }
            free(dp);
            free(acc);
        }
        /* columns: dV[j] = sum_i P[i,j] dPre[i], dK[j] = sum_i dS[i,j] Q[i] (i ascending) */
        const int64_t JB = 16;
#pragma omp parallel
        {
            float* av = (float*)malloc((size_t)JB * Dk * sizeof(float));
            float* ak = (float*)malloc((size_t)JB * Dk * sizeof(float));
#pragma omp for schedule(static)
            for (int64_t j0 = 0; j0 < S; j0 += JB) {
                const int64_t jn = (j0 + JB < S ? j0 + JB : S) - j0;
                for (int64_t t = 0; t < jn * Dk; t++) { av[t] = 0.f; ak[t] = 0.f; }
                for (int64_t i = 0; i < S; i++) {
                    const float* g = dPre + (size_t)i * D + h * Dk;
                    const float* q = Q + (size_t)i * D + h * Dk;
                    for (int64_t jj = 0; jj < jn; jj++) {
                        const float pv = P[(size_t)i * S + j0 + jj];
                        const float sv = dS[(size_t)i * S + j0 + jj];
                        for (int64_t d = 0; d < Dk; d++) {
                            av[jj * Dk + d] += pv * g[d];
                            ak[jj * Dk + d] += sv * q[d];
                        }
                    }
                }
                for (int64_t jj = 0; jj < jn; jj++)
                    for (int64_t d = 0; d < Dk; d++) {
                        dV[(size_t)(j0 + jj) * D + h * Dk + d] += av[jj * Dk + d];
                        dK[(size_t)(j0 + jj) * D + h * Dk + d] += ak[jj * Dk + d] * scale;
                    }
            }
            free(av);
            free(ak);
        }
    }
    if (dWq) or_matmul_grad_w(x, dQ, dWq, BS, D, D);
    if (dWk) or_matmul_grad_w(x, dK, dWk, BS, D, D);
    if (dWv) or_matmul_grad_w(x, dV, dWv, BS, D, D);
    if (dWo) or_matmul_grad_w(oh, dout, dWo, BS, D, D);
    if (dX) {
        float* gq = (float*)malloc(n * sizeof(float));
        float* gk = (float*)malloc(n * sizeof(float));
        float* gv = (float*)malloc(n * sizeof(float));
        or_matmul_grad_a(dQ, Wq, gq, BS, D, D);
        or_matmul_grad_a(dK, Wk, gk, BS, D, D);
        or_matmul_grad_a(dV, Wv, gv, BS, D, D);
        for (size_t t = 0; t < n; t++) dX[t] = gq[t] + gk[t] + gv[t];
        free(gq); free(gk); free(gv);
    }
    free(Q); free(K); free(V); free(dPre); free(oh); free(dQ); free(dK); free(dV);
    free(P); free(dS);
}

/* ---------------------------------------------------------------------- */
/* top-1 mixture of experts                                                */
/* ---------------------------------------------------------------------- */

static inline int is_live(const uint8_t* active, int64_t e) { return !active || active[e] != 0; }

/* Router for one token: logits (sequential k), max over live, exp, sum,
 * first strict maximum over live experts.  Writes exp'd values to lg and
 * the probabilities to p (0 for dead experts); returns best (-1 if none
 * live).  ns_moe_fwd codegen.cpp:1921-1936 / ns_moe_grad_* :1405-1419. */
static int64_t moe_route(const float* x, const float* Wg, const uint8_t* active, float* lg,
                         float* p, float* sum_out, int64_t D, int64_t E) {
    float mx = -1.0e30f, sum = 0.f;
    for (int64_t e = 0; e < E; e++) {
        float a = 0.f;
        for (int64_t k = 0; k < D; k++) a += x[k] * Wg[k * E + e];
        lg[e] = a;
        if (is_live(active, e) && a > mx) mx = a;
    }
    int64_t best = -1;
    for (int64_t e = 0; e < E; e++) {
        if (!is_live(active, e)) continue;
        lg[e] = expf(lg[e] - mx);
        sum += lg[e];
    }
    for (int64_t e = 0; e < E; e++)
        if (is_live(active, e) && (best < 0 || lg[e] > lg[best])) best = e;
    if (p)
        for (int64_t e = 0; e < E; e++) p[e] = (is_live(active, e) && sum > 0.f) ? lg[e] / sum : 0.f;
    *sum_out = sum;
    return best;
}

/* Raw gate logits (before exp) of every token, for tie reports. */
EXPORT void or_moe_gate_logits(const float* x, const float* Wg, float* logits,
                               int64_t M, int64_t D, int64_t E) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < M; i++)
        for (int64_t e = 0; e < E; e++) {
            float a = 0.f;
            for (int64_t k = 0; k < D; k++) a += x[(size_t)i * D + k] * Wg[k * E + e];
            logits[(size_t)i * E + e] = a;
        }
}

/* Routing only (best expert, its probability, raw logits) of every token:
 * the router part of ns_moe_fwd, codegen.cpp:1921-1936. */
EXPORT void or_moe_route(const float* x, const float* Wg, const uint8_t* active, int64_t* best_out,
                         float* prob_out, float* logits_out, int64_t M, int64_t D, int64_t E) {
#pragma omp parallel
    {
        float* lg = (float*)malloc((size_t)E * sizeof(float));
#pragma omp for schedule(static)
        for (int64_t i = 0; i < M; i++) {
            const float* xi = x + (size_t)i * D;
            if (logits_out)
                for (int64_t e = 0; e < E; e++) {
                    float a = 0.f;
                    for (int64_t k = 0; k < D; k++) a += xi[k] * Wg[k * E + e];
                    logits_out[(size_t)i * E + e] = a;
                }
            float sum;
            const int64_t b = moe_route(xi, Wg, active, lg, NULL, &sum, D, E);
            best_out[i] = b;
            prob_out[i] = (b >= 0 && sum > 0.f) ? lg[b] / sum : 0.f;
        }
        free(lg);
    }
}

/* out = p_best * GELU(x We1[best]) We2[best]; ns_moe_fwd codegen.cpp:1915-1945.
 * best_out (optional) receives the chosen expert per token.  A token with
 * no live expert gets zeros (the reference indexes expert -1 there). */
EXPORT void or_moe_fwd(const float* x, const float* Wg, const float* We1, const float* We2,
                       const uint8_t* active, float* out, int64_t* best_out, float* prob_out,
                       int64_t M, int64_t D, int64_t H, int64_t E) {
#pragma omp parallel
    {
        float* lg = (float*)malloc((size_t)E * sizeof(float));
        float* h = (float*)malloc((size_t)H * sizeof(float));
        float* acc = (float*)malloc((size_t)D * sizeof(float));
#pragma omp for schedule(static)
        for (int64_t i = 0; i < M; i++) {
            const float* xi = x + (size_t)i * D;
            float sum;
            const int64_t best = moe_route(xi, Wg, active, lg, NULL, &sum, D, E);
            if (best_out) best_out[i] = best;
            float* o = out + (size_t)i * D;
            if (best < 0) {
                if (prob_out) prob_out[i] = 0.f;
                for (int64_t j = 0; j < D; j++) o[j] = 0.f;
                continue;
            }
            const float p = (sum > 0.f) ? lg[best] / sum : 0.f;
            if (prob_out) prob_out[i] = p;
            const float* w1 = We1 + (size_t)best * D * H;
            for (int64_t a = 0; a < H; a++) h[a] = 0.f;
            for (int64_t k = 0; k < D; k++) {
                const float xv = xi[k];
                const float* w = w1 + (size_t)k * H;
                for (int64_t a = 0; a < H; a++) h[a] += xv * w[a];
            }
            for (int64_t a = 0; a < H; a++)
                h[a] = 0.5f * h[a] * (1.f + erff(h[a] * 0.7071067811865476f));
            const float* w2 = We2 + (size_t)best * H * D;
            for (int64_t j = 0; j < D; j++) acc[j] = 0.f;
            for (int64_t b = 0; b < H; b++) {
                const float hv = h[b];
                const float* w = w2 + (size_t)b * D;
                for (int64_t j = 0; j < D; j++) acc[j] += hv * w[j];
            }
            for (int64_t j = 0; j < D; j++) o[j] = p * acc[j];
        }
        free(lg); free(h); free(acc);
    }
}

/* MoE backward: all four outputs of ns_moe_grad_x/_wg/_we1/_we2
 * (codegen.cpp:1388-1579) from one routing recomputation (each function
 * recomputes the same routing deterministically).  dx is zeroed then
 * accumulated as the train body does (:2963-2966).  Weight grads accumulate
 * over tokens in ascending order, so the per-token pass is sequential over
 * tokens for them; the per-token quantities are computed in parallel first.
 * Any output may be NULL. */
EXPORT void or_moe_bwd(const float* dout, const float* x, const float* Wg, const float* We1,
                       const float* We2, const uint8_t* active, float* dx, float* dWg,
                       float* dWe1, float* dWe2, int64_t M, int64_t D, int64_t H, int64_t E) {
    /* per-token state: best, p[E], pre-activation u[H], dpre2[H] */
    int64_t* best = (int64_t*)malloc((size_t)(M ? M : 1) * sizeof(int64_t));
    float* P = (float*)malloc((size_t)M * E * sizeof(float));
    float* U = (float*)malloc((size_t)M * H * sizeof(float));
    float* DP = (float*)malloc((size_t)M * H * sizeof(float));
#pragma omp parallel
    {
        float* lg = (float*)malloc((size_t)E * sizeof(float));
#pragma omp for schedule(static)
        for (int64_t i = 0; i < M; i++) {
            const float* xi = x + (size_t)i * D;
            float sum;
            float* p = P + (size_t)i * E;
            const int64_t b = moe_route(xi, Wg, active, lg, p, &sum, D, E);
            best[i] = b;
            float* u = U + (size_t)i * H;
            float* dp = DP + (size_t)i * H;
            if (b < 0) {
                for (int64_t a = 0; a < H; a++) { u[a] = 0.f; dp[a] = 0.f; }
                continue;
            }
            const float* w1 = We1 + (size_t)b * D * H;
            for (int64_t a = 0; a < H; a++) u[a] = 0.f;
            for (int64_t k = 0; k < D; k++) {
                const float xv = xi[k];
                const float* w = w1 + (size_t)k * H;
                for (int64_t a = 0; a < H; a++) u[a] += xv * w[a];
            }
            /* dpre2[a] = sum_j dout[j] We2[b][a][j]  (j ascending) */
            const float* go = dout + (size_t)i * D;
            const float* w2 = We2 + (size_t)b * H * D;
            for (int64_t a = 0; a < H; a++) {
                float acc = 0.f;
                for (int64_t j = 0; j < D; j++) acc += go[j] * w2[(size_t)a * D + j];
                dp[a] = acc;
            }
        }
        free(lg);
    }
    /* derived per-token values: gelu(u), dH = dpre2 * pb * gelu'(u), dpb, dg */
    float* G = (float*)malloc((size_t)M * H * sizeof(float));
    float* DH = (float*)malloc((size_t)M * H * sizeof(float));
    float* DG = (float*)malloc((size_t)M * E * sizeof(float));
    float* PB = (float*)malloc((size_t)(M ? M : 1) * sizeof(float));
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < M; i++) {
        const int64_t b = best[i];
        const float* p = P + (size_t)i * E;
        const float pb = b >= 0 ? p[b] : 0.f;
        PB[i] = pb;
        const float* u = U + (size_t)i * H;
        const float* dp = DP + (size_t)i * H;
        float dpb = 0.f;
        for (int64_t a = 0; a < H; a++) {
            const float uu = u[a];
            const float ga = 0.5f * uu * (1.f + erff(uu * 0.7071067811865476f));
            const float gd = 0.5f * (1.f + erff(uu * 0.7071067811865476f))
                             + uu * expf(-uu * uu * 0.5f) * 0.3989422804014327f;
            G[(size_t)i * H + a] = ga;
            dpb += ga * dp[a];
            DH[(size_t)i * H + a] = dp[a] * pb * gd;
        }
        const float sd = dpb * pb;
        for (int64_t e = 0; e < E; e++)
            DG[(size_t)i * E + e] = p[e] * ((e == b ? dpb : 0.f) - sd);
    }
    if (dx) {
#pragma omp parallel
        {
            float* acc = (float*)malloc((size_t)D * sizeof(float));
#pragma omp for schedule(static)
            for (int64_t i = 0; i < M; i++) {
                float* o = dx + (size_t)i * D;
                for (int64_t k = 0; k < D; k++) o[k] = 0.f;
                const float* dg = DG + (size_t)i * E;
                for (int64_t e = 0; e < E; e++) {
                    const float g = dg[e];
                    for (int64_t k = 0; k < D; k++) o[k] += g * Wg[k * E + e];
                }
                const int64_t b = best[i];
                if (b < 0) continue;
                const float* w1 = We1 + (size_t)b * D * H;
                const float* dh = DH + (size_t)i * H;
                for (int64_t k = 0; k < D; k++) {
                    float a = 0.f;
                    for (int64_t t = 0; t < H; t++) a += dh[t] * w1[(size_t)k * H + t];
                    acc[k] = a;
                }
                for (int64_t k = 0; k < D; k++) o[k] += acc[k];
            }
            free(acc);
        }
    }
    if (dWg) {
        memset(dWg, 0, (size_t)D * E * sizeof(float));
#pragma omp parallel for schedule(static)
        for (int64_t k = 0; k < D; k++)
            for (int64_t i = 0; i < M; i++) {
                const float xv = x[(size_t)i * D + k];
                const float* dg = DG + (size_t)i * E;
                for (int64_t e = 0; e < E; e++) dWg[k * E + e] += xv * dg[e];
            }
    }
    if (dWe1) {
        memset(dWe1, 0, (size_t)E * D * H * sizeof(float));
#pragma omp parallel for schedule(static)
        for (int64_t k = 0; k < D; k++)
            for (int64_t i = 0; i < M; i++) {
                const int64_t b = best[i];
                if (b < 0) continue;
                const float xv = x[(size_t)i * D + k];
                const float* dh = DH + (size_t)i * H;
                float* w = dWe1 + (size_t)b * D * H + (size_t)k * H;
                for (int64_t a = 0; a < H; a++) w[a] += xv * dh[a];
            }
    }
    if (dWe2) {
        memset(dWe2, 0, (size_t)E * H * D * sizeof(float));
#pragma omp parallel for schedule(static)
        for (int64_t a = 0; a < H; a++)
            for (int64_t i = 0; i < M; i++) {
                const int64_t b = best[i];
                if (b < 0) continue;
                const float hp = G[(size_t)i * H + a] * PB[i];
                const float* go = dout + (size_t)i * D;
                float* w = dWe2 + (size_t)b * H * D + (size_t)a * D;
                for (int64_t j = 0; j < D; j++) w[j] += hp * go[j];
            }
    }
    free(best); free(P); free(U); free(DP); free(G); free(DH); free(DG); free(PB);
}

/* ---------------------------------------------------------------------- */
/* optimizer                                                               */
/* ---------------------------------------------------------------------- */

/* Summation order of the MGS dot products: 1 (default) is the reference's
 * order; 2..8 sum as that many interleaved partial sums (k mod P); -2..-8 as
 * that many contiguous blocks of k.  All but 1 are test-only reorderings. */
static int g_mgs_partials = 1;
EXPORT void or_set_mgs_partials(int p) {
    if (p < -8) p = -8;
    if (p > 8) p = 8;
    g_mgs_partials = (p >= -1 && p <= 1) ? 1 : p;
}

/* Modified Gram-Schmidt over columns (M >= N) or rows (M < N), in place;
 * ns_orthonom codegen.cpp:1617-1633.  Right-looking form: when column j is
 * final, every later column is projected against it.  Each column sees the
 * same projections in the same order with the same dot products as the
 * left-looking loop of the reference, so the bits agree. */
EXPORT void or_orthonom(float* G, int64_t M, int64_t N) {
    const int transposed = M < N;
    const int64_t R = transposed ? N : M;
    const int64_t C = transposed ? M : N;
    /* work on columns stored contiguously: T[j][k] */
    float* T = (float*)malloc((size_t)R * C * sizeof(float));
    for (int64_t k = 0; k < R; k++)
        for (int64_t j = 0; j < C; j++)
            T[(size_t)j * R + k] = transposed ? G[(size_t)j * R + k] : G[(size_t)k * N + j];
    for (int64_t j = 0; j < C; j++) {
        float* q = T + (size_t)j * R;
        float nrm = 0.f;
        for (int64_t k = 0; k < R; k++) nrm += q[k] * q[k];
        nrm = sqrtf(nrm) + 1e-30f;
        for (int64_t k = 0; k < R; k++) q[k] /= nrm;
#pragma omp parallel for schedule(static)
        for (int64_t c = j + 1; c < C; c++) {
            float* v = T + (size_t)c * R;
            float dot = 0.f;
            if (g_mgs_partials == 1) {
                for (int64_t k = 0; k < R; k++) dot += q[k] * v[k];
            } else if (g_mgs_partials < 0) {
                /* Test-only: -P contiguous blocks of k, summed in order. */
                float part[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
                const int P = -g_mgs_partials;
                const int64_t blk = (R + P - 1) / P;
                for (int64_t k = 0; k < R; k++) part[k / blk] += q[k] * v[k];
                for (int p = 0; p < P; p++) dot += part[p];
            } else {
                /* Test-only: the same dot product as P interleaved partial
                 * sums, to measure how far a mere change of summation order
                 * moves the reference's training trajectory. */
                float part[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
                const int P = g_mgs_partials;
                for (int64_t k = 0; k < R; k++) part[k % P] += q[k] * v[k];
                for (int p = 0; p < P; p++) dot += part[p];
            }
            for (int64_t k = 0; k < R; k++) v[k] -= dot * q[k];
        }
    }
    for (int64_t k = 0; k < R; k++)
        for (int64_t j = 0; j < C; j++) {
            const float v = T[(size_t)j * R + k];
            if (transposed) G[(size_t)j * R + k] = v; else G[(size_t)k * N + j] = v;
        }
    free(T);
}

/* Muon step with the momentum buffer reset every step (so m = g):
 * codegen.cpp:3099-3107.  g is overwritten by its orthonormalisation. */
EXPORT void or_muon_step(float* w, float* g, int64_t r, int64_t c, float lr) {
    const size_t n = (size_t)r * c;
    for (size_t i = 0; i < n; i++) g[i] = 0.95f * 0.f + g[i];
    or_orthonom(g, r, c);
    const int64_t mn = r < c ? r : c;
    const float rank = sqrtf((float)mn);
    const float le = lr * rank;
    for (size_t i = 0; i < n; i++) w[i] -= le * g[i] + (0.01f * lr) * w[i];
}

/* Bias-corrected AdamW with decoupled decay and a per-weight step counter
 * (t is the value AFTER increment); codegen.cpp:3108-3119. */
EXPORT void or_adamw_step(float* w, const float* g, float* m, float* v, size_t n,
                          int64_t t, float lr) {
    const float b1t = 1.f - powf(0.9f, (float)t), b2t = 1.f - powf(0.999f, (float)t);
    for (size_t i = 0; i < n; i++) {
        const float gg = g[i];
        m[i] = 0.9f * m[i] + 0.1f * gg;
        v[i] = 0.999f * v[i] + 0.001f * gg * gg;
        const float mh = m[i] / b1t, vh = v[i] / b2t;
        w[i] -= (lr * mh / (sqrtf(vh) + 1e-8f)) + (0.01f * lr) * w[i];
    }
}

/* Optimizer rule by shape: Muon iff r > 1, c > 1 and min(r,c) >= 8
 * (codegen.cpp:3097). */
EXPORT int or_use_muon(int64_t r, int64_t c) {
    return r > 1 && c > 1 && (r < c ? r : c) >= 8;
}

/* The runtime wrapper's multiplier lr_scale (optim_params.hpp:54-62, emitted
 * as ns_lr_schedule codegen.cpp:23-39): kind 0 constant; kind 1 linear
 * warmup over `warmup` steps, then a half cosine to `min_factor` at `total`. */
EXPORT float or_lr_scale(int kind, int64_t warmup, int64_t total, float min_factor, int64_t step) {
    if (kind == 0) return 1.0f;
    if (step < warmup) return warmup > 0 ? (float)step / (float)warmup : 1.0f;
    const int64_t end = total > warmup ? total : warmup + 1;
    const int64_t s = step >= end ? end : step;
    const float t = (float)(s - warmup) / (float)(end - warmup);
    return min_factor + 0.5f * (1.0f - min_factor) * (1.0f + cosf(3.14159265f * t));
}

/* Cosine-with-warmup at optim_params.hpp's constants (warmup 100, total
 * 10000, floor 0.05), for hosts that apply the schedule themselves. */
EXPORT float or_lr_scale_cosine(int64_t step) { return or_lr_scale(1, 100, 10000, 0.05f, step); }
