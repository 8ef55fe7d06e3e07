"""fp32-MFMA GEMM (nsh_op_gemm) against the oracle's sequential-k product,
all three operand layouts the runtime uses, ragged and aligned shapes."""
import numpy as np
import pytest

import helpers
import oracle
from neuralscript_amd import runtime, synth

pytestmark = pytest.mark.gpu

# M >= 2048 (nn) runs the 256-row tiles: (2050, 260, 100) has ragged edges on every side
SHAPES = [(1, 1, 1), (3, 5, 2), (37, 45, 29), (128, 128, 16), (130, 257, 100),
          (256, 384, 64), (513, 129, 1031), (1024, 1024, 1024), (8, 4096, 512), (2050, 260, 100),
          (4096, 384, 256)]


def operands(M, N, K, seed):
    A = synth.uniform(seed, M * K, -1, 1)
    B = synth.normal(seed + 1, K * N, float(1 / np.sqrt(max(K, 1))))
    return A, B


@pytest.mark.parametrize("M,N,K", SHAPES)
@pytest.mark.parametrize("variant", ["nn", "nt", "tn"])
def test_gemm_matches_oracle(M, N, K, variant):
    print(f"gemm {variant} M={M} N={N} K={K}", flush=True)
    A, B = operands(M, N, K, M * 7 + N * 3 + K)
    if variant == "nn":
        ref = oracle.matmul(A, B, M, K, N)
        dA, dB, tA, tB, lda, ldb = A, B, False, False, K, N
    elif variant == "nt":  # C = A . Bt^T with Bt [N, K]  (ns_matmul_grad_a)
        Bt = np.ascontiguousarray(B.reshape(K, N).T).ravel()
        ref = oracle.matmul_grad_a(A, Bt, M, N, K)   # dA[M,N] = A[M,K] . Bt[N,K]^T
        dA, dB, tA, tB, lda, ldb = A, Bt, False, True, K, K
    else:  # C = At^T . B with At [K, M]  (ns_matmul_grad_w)
        At = np.ascontiguousarray(A.reshape(M, K).T).ravel()
        ref = oracle.matmul_grad_w(At, B, K, M, N)   # dB[M,N] = At[K,M]^T . B[K,N]
        dA, dB, tA, tB, lda, ldb = At, B, True, False, M, N
    gA, gB = runtime.DeviceArray.from_host(dA), runtime.DeviceArray.from_host(dB)
    gC = runtime.DeviceArray(M * N)
    runtime.gemm(gA, gB, gC, M, N, K, lda, ldb, N, tA, tB, 0)
    helpers.assert_close(gC.to_host(), ref, f"gemm {variant} {M}x{N}x{K}")


@pytest.mark.parametrize("M,N,K", [(70, 96, 48), (2100, 136, 32)])
@pytest.mark.parametrize("act", range(7))
def test_gemm_fused_activation_epilogue(act, M, N, K):
    A, B = operands(M, N, K, 500 + act)
    ref = oracle.matmul(A, B, M, K, N, act)
    gA, gB = runtime.DeviceArray.from_host(A), runtime.DeviceArray.from_host(B)
    gC = runtime.DeviceArray(M * N)
    runtime.gemm(gA, gB, gC, M, N, K, K, N, N, False, False, act)
    helpers.assert_close(gC.to_host(), ref, f"gemm act={act}")


def test_gemm_strided_output_and_zero_k():
    M, N, K = 20, 24, 0
    A = np.zeros(4, np.float32)
    gA, gB = runtime.DeviceArray.from_host(A), runtime.DeviceArray.from_host(A)
    gC = runtime.DeviceArray(M * N)
    runtime.gemm(gA, gB, gC, M, N, K, 4, 24, N, False, False, 3)  # sigmoid(0) = 0.5
    assert np.all(gC.to_host() == 0.5)


@pytest.mark.parametrize("M,N,K,splits", [(64, 64, 4096, 0), (512, 512, 16384, 0), (130, 70, 3001, 5),
                                          (256, 128, 2048, 32), (100, 200, 40, 3), (64, 64, 16, 4)])
@pytest.mark.parametrize("variant", ["tn", "nt"])
def test_gemm_split_k_matches_oracle(M, N, K, splits, variant):
    """Split K (the weight-gradient path of training): fixed-order sum of the
    chunk partials, same result as the one-pass product to fp32 tolerance."""
    print(f"gemm split-k {variant} M={M} N={N} K={K} splits={splits}", flush=True)
    A, B = operands(M, N, K, 900 + M + N + K + splits)
    if variant == "tn":
        At = np.ascontiguousarray(A.reshape(M, K).T).ravel()
        ref = oracle.matmul_grad_w(At, B, K, M, N)
        dA, dB, tA, tB, lda, ldb = At, B, True, False, M, N
    else:
        Bt = np.ascontiguousarray(B.reshape(K, N).T).ravel()
        ref = oracle.matmul_grad_a(A, Bt, M, N, K)
        dA, dB, tA, tB, lda, ldb = A, Bt, False, True, K, K
    gA, gB = runtime.DeviceArray.from_host(dA), runtime.DeviceArray.from_host(dB)
    gC = runtime.DeviceArray(M * N)
    runtime.gemm_splitk(gA, gB, gC, M, N, K, lda, ldb, N, tA, tB, 0, splits)
    helpers.assert_close(gC.to_host(), ref, f"gemm split {variant} {M}x{N}x{K}/{splits}")
