"""Bandwidth kernels against the oracle: embedding gather (bit-exact rows),
LayerNorm forward/backward, fused softmax cross-entropy, activation
backward, embedding weight gradient (bit-exact, token order)."""
import numpy as np
import pytest

import helpers
import oracle
from neuralscript_amd import runtime, synth
from neuralscript_amd.runtime import DeviceArray as DA

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n,V,D", [(1, 1, 1), (333, 50, 96), (2048, 32000, 1024), (100, 7, 13)])
def test_embedding_gather_is_bit_exact(n, V, D):
    print(f"embedding n={n} V={V} D={D}", flush=True)
    W = synth.normal(n + V, V * D)
    idx = synth.token_ids(7, n, V)
    if n >= 100:  # edge ids: negatives above -1, out of range, NaN, huge
        idx[:9] = np.array([-0.5, -1, V, V - 0.25, 1e30, -1e30, np.nan, np.inf, V + 3], np.float32)
    out = DA(n * D)
    runtime.op("embedding", DA.from_host(W), DA.from_host(idx), out, n, V, D)
    assert helpers.bitwise_equal(out.to_host(), oracle.embedding(W, idx, V, D))


# (1, 4), (77, 96), (5, 300), (31, 256), (4096, 512): two rows per wave, row
# counts not a multiple of the 8 rows a workgroup covers
@pytest.mark.parametrize("rows,last", [(1, 4), (77, 96), (5, 300), (31, 256), (4096, 512), (1000, 1024), (37, 2048),
                                       (5, 3000), (9, 7)])
def test_layernorm_forward(rows, last):
    x = synth.normal(rows * 3 + last, rows * last, 2.0) + 0.5
    y = DA(rows * last)
    runtime.op("layernorm", DA.from_host(x), y, rows, last)
    helpers.assert_close(y.to_host(), oracle.layernorm(x, last), f"layernorm {rows}x{last}")


# rows in registers (up to 256, 512, 1024 columns, ragged ones included) and
# the streaming kernel (wider rows, or widths off a multiple of 4)
@pytest.mark.parametrize("rows,last", [(50, 64), (77, 96), (5, 300), (4096, 512), (3, 1000), (1000, 1024),
                                       (37, 2048), (9, 7)])
def test_layernorm_backward(rows, last):
    x = synth.normal(rows + 1, rows * last, 1.5)
    d = synth.normal(rows + 2, rows * last, 0.1)
    dx = DA(rows * last)
    runtime.op("layernorm_grad", DA.from_host(d), DA.from_host(x), dx, rows, last)
    helpers.assert_close(dx.to_host(), oracle.layernorm_grad(d, x, last), f"layernorm_grad {rows}x{last}")


@pytest.mark.parametrize("rows,C", [(1, 2), (129, 10), (512, 8192), (64, 2048), (100, 4096), (33, 4000), (7, 12288),
                                    (5, 2050), (16387, 16)])
def test_softmax_cross_entropy_and_seed(rows, C):
    x = synth.normal(rows + C, rows * C, 3.0)
    y = synth.one_hot(synth.token_ids(rows, rows, C), C)
    g, rl, loss = DA(rows * C), DA(rows), DA(1)
    runtime.op("softmax_xent", DA.from_host(x), DA.from_host(y), g, rl, loss, rows, C)
    helpers.assert_close(g.to_host(), oracle.loss_grad(x, y, C), "loss grad")
    ref = oracle.cross_entropy(x, y, C)
    assert abs(loss.to_host()[0] - ref) <= 1e-5 + 1e-4 * abs(ref)


@pytest.mark.parametrize("act", range(7))
def test_activation_backward(act):
    n = 10007
    din, pre = synth.normal(1, n), synth.normal(2, n, 2.0)
    out = DA(n)
    runtime.op("act_grad", DA.from_host(din), DA.from_host(pre), out, n, act)
    helpers.assert_close(out.to_host(), oracle.act_grad(din, pre, act), f"act_grad {act}")


@pytest.mark.parametrize("n,V,D,mode", [(16384, 8192, 512, "uniform"), (3000, 40, 16, "uniform"),
                                        (700, 50, 33, "same"), (500, 1000, 8, "edge"),
                                        (4096, 64, 512, "same"), (20000, 300, 1024, "skew"),
                                        (5000, 20000, 64, "uniform"), (32768, 8191, 1000, "uniform"),
                                        (0, 37, 8, "uniform"), (40000, 8192, 512, "uniform"),
                                        (50000, 300, 64, "skew"), (33000, 17, 20, "same"),
                                        (16384, 8192, 512, "zipf"), (16384, 8192, 512, "heavy65"),
                                        (32768, 8191, 1000, "skew"), (12000, 700, 60, "skew"),
                                        (9000, 100, 21, "zipf")])
def test_embedding_grad_is_bit_exact(n, V, D, mode):
    """Row sums in ascending token order, float4 columns (D % 4 == 0: one,
    two or four float4 per lane) or scalar ones.  Up to 32768 tokens one
    launch walks per-row token bitmaps (32768: the bitmaps fill 128 KB of
    LDS; no tokens: every row zero), and a float4 row hit by more than 64
    tokens is summed by the whole workgroup, 8 tokens per load, in token
    order (one row taking every token, Zipf-distributed ids, rows of exactly
    64 and 65 tokens, partial column groups at D = 60 and 1000); beyond 32768
    tokens, the counting-sort path: short segments sorted per thread, long
    ones (one row taking every token; several heavy rows in one block under
    skewed ids) by the workgroup."""
    print(f"embedding_grad n={n} V={V} D={D} {mode}", flush=True)
    if mode == "same":
        idx = np.full(n, 3.0, np.float32)   # one row takes every token
    elif mode == "skew":
        # a few rows take most tokens: segments of hundreds to thousands
        idx = np.minimum(np.random.default_rng(13).pareto(1.1, n), V - 1).astype(np.int64).astype(np.float32)
    elif mode == "zipf":
        # word-frequency-like ids: row 0 takes ~18% of the tokens
        idx = np.minimum(np.random.default_rng(14).zipf(1.2, n) - 1, V - 1).astype(np.float32)
    elif mode == "heavy65":
        # rows 5 and 6 (one workgroup) hit by exactly 64 and 65 tokens, row 40
        # (another) by 65, the rest uniform over rows >= 64
        idx = synth.token_ids(11, n, V - 64) + 64
        pos = np.random.default_rng(15).permutation(n)[:194]
        idx[pos[:64]], idx[pos[64:129]], idx[pos[129:]] = 5, 6, 40
    else:
        idx = synth.token_ids(11, n, V)
    if mode == "edge":
        idx[:6] = np.array([-1, V, np.nan, -0.5, V - 0.5, 1e20], np.float32)
    d = synth.normal(12, n * D)
    ws = DA(runtime.lib().nsh_op_embedding_grad_workspace(n, V) // 4 + 1)
    dW = DA(V * D)
    runtime.op("embedding_grad", DA.from_host(d), DA.from_host(idx), dW, n, V, D, ws)
    assert helpers.bitwise_equal(dW.to_host(), oracle.embedding_grad_w(d, idx, V, D))
