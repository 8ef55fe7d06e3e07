"""Shared test helpers: bundled network plans, seeded weights and inputs, and
the parity check used against the oracle."""
import os

import numpy as np

from neuralscript_amd import synth, workloads

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
NETS = os.path.join(ROOT, "neuralscript_amd", "nets")
GOLDEN = os.path.join(ROOT, "tests", "golden")
REF = os.path.join(ROOT, "oracle", "_ref")

# Parity bar for fp32 outputs:
# |gpu - oracle| <= 1e-5 + 1e-4 * |oracle|.
ATOL, RTOL = 1e-5, 1e-4


def ir_text(name):
    with open(os.path.join(NETS, name + ".mlir")) as f:
        return f.read()


def shapes(name):
    return workloads.ir_shapes(ir_text(name))


def layout(name):
    out, off = [], 0
    for n, (r, c) in shapes(name).items():
        out.append((n, off, r * c))
        off += r * c
    return out


def net_weights(name, seed, std=0.2):
    return workloads.generic_weights(layout(name), shapes(name), seed, std)


def net_inputs(net, name, seed, M):
    """Token ids for embedding-first nets, N(0,1) rows for MoE-first nets,
    U[-1,1] rows otherwise."""
    s = synth.stream_seed(seed, "x")
    if net.in_cols == 1 and net.moe is None or net.fwd.instrs and any(
            i.op == "ns.layer.embedding" for i in net.fwd.instrs):
        V = net.weights[0][1]
        return synth.token_ids(s, M, V)
    if net.moe is not None and net.in_cols == 1:
        return synth.normal(s, M * net.moe["D"])
    return synth.uniform(s, M * net.in_cols, -1, 1)


def net_labels(net, seed, M):
    C = net.out_cols
    return synth.one_hot(synth.token_ids(synth.stream_seed(seed, "y"), M, C), C)


def violation(out, ref, atol=ATOL, rtol=RTOL):
    """Largest |out-ref| / (atol + rtol*|ref|); <= 1 passes."""
    out = np.asarray(out, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    if out.shape != ref.shape:
        raise AssertionError(f"shape {out.shape} != {ref.shape}")
    if out.size == 0:
        return 0.0
    return float(np.max(np.abs(out - ref) / (atol + rtol * np.abs(ref))))


def assert_close(out, ref, what, atol=ATOL, rtol=RTOL):
    v = violation(out, ref, atol, rtol)
    assert np.all(np.isfinite(out)), f"{what}: non-finite output"
    assert v <= 1.0, f"{what}: tolerance exceeded by x{v:.3g} (max |d| {np.max(np.abs(np.asarray(out, np.float64) - ref)):.3g})"


def bitwise_equal(a, b):
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))
