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


# ---- the first Muon update at full size (tests/golden/c5_full_update.npz) ----
# Muon's update is -lr sqrt(k) Q - 0.01 lr W with Q = MGS(gradient), k =
# min(r, c): its Frobenius norm is lr * k up to the decay term whatever the
# summation order (every Q vector is a unit vector), and Q's vectors on the
# gradient's determined prefix are implementation-independent.  Q entries are
# compared at the fixture's sampled (vector, element) positions.

MUON_NORM_RTOL = 1e-3
# Largest |Q_gpu - Q_oracle| allowed on c5's full-size first update (entries
# of unit vectors of length 512..8192, i.e. typically 0.011..0.044) unless
# the oracle's own Q moves more than an eighth of that under 1-ulp weight
# noise (muon_q_tolerance).
C5_Q_ATOL = 2e-3


def muon_update_stats(w0, w1, lr, weights, offsets, ref):
    """Per Muon matrix: (|W1 - W0|_F, Q at the fixture's sampled positions)
    of the step W0 -> W1 taken at learning rate lr."""
    out = {}
    lr = np.float32(lr)
    for name, r, c in weights:
        o = offsets[name]
        a = np.asarray(w0[o:o + r * c], np.float64)
        b = np.asarray(w1[o:o + r * c], np.float64)
        le = np.float64(lr) * np.sqrt(np.float32(min(r, c)))
        q = ((a - b) - 0.01 * np.float64(lr) * a) / le
        q = q.reshape(r, c) if r < c else q.reshape(r, c).T
        out[name] = (float(np.linalg.norm(b - a)), q[ref[f"{name}:vi"], ref[f"{name}:ei"]])
    return out


def muon_q_tolerance(ref, name, q_atol):
    """q_atol, or 8x the largest movement of the same Q entries in the
    oracle's own step from 1-ulp-perturbed weights, whichever is larger (the
    GPU's reductions differ from the reference's in every operation, not by
    one ulp of the inputs; at c5's full size its deviations measure 1-6x
    that movement)."""
    key = f"{name}:q_ulp"
    if key not in ref:
        return q_atol
    return max(q_atol, 8.0 * float(np.max(np.abs(ref[key] - ref[f"{name}:q"]))))


def muon_update_failures(stats, ref, q_atol):
    """Reasons the update `stats` disagrees with the oracle's (empty list:
    agrees): the norm within MUON_NORM_RTOL, the sampled Q entries (all on
    the determined prefix) within muon_q_tolerance."""
    fails = []
    for name, (norm, q) in stats.items():
        rn = float(ref[f"{name}:norm"])
        if not abs(norm - rn) <= MUON_NORM_RTOL * rn:
            fails.append(f"{name}: |dW| {norm:.6g} vs {rn:.6g}")
        d = float(np.max(np.abs(q - ref[f"{name}:q"])))
        tol = muon_q_tolerance(ref, name, q_atol)
        if not d <= tol:
            fails.append(f"{name}: max |dQ| {d:.3g} > {tol:.3g} on the determined prefix")
    return fails
