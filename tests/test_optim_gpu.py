"""Optimizer kernels against the oracle: MGS orthonormalisation (columns and
rows), the Muon step, the AdamW step over several steps."""
import ctypes

import numpy as np
import pytest

import helpers
import oracle
from neuralscript_amd import runtime, synth
from neuralscript_amd.runtime import DeviceArray as DA

pytestmark = pytest.mark.gpu


def ws(r, c):
    return DA(runtime.lib().nsh_op_muon_workspace(r, c) // 4 + 64)


# Register panels (512 threads, up to 16 elements a thread): every vector
# length class, 1 (<= 512), 2 (<= 1024), 4, 8 (<= 4096) and 16 (<= 8192)
# elements a thread, with float4 rows (length % 4 == 0) and scalar ones, and
# ragged last panels (vector counts not multiples of 8).
# (9000, 24), (24, 9000), (8193, 40), (20000, 19), (19, 20001), (262144, 64),
# (64, 100000): vectors longer than 8192 floats take the sliced path
# (2048-float slices, panels of 8 columns: MGS inside a panel, block
# projections across panels) instead of the register panels; odd lengths
# take its scalar loads, 19 vectors a ragged last panel of 3
@pytest.mark.parametrize("r,c", [(16, 16), (40, 16), (16, 24), (64, 24), (512, 512), (2048, 512), (512, 8192),
                                 (1000, 40), (3001, 24), (4096, 20), (5001, 24), (24, 6000), (8192, 9),
                                 (9000, 24), (24, 9000), (8193, 40), (20000, 19), (19, 20001), (262144, 64),
                                 (64, 100000)])
def test_orthonormalize_matches_oracle_mgs(r, c):
    """Q within the fp32 bar (1e-5 + 1e-4 |ref|) of the oracle's.  A square
    Gaussian matrix is ill-conditioned (cond ~ n), and MGS's Q moves by ~eps
    * cond under a change of summation order, so the square case is made
    well-conditioned by a diagonal shift."""
    print(f"mgs {r}x{c}", flush=True)
    g = synth.normal(r * 7 + c, r * c)
    if r == c:
        g = (g.reshape(r, c) + 4.0 * np.sqrt(r) * np.eye(r, dtype=np.float32)).ravel()
    q = DA(r * c)
    runtime.op("orthonormalize", DA.from_host(g), q, r, c, ws(r, c))
    ref = oracle.orthonom(g, r, c)
    got = q.to_host()
    Q = got.reshape(r, c).astype(np.float64)
    if r < c:
        Q = Q.T
    orth = np.abs(Q.T @ Q - np.eye(Q.shape[1])).max()
    print(f"  max |Q^T Q - I| = {orth:.3g}, max |q - ref| = {np.abs(got - ref).max():.3g}")
    helpers.assert_close(got, ref, f"mgs {r}x{c}")


# Gradients whose rows are zero in every vector (an embedding's unused
# vocabulary rows).  Compacted to the live rows when that moves the vectors
# into a smaller register layout: 8192 -> ~3300 (16 -> 8 elements a thread),
# 2048 -> ~410 (4 -> 1), odd 5001 -> ~2500 (scalar rows, 16 -> 8), and the
# transposed case (zero columns of a [64, 8192] gradient); left as they are
# otherwise: 30% zero rows of 8192 (still 16 a thread), an all-zero matrix.
@pytest.mark.parametrize("r,c,frac", [(8192, 64, 0.6), (64, 8192, 0.6), (2048, 100, 0.8), (5001, 24, 0.5),
                                      (8192, 40, 0.3), (4096, 16, 1.0)])
def test_orthonormalize_with_zero_rows(r, c, frac):
    """Q against the oracle at the fp32 bar, exactly zero in the zero rows;
    then the whole Muon step (the weight decay still applies to those
    rows)."""
    print(f"mgs zero rows {r}x{c} frac={frac}", flush=True)
    g = synth.normal(r + 3 * c, r * c).reshape(r, c)
    rng = np.random.default_rng(r + c)
    if r >= c:
        dead = rng.random(r) < frac
        g[dead, :] = 0.0
    else:
        dead = rng.random(c) < frac
        g[:, dead] = 0.0
    g = g.ravel()
    q = DA(r * c)
    runtime.op("orthonormalize", DA.from_host(g), q, r, c, ws(r, c))
    got = q.to_host()
    helpers.assert_close(got, oracle.orthonom(g, r, c), f"mgs {r}x{c} with zero rows")
    G = got.reshape(r, c)
    assert not np.any(G[dead, :] if r >= c else G[:, dead])
    w = synth.normal(5, r * c, 0.2)
    dw, dg, dws = DA.from_host(w), DA.from_host(g), ws(r, c)  # buffers live across the call
    runtime.lib().nsh_op_muon_step(dw.ptr, dg.ptr, r, c, ctypes.c_float(0.02), dws.ptr)
    ref = w.copy()
    oracle.lib().or_muon_step(oracle.fp(ref), oracle.fp(g.copy()), r, c, ctypes.c_float(0.02))
    helpers.assert_close(dw.to_host(), ref, f"muon step {r}x{c} with zero rows")


def shifted(a, off):
    """A device copy of `a` starting `off` floats into its buffer (off = 1
    leaves the data 4 bytes past a 16-byte boundary)."""
    d = DA.from_host(np.concatenate([np.zeros(off, np.float32), a]))
    return d, d.ptr + 4 * off


# float4 transposes with ragged 64 x 64 tiles (r, c multiples of 4), the
# scalar 32 x 32 path (r or c odd, or a base off 16-byte alignment), and the
# row-vector (r < c) copies of both kinds
@pytest.mark.parametrize("r,c,off", [(16, 12, 0), (24, 16, 0), (16, 40, 0), (200, 72, 0), (72, 200, 0),
                                     (18, 12, 0), (12, 42, 0), (200, 72, 1), (72, 200, 1)])
def test_muon_step_matches_oracle(r, c, off):
    w = synth.normal(1, r * c, 0.2)
    g = synth.normal(2, r * c, 0.5)
    (dw, pw), (dg, pg), dws = shifted(w, off), shifted(g, off), ws(r, c)  # buffers live across the call
    runtime.lib().nsh_op_muon_step(pw, pg, r, c, ctypes.c_float(0.02), dws.ptr)
    ref = w.copy()
    oracle.lib().or_muon_step(oracle.fp(ref), oracle.fp(g.copy()), r, c, ctypes.c_float(0.02))
    helpers.assert_close(dw.to_host()[off:], ref, "muon step")


# float4 path with and without an n % 4 tail, one-element path (n < 4 or a
# base off 16-byte alignment)
@pytest.mark.parametrize("n,off", [(1000, 0), (1003, 0), (3, 0), (1003, 1), (262147, 0)])
def test_adamw_steps_are_bit_exact_given_the_gradient(n, off):
    w = synth.normal(3, n)
    z = np.zeros(n, np.float32)
    (dw, pw), (dm, pm), (dv, pv) = shifted(w, off), shifted(z, off), shifted(z, off)
    rw, rm, rv = w.copy(), np.zeros(n, np.float32), np.zeros(n, np.float32)
    for t in range(1, 6):
        g = synth.normal(10 + t, n)
        dg, pg = shifted(g, off)
        runtime.lib().nsh_op_adamw_step(pw, pg, pm, pv, n, t, ctypes.c_float(0.01))
        oracle.lib().or_adamw_step(oracle.fp(rw), oracle.fp(g), oracle.fp(rm), oracle.fp(rv), n, t,
                                   ctypes.c_float(0.01))
    assert helpers.bitwise_equal(dw.to_host()[off:], rw)
    assert helpers.bitwise_equal(dm.to_host()[off:], rm) and helpers.bitwise_equal(dv.to_host()[off:], rv)


@pytest.mark.parametrize("shapes", [[(16, 12), (24, 16), (16, 40)],
                                    [(40, 16), (16, 16), (16, 16), (16, 16), (16, 16), (16, 24), (24, 16), (16, 12)],
                                    # more matrices than one gather launch takes (64), ragged and float4 shapes
                                    [(16 + i % 5, 12 + 4 * (i % 3)) if i % 2 else (12 + 4 * (i % 3), 17 + i % 4)
                                     for i in range(70)] + [(130, 72), (72, 260)],
                                    # long vectors (sliced path) beside register-panel matrices
                                    [(9000, 24), (64, 24), (20, 20000), (24, 16)]])
def test_muon_multi_matches_oracle(shapes):
    n = len(shapes)
    ws_ = [synth.normal(20 + i, r * c, 0.2) for i, (r, c) in enumerate(shapes)]
    gs_ = [synth.normal(40 + i, r * c, 0.5) for i, (r, c) in enumerate(shapes)]
    dw = [DA.from_host(w) for w in ws_]
    dg = [DA.from_host(g) for g in gs_]
    R = np.array([r for r, c in shapes], np.int64)
    C = np.array([c for r, c in shapes], np.int64)
    wp = (ctypes.c_void_p * n)(*[d.ptr for d in dw])
    gp = (ctypes.c_void_p * n)(*[d.ptr for d in dg])
    wsz = runtime.lib().nsh_op_muon_multi_workspace(n, R.ctypes.data, C.ctypes.data)
    work = DA(wsz // 4 + 64)
    runtime.check(runtime.lib().nsh_op_muon_multi(n, wp, gp, R.ctypes.data, C.ctypes.data, ctypes.c_float(0.02),
                                                  work.ptr), "muon_multi")
    for i, (r, c) in enumerate(shapes):
        ref = ws_[i].copy()
        oracle.lib().or_muon_step(oracle.fp(ref), oracle.fp(gs_[i].copy()), r, c, ctypes.c_float(0.02))
        helpers.assert_close(dw[i].to_host(), ref, f"muon multi matrix {i} {r}x{c}")


@pytest.mark.parametrize("r,c,zero", [(24, 9000, (3, 10, 17)), (20000, 19, (0, 8, 18)),
                                      (32, 30000, tuple(range(20, 32))), (40000, 24, (5,) + tuple(range(9, 24)))])
def test_sliced_orthonormalize_with_zero_vectors(r, c, zero):
    """Zero gradient vectors (a MoE expert without tokens) on the sliced
    path: MGS's +1e-30 guard gives them q = 0, in the panel that holds them
    and as projections of the later panels; everything else as the oracle.
    Zero vectors are not processed at all: the sliced launches run over the
    list of nonzero ones (here also the last 12 of 32, the last 15 of 24)."""
    print(f"mgs zero vectors {r}x{c} {zero}", flush=True)
    g = synth.normal(r * 5 + c, r * c).reshape(r, c)
    for z in zero:
        if r < c:
            g[z, :] = 0.0
        else:
            g[:, z] = 0.0
    g = g.ravel()
    q = DA(r * c)
    runtime.op("orthonormalize", DA.from_host(g), q, r, c, ws(r, c))
    got = q.to_host()
    helpers.assert_close(got, oracle.orthonom(g, r, c), f"mgs {r}x{c} with zero vectors")
    Q = got.reshape(r, c)
    for z in zero:
        assert not np.any(Q[z, :] if r < c else Q[:, z]), z
