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


@pytest.mark.parametrize("r,c", [(16, 16), (40, 16), (16, 24), (64, 24), (512, 512), (2048, 512), (512, 8192)])
def test_orthonormalize_matches_oracle_mgs(r, c):
    """A square Gaussian matrix is ill-conditioned (cond ~ n), and MGS's Q
    moves by ~eps * cond under a change of summation order, so the square
    case is made well-conditioned by a diagonal shift."""
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
    helpers.assert_close(got, ref, f"mgs {r}x{c}", atol=1e-5, rtol=1e-3)


@pytest.mark.parametrize("r,c", [(16, 12), (24, 16), (16, 40)])
def test_muon_step_matches_oracle(r, c):
    w = synth.normal(1, r * c, 0.2)
    g = synth.normal(2, r * c, 0.5)
    dw, dg, dws = DA.from_host(w), DA.from_host(g), ws(r, c)   # keep the buffers alive across the call
    runtime.lib().nsh_op_muon_step(dw.ptr, dg.ptr, r, c, ctypes.c_float(0.02), dws.ptr)
    ref = w.copy()
    oracle.lib().or_muon_step(oracle.fp(ref), oracle.fp(g.copy()), r, c, ctypes.c_float(0.02))
    helpers.assert_close(dw.to_host(), ref, "muon step")


def test_adamw_steps_are_bit_exact_given_the_gradient():
    n = 1000
    w = synth.normal(3, n)
    dw, dm, dv = DA.from_host(w), DA.from_host(np.zeros(n, np.float32)), DA.from_host(np.zeros(n, np.float32))
    rw, rm, rv = w.copy(), np.zeros(n, np.float32), np.zeros(n, np.float32)
    for t in range(1, 6):
        g = synth.normal(10 + t, n)
        dg = DA.from_host(g)
        runtime.lib().nsh_op_adamw_step(dw.ptr, dg.ptr, dm.ptr, dv.ptr, n, t, ctypes.c_float(0.01))
        oracle.lib().or_adamw_step(oracle.fp(rw), oracle.fp(g), oracle.fp(rm), oracle.fp(rv), n, t,
                                   ctypes.c_float(0.01))
    assert helpers.bitwise_equal(dw.to_host(), rw)
    assert helpers.bitwise_equal(dm.to_host(), rm) and helpers.bitwise_equal(dv.to_host(), rv)


@pytest.mark.parametrize("shapes", [[(16, 12), (24, 16), (16, 40)],
                                    [(40, 16), (16, 16), (16, 16), (16, 16), (16, 16), (16, 24), (24, 16), (16, 12)]])
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
