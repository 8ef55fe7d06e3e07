"""Whole networks through the ns_* C-ABI of the per-network drivers built on
libnship, against the reference fixtures (tests/golden) and the oracle."""
import os

import numpy as np
import pytest

import helpers
import oracle
from golden.make_golden import CASES, case_inputs
from neuralscript_amd import runtime, workloads

pytestmark = pytest.mark.gpu

FWD_NETS = ["c1", "c2s", "xor", "mlpt", "c3s", "c4s", "c4k", "c5t", "moet", "c5s", "moeb", "dmv", "dmw", "bop",
            "dmx", "drp", "c5w"]
# outputs that are pure copies of the input (concat / slice / index / scatter):
# bit-exact
BITWISE = {"dmx"}


def golden(name):
    return np.load(os.path.join(helpers.GOLDEN, f"{name}.npz"))


@pytest.mark.parametrize("case", [c for c in CASES if c[0] in FWD_NETS], ids=lambda c: c[0])
def test_forward_matches_reference_fixture(case):
    name, rows, seed = case[:3]
    print(f"forward {name} rows={rows}", flush=True)
    net, x, _ = case_inputs(name, rows, seed)
    lib = runtime.net_lib(name)
    m = lib.init(helpers.net_weights(name, seed))
    assert m
    out = lib.eval_infer(m, x)
    g = golden(name)["out"]
    if name in BITWISE:
        assert helpers.bitwise_equal(out[: g.size], g), f"{name} forward not bit-exact"
    else:
        helpers.assert_close(out[: g.size], g, f"{name} forward")
    lib.free(m)


@pytest.mark.parametrize("name", FWD_NETS)
def test_forward_of_an_empty_batch(name):
    """ns_eval_infer with zero input rows returns 0 and writes nothing (the
    reference's loops simply do not run); the model stays usable.  dmx slices
    rows 1..2 of a batch-sized value, which the reference would read out of
    bounds: there the call returns -1 instead."""
    print(f"empty batch {name}", flush=True)
    case = next(c for c in CASES if c[0] == name)
    net, x, _ = case_inputs(name, case[1], case[2])
    lib = runtime.net_lib(name)
    m = lib.init(helpers.net_weights(name, case[2]))
    assert lib.output_numel(m, 0) == 0
    empty = np.zeros(0, np.float32)
    if name == "dmx":
        with pytest.raises(RuntimeError):
            lib.eval_infer(m, empty)
    else:
        assert lib.eval_infer(m, empty).size == 0
    out = lib.eval_infer(m, x)
    g = golden(name)["out"]
    if name in BITWISE:
        assert helpers.bitwise_equal(out[: g.size], g)
    else:
        helpers.assert_close(out[: g.size], g, f"{name} forward after an empty batch")
    lib.free(m)


@pytest.mark.parametrize("name", ["c1", "mlpt", "c2s", "xor", "dmv", "smt", "bop"])
def test_forward_of_a_ragged_batch(name):
    """input_numel not a multiple of in_cols: the reference takes
    floor(numel / in_cols) rows (codegen.cpp:1257-1265 with M = numel / K)
    and leaves the partial row unread; outputs against the oracle on the same
    ragged buffer."""
    print(f"ragged batch {name}", flush=True)
    net = oracle.Net(helpers.ir_text(name))
    w = helpers.net_weights(name, 4)
    x = helpers.net_inputs(net, name, 9, 5)
    xr = np.concatenate([x, np.full(net.in_cols - 1, 0.5, np.float32)])
    lib = runtime.net_lib(name)
    m = lib.init(w)
    out = lib.eval_infer(m, xr)
    ref = oracle.Model(net, w).eval_infer(xr)
    lib.free(m)
    helpers.assert_close(out[: ref.size], ref, f"{name} ragged forward")


@pytest.mark.parametrize("name", ["xor"])
def test_train_step_on_a_ragged_batch(name):
    """Training with input_numel not a multiple of in_cols (a net whose
    weights all take AdamW, so the step is determined; Muon on a six-row
    gradient is not): loss and weights after three steps against the oracle
    on the same ragged buffer."""
    print(f"ragged train {name}", flush=True)
    net = oracle.Net(helpers.ir_text(name))
    w = helpers.net_weights(name, 4)
    rows = 6
    x = helpers.net_inputs(net, name, 9, rows)
    xr = np.concatenate([x, np.full(net.in_cols - 1, 0.5, np.float32)])
    y = helpers.net_labels(net, 10, rows)
    lib = runtime.net_lib(name)
    m = lib.init(w)
    om = oracle.Model(net, w)
    for _ in range(3):
        loss, ref = lib.train_step(m, xr, y, 0.05), om.train_step(xr, y, 0.05)
        helpers.assert_close(np.float32([loss]), np.float32([ref]), f"{name} ragged loss")
    helpers.assert_close(lib.get_weights(m), np.asarray(om.w, np.float32), f"{name} ragged weights")
    lib.free(m)


@pytest.mark.parametrize("name", ["c1", "mlpt", "c2s", "smt"])
def test_forward_propagates_inf_and_nan_like_the_reference(name):
    """Rows holding +inf, -inf or NaN inputs: the non-finite outputs sit where
    the oracle's do (same sign for infinities; an infinity and its opposite
    in one sum give NaN in any order), and the rows without special values
    match to the fp32 bar."""
    print(f"special values {name}", flush=True)
    net = oracle.Net(helpers.ir_text(name))
    w = helpers.net_weights(name, 4)
    rows = 8
    x = helpers.net_inputs(net, name, 9, rows).reshape(rows, net.in_cols).copy()
    x[1, 0] = np.inf
    x[3, -1] = -np.inf
    x[5, 1] = np.nan
    x[6, 0], x[6, 1] = np.inf, -np.inf
    lib = runtime.net_lib(name)
    m = lib.init(w)
    out = lib.eval_infer(m, x.ravel())
    ref = oracle.Model(net, w).eval_infer(x.ravel())
    lib.free(m)
    out = out[: ref.size].reshape(rows, -1)
    ref = ref.reshape(rows, -1)
    assert np.array_equal(np.isnan(out), np.isnan(ref)), "NaN positions differ"
    assert np.array_equal(np.isposinf(out), np.isposinf(ref)) and np.array_equal(np.isneginf(out), np.isneginf(ref))
    clean = [r for r in range(rows) if r not in (1, 3, 5, 6)]
    helpers.assert_close(out[clean], ref[clean], f"{name} rows without special values")


def test_c2_full_size_rows_match_oracle():
    """Config 2 at its full batch (8192 x 1024 -> 4096 -> 4096 -> 1024, GELU);
    the oracle recomputes 96 rows spread over the batch (rows are independent)."""
    print("c2 full size", flush=True)
    ir = helpers.ir_text("c2")
    plan = runtime.Plan(ir)
    shapes = workloads.ir_shapes(ir)
    w = workloads.weights("c2", plan.layout(), shapes)
    x = workloads.inputs("c2")
    lib = runtime.net_lib("c2")
    m = lib.init(w)
    out = lib.eval_infer(m, x).reshape(8192, 1024)
    lib.free(m)
    rows = np.unique(np.linspace(0, 8191, 96).astype(np.int64))
    om = oracle.Model(oracle.Net(ir), w)
    ref = om.eval_infer(x.reshape(8192, 1024)[rows]).reshape(len(rows), 1024)
    helpers.assert_close(out[rows], ref, "c2 rows")
    assert np.isfinite(out).all()


def test_c1_stated_workload_matches_reference_driver():
    """Config 1 exactly as stated (batch 256, Xavier-uniform weights, U[-1,1]
    inputs): the network driver over libnship against the reference's own
    emitted driver's output (tests/golden/c1_workload.npz)."""
    from golden.make_golden import digest
    g = np.load(os.path.join(helpers.GOLDEN, "c1_workload.npz"))
    ir = helpers.ir_text("c1")
    plan = runtime.Plan(ir)
    w = workloads.weights("c1", plan.layout(), workloads.ir_shapes(ir))
    x = workloads.inputs("c1")
    assert digest(x) == str(g["x_digest"]) and digest(w) == str(g["w_digest"]), "input generator drifted"
    lib = runtime.net_lib("c1")
    m = lib.init(w)
    out = lib.eval_infer(m, x)
    lib.free(m)
    helpers.assert_close(out, g["out"], "c1 at its stated workload")


def test_checkpoint_round_trip_and_errors(tmp_path):
    name = "c2s"
    lib = runtime.net_lib(name)
    w0 = helpers.net_weights(name, 1)
    w1 = helpers.net_weights(name, 2)
    a, b = lib.init(w0), lib.init(w1)
    pa, pb = str(tmp_path / "a.nsm"), str(tmp_path / "b.nsm")
    assert lib.save(a, pa) == 0 and lib.save(b, pb) == 0
    assert lib.load(a, pb) == 0
    assert helpers.bitwise_equal(lib.get_weights(a), w1)
    net = oracle.Net(helpers.ir_text(name))
    x = helpers.net_inputs(net, name, 3, 11)
    assert helpers.bitwise_equal(lib.eval_infer(a, x), lib.eval_infer(b, x))
    assert lib.load(a, str(tmp_path / "missing.nsm")) == -1
    assert lib.save(None, pa) == -1
    with open(pa, "rb") as f:
        raw = f.read()
    assert raw[:4] == b"2MSN" and int.from_bytes(raw[4:12], "little") == w0.size
    with open(str(tmp_path / "trunc.nsm"), "wb") as f:
        f.write(raw[:100])
    assert lib.load(a, str(tmp_path / "trunc.nsm")) == -1
    assert helpers.bitwise_equal(lib.get_weights(a), w1)  # failed load leaves the model intact
    assert lib.lib.ns_runtime_init(None, 0) is None
    short = np.zeros(3, np.float32)
    assert lib.init(short) is None
    lib.free(a)
    lib.free(b)
    lib.free(None)
