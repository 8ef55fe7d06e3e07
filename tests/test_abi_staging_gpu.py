"""The host-pointer entry points move their data through pinned staging
(chunks of 16 MiB rotating through three pinned slots; transfers under 2 MiB
go straight through hipMemcpyAsync).  Their results must be bit-identical to
the device-pointer entry points fed by plain copies, for transfers below,
at and across several chunk boundaries."""
import numpy as np
import pytest

import helpers
import oracle
from golden.make_golden import CASES, case_inputs
from neuralscript_amd import runtime, synth, workloads

pytestmark = pytest.mark.gpu

DA = runtime.DeviceArray


@pytest.mark.parametrize("rows", [300, 4096, 6001, 20000])
def test_eval_infer_host_equals_device_path(rows):
    """c2 (1024 -> 4096 -> 4096 -> 1024): 1.2 MB unstaged, 16 MiB exactly one
    chunk, 24.6 MB one and a half chunks, 82 MB five chunks each way (the
    slots wrap around)."""
    print(f"c2 eval rows={rows}", flush=True)
    ir = helpers.ir_text("c2")
    plan = runtime.Plan(ir)
    w = workloads.weights("c2", plan.layout(), workloads.ir_shapes(ir))
    x = synth.uniform(rows, rows * 1024, -1.0, 1.0)
    m = runtime.Model(plan, w)
    host = m.eval_infer(x)
    again = np.full(rows * 1024, np.nan, dtype=np.float32)
    m.eval_infer(x, out=again)  # into the caller's existing array
    dx, dout = DA.from_host(x), DA(rows * 1024)
    m.eval_infer_device(dx, dout)
    m.sync()
    dev = dout.to_host()
    m.free()
    assert np.isfinite(host).all()
    assert helpers.bitwise_equal(host, dev), f"rows={rows}: staged output differs from the device path"
    assert helpers.bitwise_equal(again, dev), f"rows={rows}: a second call into the same array differs"


def test_train_step_host_equals_device_path_and_weights_read_back():
    """c5a (emb 8192x512 ... fc 8192) on 1024 tokens: labels 32 MiB (two
    chunks), weights 46 MB (three chunks) read back after the step."""
    name, rows = "c5a", 1024
    print(f"{name} train rows={rows}", flush=True)
    plan = runtime.Plan(helpers.ir_text(name))
    w = helpers.net_weights(name, 5)
    net = oracle.Net(helpers.ir_text(name))
    x = helpers.net_inputs(net, name, 6, rows)
    y = synth.one_hot(synth.token_ids(7, rows, plan.out_cols), plan.out_cols)
    a, b = runtime.Model(plan, w), runtime.Model(plan, w)
    la = a.train_step(x, y, 0.01)
    lb = b.train_step_device(DA.from_host(x), DA.from_host(y), 0.01)
    assert helpers.bitwise_equal(np.float32(la), np.float32(lb))
    wa, wb = a.get_weights(), b.get_weights()
    assert not helpers.bitwise_equal(wa, w), "the step changed no weight"
    assert helpers.bitwise_equal(wa, wb), "weights after the staged step differ from the device path's"
    # at lr 0 the step leaves every weight as it was: the staged read-back of
    # a device blob newer than the host copy must return it exactly
    c = runtime.Model(plan, w)
    c.train_step(x, y, 0.0)
    assert helpers.bitwise_equal(c.get_weights(), w), "staged weight read-back differs from the blob"
    for mm in (a, b, c):
        mm.free()


@pytest.mark.parametrize("case", CASES, ids=lambda c: c[0])
def test_device_forward_writes_the_callers_buffer(case):
    """The device-pointer forward has the instruction that produces the
    return value write the caller's output buffer itself (no copy after the
    forward); the host-pointer forward keeps the model's own buffer and
    copies it out.  Both must agree bit for bit (outputs pre-filled with NaN:
    some data-movement programs write fewer values than the output size),
    and so must a device call whose output buffer is the input buffer (the
    library then falls back to its own buffer and a copy, as the last
    instruction may still read the input)."""
    name, rows, seed = case[:3]
    print(f"device forward {name} rows={rows}", flush=True)
    ir = helpers.ir_text(name)
    plan = runtime.Plan(ir)
    net, x, _ = case_inputs(name, rows, seed)
    w = helpers.net_weights(name, seed)
    m = runtime.Model(plan, w)
    try:
        n_out = plan.output_numel(x.size)
        host = np.full(n_out, np.nan, np.float32)
        m.eval_infer(x, out=host)
        dx, dout = DA.from_host(x), DA.from_host(np.full(n_out, np.nan, np.float32))
        m.eval_infer_device(dx, dout)
        m.sync()
        assert helpers.bitwise_equal(host, dout.to_host()), f"{name}: device forward differs from the host path"
        both_h = np.full(max(n_out, x.size), np.nan, np.float32)
        both_h[:x.size] = x
        both = DA.from_host(both_h)
        runtime.check(runtime.lib().nsh_eval_infer_device(m.h, both.ptr, both.ptr, x.size), "eval in place")
        m.sync()
        got = both.to_host()[:n_out]
        written = ~np.isnan(host)
        assert helpers.bitwise_equal(host[written], got[written]), f"{name}: in-place device forward differs"
    finally:
        m.free()
