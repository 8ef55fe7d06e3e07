"""The emitted TU's other visible symbols on the GPU (include/ns_emitted.h):
the entry function `forward(input, weights, output, n[, moe_active])`
(codegen.cpp:2263-2288) and `ns_train_core(ctx, ...)` (:2753-3157), held to
the contract the reference's own build shows for them (test_abi.py:
test_reference_forward_symbol_is_eval_infer_with_passed_weights,
test_reference_train_core_symbol_semantics), and the compiled-in LR schedule
carried by the plan (optim_params.hpp:54-62)."""
import numpy as np
import pytest

import helpers
import oracle
from golden.make_golden import case_inputs
from neuralscript_amd import runtime

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name,rows,seed", [("c2s", 29, 102), ("c4k", 37, 105), ("c5s", 64, 103)])
def test_forward_symbol_reads_the_weights_it_is_given(name, rows, seed):
    """forward() equals ns_eval_infer of a model holding the same weights,
    bit for bit, and the oracle within the fp32 bar; a second call with
    other weights gives those weights' output (the blob is read on every
    call); MoE: a NULL mask makes every expert live, a mask with the initial
    experts gives ns_eval_infer's routing; nothing past the output is
    written."""
    print(f"forward symbol {name} rows={rows}", flush=True)
    lib = runtime.net_lib(name)
    net, x, _ = case_inputs(name, rows, seed)
    n_out = net.output_numel(x.size)
    for s in (seed, seed + 1):
        w = helpers.net_weights(name, s)
        ref = oracle.Model(net, w)
        want = ref.eval_infer(x)
        k = want.size
        m = lib.init(w)
        infer = lib.eval_infer(m, x)[:k]
        lib.free(m)
        mask = None
        if net.moe:
            mask = np.zeros(net.moe["E"], np.uint8)
            mask[: net.moe["K0"]] = 1
        got = lib.forward(x, w, n_out, mask)
        assert helpers.bitwise_equal(got[:k], infer)
        assert np.isnan(got[k:]).all()
        helpers.assert_close(got[:k], want, f"{name} forward()")
        if net.moe:
            ref.active[:] = 1
            helpers.assert_close(lib.forward(x, w, n_out, None)[:k], ref.eval_infer(x), f"{name} forward(NULL mask)")


@pytest.mark.parametrize("name,rows,seed", [("mlpt", 17, 7), ("c5s", 64, 11), ("moet", 41, 13)])
def test_train_core_symbol(name, rows, seed):
    """ns_train_core(model, x, n, y, w, wout, &loss, lr, 1) over a model made
    with other weights is one training step from `w`: loss and wout equal
    ns_runtime_train_step of a model made with `w` (constant schedule), bit
    for bit; with train_mode 0 the loss is ns_objective_loss's and wout is
    not written."""
    print(f"ns_train_core symbol {name} rows={rows}", flush=True)
    lib = runtime.net_lib(name)
    net = oracle.Net(helpers.ir_text(name))
    x = helpers.net_inputs(net, name, seed, rows)
    y = helpers.net_labels(net, seed, rows)
    w = helpers.net_weights(name, seed)
    a, b = lib.init(w), lib.init(helpers.net_weights(name, seed + 5))
    loss_a = lib.train_step(a, x, y, 0.02)
    wa = lib.get_weights(a)
    loss_b, wb = lib.train_core(b, x, y, w, 0.02, 1)
    assert helpers.bitwise_equal(np.float32(loss_b), np.float32(loss_a))
    assert helpers.bitwise_equal(wb, wa)
    obj = lib.objective_loss(a, x, y)
    loss_c, wc = lib.train_core(b, x, y, wa, 0.02, 0)
    assert helpers.bitwise_equal(np.float32(loss_c), np.float32(obj))
    assert np.isnan(wc).all()
    lib.free(a)
    lib.free(b)


COSINE = "// ns.lr_schedule cosine_warmup warmup=100 total=10000 min=0.0500000007\n"


def test_cosine_schedule_in_the_plan_scales_the_train_step():
    """A plan carrying the cosine-with-warmup schedule: the first step runs
    at multiplier 0 (warmup from step 0), so both optimizers leave every
    weight exactly as it was while the loss is the forward's; the next four
    steps run at 0.01..0.04 of lr, and losses and weights follow the oracle,
    which applies the same schedule (the weights at the fp32 bar: c5sa's
    step is the AdamW variant, every weight on AdamW)."""
    text = COSINE + helpers.ir_text("c5sa")
    net = oracle.Net(text)
    rows, seed = 64, 21
    x = helpers.net_inputs(net, "c5sa", seed, rows)
    y = helpers.net_labels(net, seed, rows)
    w = helpers.net_weights("c5sa", seed, std=0.1)
    om = oracle.Model(net, w)
    model = runtime.Model(runtime.Plan(text), w)
    for step in range(5):
        loss = model.train_step(x, y, 0.02)
        ref = om.train_step(x, y, 0.02)
        helpers.assert_close(np.float32(loss), ref, f"loss at step {step}")
        wg = model.get_weights()
        if step == 0:
            assert helpers.bitwise_equal(wg, w), "multiplier 0 must leave the weights unchanged"
        helpers.assert_close(wg, om.w, f"weights after step {step}")
    assert not np.array_equal(model.get_weights(), w)
    model.free()
