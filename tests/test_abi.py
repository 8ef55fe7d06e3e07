"""CPU checks of the drop-in boundary: the libraries load, export every
symbol the headers declare, and the plan parser reproduces the reference's
static tables (no device calls)."""
import ctypes
import os
import re

import numpy as np
import pytest

import helpers
import oracle
from neuralscript_amd import runtime
from neuralscript_amd.abi import NsLib

INCLUDE = os.path.join(helpers.ROOT, "include")


def declared(header):
    text = open(os.path.join(INCLUDE, header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ns[h]?_\w+)\s*\(", text)))


def test_libnship_exports_every_declared_symbol():
    L = ctypes.CDLL(runtime.LIB_PATH)
    missing = [s for s in declared("nship.h") if not hasattr(L, s)]
    assert not missing, missing


@pytest.mark.parametrize("name", runtime.bundled_nets())
def test_network_driver_exports_the_runtime_abi(name):
    lib = runtime.net_lib(name)
    net = oracle.Net(helpers.ir_text(name))
    want = [s for s in declared("ns_runtime.h")
            if not s.startswith("ns_expert") and s not in ("ns_runtime_train_step", "ns_objective_loss")]
    if net.moe:
        want += ["ns_expert_count", "ns_expert_birth", "ns_expert_merge", "ns_expert_kill"]
    if net.train:
        want += ["ns_runtime_train_step", "ns_objective_loss"]
    # the emitted TU's other visible symbols (include/ns_emitted.h)
    want += [s for s in declared("ns_emitted.h") if s != "ns_train_core" or net.train]
    want.append("forward")
    missing = [s for s in want if not hasattr(lib.lib, s)]
    assert not missing, missing


def _ref_lib(name):
    path = os.path.join(helpers.REF, f"lib{name}.so")
    if not os.path.exists(path):
        pytest.skip("reference build not present")
    return NsLib(path)


@pytest.mark.parametrize("name,rows,seed", [("c2s", 29, 102), ("c4k", 37, 105), ("c5s", 64, 103)])
def test_reference_forward_symbol_is_eval_infer_with_passed_weights(name, rows, seed):
    """What the reference's exported entry function does (codegen.cpp:
    2263-2288), on its own build: forward(input, weights, output, n[,
    moe_active]) equals ns_eval_infer of a model holding `weights`, bit for
    bit; the weights are read on every call (a second blob gives that
    blob's output); for MoE networks the mask decides the live experts
    (NULL = all live).  The GPU tests hold libnship's `forward` to the same
    contract."""
    from golden.make_golden import case_inputs
    ref = _ref_lib(name)
    net, x, _ = case_inputs(name, rows, seed)
    w = helpers.net_weights(name, seed)
    w2 = helpers.net_weights(name, seed + 1)
    n_out = net.output_numel(x.size)
    for weights in (w, w2):
        m = ref.init(weights)
        k = oracle.Model(net, weights).eval_infer(x).size  # floats the forward writes (F3: < n_out for MoE)
        want = ref.eval_infer(m, x)[:k]
        ref.free(m)
        mask = np.zeros(net.moe["E"], np.uint8) if net.moe else None
        if net.moe:
            mask[: net.moe["K0"]] = 1
        got = ref.forward(x, weights, n_out, mask)
        assert helpers.bitwise_equal(got[:k], want)
        assert np.isnan(got[k:]).all()
        if net.moe:
            allive = oracle.Model(net, weights)
            allive.active[:] = 1
            assert helpers.bitwise_equal(ref.forward(x, weights, n_out, None)[:k], allive.eval_infer(x)[:k])


@pytest.mark.parametrize("name,rows,seed", [("mlpt", 17, 7), ("c5s", 64, 11)])
def test_reference_train_core_symbol_semantics(name, rows, seed):
    """The reference's exported training core on its own build:
    ns_train_core(ctx, x, n, y, w, wout, &loss, lr, 1) with w = the model's
    weights is one ns_runtime_train_step under the constant schedule (same
    loss, wout = the trained weights, bit for bit), and with train_mode 0 it
    returns the objective and writes nothing to wout."""
    from neuralscript_amd.abi import reference_ctx
    ref = _ref_lib(name)
    net = oracle.Net(helpers.ir_text(name))
    x = helpers.net_inputs(net, name, seed, rows)
    y = helpers.net_labels(net, seed, rows)
    w = helpers.net_weights(name, seed)
    a, b = ref.init(w), ref.init(w)
    loss_a = ref.train_step(a, x, y, 0.02)
    wa = ref.get_weights(a)
    loss_b, wb = ref.train_core(reference_ctx(b), x, y, w, 0.02, 1)
    assert helpers.bitwise_equal(np.float32(loss_b), np.float32(loss_a))
    assert helpers.bitwise_equal(wb, wa)
    obj = ref.objective_loss(a, x, y)
    loss_c, wc = ref.train_core(reference_ctx(a), x, y, wa, 0.02, 0)
    assert helpers.bitwise_equal(np.float32(loss_c), np.float32(obj))
    assert np.isnan(wc).all()
    ref.free(a)
    ref.free(b)


COSINE = "// ns.lr_schedule cosine_warmup warmup=100 total=10000 min=0.0500000007\n"


def test_plan_carries_the_lr_schedule():
    """The IR line `// ns.lr_schedule ...` selects the wrapper's multiplier
    (optim_params.hpp:54-62): absent = constant 1 (what the reference
    compiles); cosine_warmup at optim_params.hpp's constants gives the
    oracle's lr_scale_cosine bit for bit at every step tried (warmup, the
    cosine tail, the clamp past `total`); other constants follow the same
    formula; a malformed line fails the parse."""
    L = runtime.lib()
    L.nsh_plan_lr_scale.restype = ctypes.c_float
    L.nsh_plan_lr_scale.argtypes = [ctypes.c_void_p, ctypes.c_int64]
    ir = helpers.ir_text("mlpt")
    const = runtime.Plan(ir)
    cos = runtime.Plan(COSINE + ir)
    other = runtime.Plan("// ns.lr_schedule cosine_warmup warmup=10 total=50 min=0.25\n" + ir)
    sched = {"kind": 1, "warmup": 10, "total": 50, "min": 0.25}
    assert oracle.Net(COSINE + ir).lr_schedule == {"kind": 1, "warmup": 100, "total": 10000,
                                                   "min": float(np.float32(0.05))}
    for step in [0, 1, 50, 99, 100, 101, 777, 5050, 9999, 10000, 10001, 123456789]:
        assert L.nsh_plan_lr_scale(const.h, step) == 1.0
        assert np.float32(L.nsh_plan_lr_scale(cos.h, step)) == np.float32(oracle.lr_scale_cosine(step)), step
        assert np.float32(L.nsh_plan_lr_scale(other.h, step)) == np.float32(oracle.lr_scale(sched, step)), step
    assert abs(oracle.lr_scale(sched, 30) - (0.25 + 0.375 * (1 + np.cos(np.pi * 0.5)))) < 1e-6
    for bad in ("// ns.lr_schedule linear\n", "// ns.lr_schedule cosine_warmup warmup=x\n",
                "// ns.lr_schedule cosine_warmup steps=3\n"):
        with pytest.raises(runtime.NshipError):
            runtime.Plan(bad + ir)


@pytest.mark.parametrize("name", runtime.bundled_nets())
def test_plan_tables_match_the_reference(name):
    """Weight layout, blob size and output geometry as the reference driver
    computes them; checked against the independent Python parser, and
    against the reference build itself when present."""
    plan = runtime.Plan(helpers.ir_text(name))
    net = oracle.Net(helpers.ir_text(name))
    lay = plan.layout()
    assert [(n, o, c) for n, o, c in lay] == [(n, net.offsets[n], r * c) for n, r, c in net.weights]
    assert plan.weight_count == net.total
    assert (plan.in_cols, plan.out_cols) == (net.in_cols, net.out_cols)
    lib = runtime.net_lib(name)
    assert lib.weight_count_static() == net.total
    assert lib.layout() == lay
    for n in (0, 7, 4096):
        assert lib.output_numel(None, n) == net.output_numel(n)
    ref = os.path.join(helpers.REF, f"lib{name}.so")
    if os.path.exists(ref):
        R = NsLib(ref)
        assert R.layout() == lay and R.weight_count_static() == net.total
        for n in (0, 7, 4096):
            assert R.output_numel(None, n) == lib.output_numel(None, n)


def test_plan_rejects_unsupported_and_malformed_ir():
    bad = ["ns.func @F {\n  ns.tensor.alloc %w : Tensor[4, 4] float32\n  ns.softmax %a %x\n}\n",
           "ns.func @F {\n  ns.matmul %a %x\n}\n",
           "garbage"]
    for text in bad:
        with pytest.raises(runtime.NshipError):
            runtime.Plan(text)


def test_reference_build_drivers_load_when_present():
    ref = os.path.join(helpers.REF, "libc1.so")
    if not os.path.exists(ref):
        pytest.skip("reference build not present")
    assert NsLib(ref).weight_count_static() == 64 * 256 + 256 * 256 + 256 * 10


@pytest.mark.parametrize("name", ["c4k", "moet", "c4"])
def test_moe_plan_without_initial_experts_is_rejected(name):
    """The reference's own `nsc --mlir` printer drops MoE(initial_experts)
    (mlir_compiler.cpp:896-902); a plan without `initial=` would not know which
    experts start live, so it is refused instead of assuming all of them."""
    import re
    text = helpers.ir_text(name)
    plain = re.sub(r" initial=\d+", "", text)
    assert plain != text
    with pytest.raises(runtime.NshipError, match="initial"):
        runtime.Plan(plain)
    runtime.Plan(text)  # the attribute-preserving text parses


# Each op entry point with a null buffer that a nonempty call would touch:
# -1 and a message, decided before any device work (so it runs without a GPU).
NULL_CALLS = [
    ("nsh_op_embedding", (None, None, None, 4, 10, 8)),
    ("nsh_op_layernorm", (None, None, 4, 8)),
    ("nsh_op_layernorm_grad", (None, None, None, 4, 8)),
    ("nsh_op_softmax_xent", (None, None, None, None, None, 4, 8)),
    ("nsh_op_act_grad", (None, None, None, 16, 1)),
    ("nsh_op_embedding_grad", (None, None, None, 4, 10, 8, None)),
    ("nsh_op_adamw_step", (None, None, None, None, 16, 1, 0.01)),
    ("nsh_op_attention_fwd", (None, None, None, None, None, 16, 64, 1)),
    ("nsh_op_attention_bwd", (None,) * 9 + (16, 64, 1, 0, None)),
    ("nsh_op_orthonormalize", (None, None, 16, 8, None)),
    ("nsh_op_muon_step", (None, None, 16, 8, 0.01, None)),
    ("nsh_op_gemm", (None, None, None, 4, 4, 4, 4, 4, 4, 0, 0, 0)),
]


@pytest.mark.parametrize("name,args", NULL_CALLS, ids=[c[0] for c in NULL_CALLS])
def test_op_entry_points_reject_null_buffers(name, args):
    L = runtime.lib()
    assert getattr(L, name)(*args) == -1
    assert runtime.last_error(), f"{name}: no error message"


@pytest.mark.parametrize("name", ["nsh_op_embedding_grad", "nsh_op_embedding_grad_noalloc"])
@pytest.mark.parametrize("V,D", [(0, 8), (10, 0), (0, 0)])
def test_embedding_grad_of_an_empty_vocabulary_succeeds(name, V, D):
    """dW with no elements (V == 0 or D == 0): both entry points return 0
    without device work (so this runs without a GPU), the workspace one and
    the allocation-free one alike."""
    assert getattr(runtime.lib(), name)(None, None, None, 0, V, D, None) == 0
