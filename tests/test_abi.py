"""CPU checks of the drop-in boundary: the libraries load, export every
symbol the headers declare, and the plan parser reproduces the reference's
static tables (no device calls)."""
import ctypes
import os
import re

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
    missing = [s for s in want if not hasattr(lib.lib, s)]
    assert not missing, missing


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
