"""Attention core (flash forward) against the oracle's exact-softmax
attention, and the c3 network."""
import numpy as np
import pytest

import helpers
import oracle
from neuralscript_amd import runtime, synth, workloads
from neuralscript_amd.runtime import DeviceArray as DA

pytestmark = pytest.mark.gpu


def core_ref(Q, K, V, S, D, H):
    """The attention core (scores, softmax, P V) in float64; the layer-level
    tests below compare against the oracle's bit-faithful restatement."""
    dk = D // H
    out = np.zeros((S, D))
    Qd, Kd, Vd = (a.reshape(S, D).astype(np.float64) for a in (Q, K, V))
    for h in range(H):
        sl = slice(h * dk, (h + 1) * dk)
        s = Qd[:, sl] @ Kd[:, sl].T * (1.0 / np.sqrt(np.float32(dk)))
        p = np.exp(s - s.max(1, keepdims=True))
        out[:, sl] = (p / p.sum(1, keepdims=True)) @ Vd[:, sl]
    return out


# Head sizes: 64 and 32 and 128 in place; 8, 16, 48, 80, 96, 7 (rows not
# 16-byte aligned) on copies padded with zero columns to 32, 64 or 128.
SHAPES_FWD = [(1, 64, 1), (100, 128, 2), (333, 64, 1), (1024, 1024, 16), (300, 64, 2), (257, 16, 2), (90, 64, 8),
              (2048, 512, 8), (100, 128, 1), (77, 192, 2), (2048, 1024, 8), (333, 256, 2), (300, 96, 2),
              (257, 64, 4), (130, 160, 2), (77, 21, 3), (64, 128, 4)]


@pytest.mark.parametrize("S,D,H", SHAPES_FWD)
def test_attention_core_matches_float64(S, D, H):
    print(f"attention core S={S} D={D} H={H}", flush=True)
    Q, K, V = (synth.normal(S * 10 + i, S * D, 1.0) for i in range(3))
    ctx, lse = DA(S * D), DA(S * H)
    runtime.op("attention_fwd", DA.from_host(Q), DA.from_host(K), DA.from_host(V), ctx, lse, S, D, H)
    helpers.assert_close(ctx.to_host(), core_ref(Q, K, V, S, D, H).ravel(), f"attention S={S} D={D} H={H}")


def core_bwd_ref(Q, K, V, dO, S, D, H):
    """Gradient of the attention core in float64: per head, with P the
    softmax of the scaled scores, dV = P^T dO, dS = P o (dO V^T - rowsum(dO o O)),
    dQ = scale dS K, dK = scale dS^T Q."""
    dk = D // H
    sc = 1.0 / np.sqrt(np.float32(dk))
    Qd, Kd, Vd, dOd = (a.reshape(S, D).astype(np.float64) for a in (Q, K, V, dO))
    dQ, dK, dV = np.zeros((S, D)), np.zeros((S, D)), np.zeros((S, D))
    for h in range(H):
        sl = slice(h * dk, (h + 1) * dk)
        s = Qd[:, sl] @ Kd[:, sl].T * sc
        p = np.exp(s - s.max(1, keepdims=True))
        p /= p.sum(1, keepdims=True)
        o = p @ Vd[:, sl]
        dV[:, sl] = p.T @ dOd[:, sl]
        ds = p * (dOd[:, sl] @ Vd[:, sl].T - (dOd[:, sl] * o).sum(1, keepdims=True))
        dQ[:, sl] = ds @ Kd[:, sl] * sc
        dK[:, sl] = ds.T @ Qd[:, sl] * sc
    return dQ, dK, dV


@pytest.mark.parametrize("S,D,H", [(64, 128, 2), (128, 128, 2), (192, 128, 2), (100, 128, 2), (256, 64, 2),
                                   (130, 64, 2), (90, 64, 8), (1024, 512, 8), (2048, 512, 8), (100, 128, 1),
                                   (77, 192, 2), (2048, 1024, 8), (333, 256, 2), (320, 256, 2), (300, 96, 2),
                                   (257, 64, 4), (130, 160, 2), (77, 21, 3)])
@pytest.mark.parametrize("store_ds", [0, 1])
def test_attention_core_backward_matches_float64(S, D, H, store_ds):
    """Flash backward (key-parallel dK/dV pass, then dQ either from the
    stored dS or from a query-parallel pass recomputing S and dP) at head
    sizes 32, 64, 128 in place and the others padded, vs the float64
    gradient at the fp32 bar |d| <= 1e-5 + 1e-4 |ref|."""
    print(f"attention backward S={S} D={D} H={H} store_ds={store_ds}", flush=True)
    Q, K, V, dO = (synth.normal(S * 20 + i, S * D, 1.0) for i in range(4))
    dQ_, dK_, dV_ = (DA(S * D) for _ in range(3))
    gQ, gK, gV, gdO = (DA.from_host(a) for a in (Q, K, V, dO))
    ctx, lse = DA(S * D), DA(S * H)
    runtime.op("attention_fwd", gQ, gK, gV, ctx, lse, S, D, H)
    nb = runtime.lib().nsh_op_attention_bwd_workspace(S, D, H, store_ds)
    ws = DA(max(1, (nb + 3) // 4))
    runtime.op("attention_bwd", gQ, gK, gV, ctx, gdO, lse, dQ_, dK_, dV_, S, D, H, store_ds, ws)
    for name, got, ref in zip(("dQ", "dK", "dV"), (dQ_, dK_, dV_), core_bwd_ref(Q, K, V, dO, S, D, H)):
        ref = ref.ravel()
        print(f"  {name}: violation at the plain bar x{helpers.violation(got.to_host(), ref):.3g}, "
              f"max|ref| {float(np.abs(ref).max()):.3g}")
        helpers.assert_close(got.to_host(), ref, f"attention {name} S={S} D={D} H={H} ds={store_ds}")


# Head sizes above 128 (160, 256, 129 with rows not 16-byte aligned, 300
# with an odd sequence length): scores materialised per block of query rows
# and multiplied out by the GEMM kernels.  rows: query rows per block
# (NSHIP_ATTN_WIDE_ROWS; None = the whole sequence in one block).  Score
# rows held in registers at 4, 8 and 16 floats per thread (S up to 4096,
# 8192, 16384 and a multiple of 4), streamed three times otherwise (S = 257,
# 130).
WIDE = [(64, 320, 2, None), (64, 1024, 4, None), (100, 387, 3, None), (257, 600, 2, None), (1000, 1536, 6, None),
        (300, 512, 2, 64), (257, 600, 2, 100), (130, 320, 2, 1), (6000, 160, 1, None), (9000, 136, 1, 3000)]


@pytest.mark.parametrize("S,D,H,rows", WIDE)
def test_wide_head_attention_matches_float64(S, D, H, rows, monkeypatch):
    """Forward and backward at head sizes above 128 vs float64, at the fp32
    bar; lse as the flash kernels define it."""
    if rows:
        monkeypatch.setenv("NSHIP_ATTN_WIDE_ROWS", str(rows))
    print(f"wide attention S={S} D={D} H={H} rows={rows}", flush=True)
    Q, K, V, dO = (synth.normal(S * 30 + i, S * D, 1.0) for i in range(4))
    gQ, gK, gV, gdO = (DA.from_host(a) for a in (Q, K, V, dO))
    ctx, lse = DA(S * D), DA(S * H)
    runtime.op("attention_fwd", gQ, gK, gV, ctx, lse, S, D, H)
    helpers.assert_close(ctx.to_host(), core_ref(Q, K, V, S, D, H).ravel(), f"wide attention S={S} D={D} H={H}")
    dk = D // H
    Qd, Kd = Q.reshape(S, D).astype(np.float64), K.reshape(S, D).astype(np.float64)
    lref = np.empty((H, S))
    for h in range(H):
        sl = slice(h * dk, (h + 1) * dk)
        sc = Qd[:, sl] @ Kd[:, sl].T * (1.0 / np.sqrt(np.float32(dk)))
        m = sc.max(1)
        lref[h] = (m + np.log(np.exp(sc - m[:, None]).sum(1))) / np.log(2.0)
    helpers.assert_close(lse.to_host(), lref.ravel(), "wide attention lse")
    dQ_, dK_, dV_ = (DA(S * D) for _ in range(3))
    nb = runtime.lib().nsh_op_attention_bwd_workspace(S, D, H, 1)
    ws = DA(max(1, (nb + 3) // 4))
    runtime.op("attention_bwd", gQ, gK, gV, ctx, gdO, lse, dQ_, dK_, dV_, S, D, H, 1, ws)
    for name, got, ref in zip(("dQ", "dK", "dV"), (dQ_, dK_, dV_), core_bwd_ref(Q, K, V, dO, S, D, H)):
        helpers.assert_close(got.to_host(), ref.ravel(), f"wide attention {name} S={S} D={D} H={H} rows={rows}")


def test_attention_layer_matches_oracle():
    """Whole layer x -> (QKV projections, core, output projection) through a
    network driver vs the oracle's ns_attention_fwd restatement."""
    from golden.make_golden import case_inputs
    g = np.load(f"{helpers.GOLDEN}/c3s.npz")
    _, x, _ = case_inputs("c3s", 45, 105)
    lib = runtime.net_lib("c3s")
    m = lib.init(helpers.net_weights("c3s", 105))
    out = lib.eval_infer(m, x)
    lib.free(m)
    helpers.assert_close(out, g["out"], "c3s forward vs reference fixture")


@pytest.mark.parametrize("rows", [700, 1500])
def test_c3_small_sequence_matches_oracle(rows):
    ir = helpers.ir_text("c3s")
    w = helpers.net_weights("c3s", rows, std=0.1)
    net = oracle.Net(ir)
    x = helpers.net_inputs(net, "c3s", rows, rows)
    ref = oracle.Model(net, w).eval_infer(x)
    lib = runtime.net_lib("c3s")
    m = lib.init(w)
    out = lib.eval_infer(m, x)
    lib.free(m)
    helpers.assert_close(out, ref, f"c3s S={rows}")


def test_c3_full_size_rows_match_oracle():
    """Config 3 at full size: 16384 ids as one sequence, d_model 1024, 16
    heads; the oracle recomputes 24 query rows (full K/V) and their LN."""
    print("c3 full size", flush=True)
    ir = helpers.ir_text("c3")
    plan = runtime.Plan(ir)
    shapes = workloads.ir_shapes(ir)
    w = workloads.weights("c3", plan.layout(), shapes)
    x = workloads.inputs("c3")
    lib = runtime.net_lib("c3")
    m = lib.init(w)
    out = lib.eval_infer(m, x).reshape(16384, 1024)
    lib.free(m)
    assert np.isfinite(out).all()
    net = oracle.Net(ir)
    o = net.offsets
    emb = oracle.embedding(w[: 32000 * 1024], x, 32000, 1024)
    Wq, Wk, Wv, Wo = (w[o[n]: o[n] + 1024 * 1024] for n in ("attn_q_w", "attn_k_w", "attn_v_w", "attn_o_w"))
    rows = np.unique(np.linspace(0, 16383, 24).astype(np.int64))
    att = oracle.attention_fwd_rows(emb, Wq, Wk, Wv, Wo, rows, 16384, 1024, 16)
    ref = oracle.layernorm(att, 1024).reshape(len(rows), 1024)
    helpers.assert_close(out[rows], ref, "c3 rows")


@pytest.mark.parametrize("rows", [2048, 333])
def test_c3_with_head_size_128_matches_oracle(rows):
    """c3d (c3's network with Attention(1024, 8): head size 128, the flash
    kernels' DK = 128 instantiation) against the oracle at 2048 and 333
    tokens, all rows."""
    print(f"c3d S={rows}", flush=True)
    ir = helpers.ir_text("c3d")
    w = helpers.net_weights("c3d", rows, std=0.1)
    net = oracle.Net(ir)
    x = helpers.net_inputs(net, "c3d", rows, rows)
    ref = oracle.Model(net, w).eval_infer(x)
    lib = runtime.net_lib("c3d")
    m = lib.init(w)
    out = lib.eval_infer(m, x)
    lib.free(m)
    helpers.assert_close(out, ref, f"c3d S={rows}")


def test_c3d_full_size_rows_match_oracle():
    """c3d at c3's full size (16384 tokens as one sequence, 8 heads of 128):
    24 query rows recomputed by the oracle (full K/V) and their LN."""
    print("c3d full size", flush=True)
    ir = helpers.ir_text("c3d")
    plan = runtime.Plan(ir)
    w = workloads.weights("c3d", plan.layout(), workloads.ir_shapes(ir))
    x = workloads.inputs("c3d")
    lib = runtime.net_lib("c3d")
    m = lib.init(w)
    out = lib.eval_infer(m, x).reshape(16384, 1024)
    lib.free(m)
    assert np.isfinite(out).all()
    net = oracle.Net(ir)
    o = net.offsets
    emb = oracle.embedding(w[: 32000 * 1024], x, 32000, 1024)
    Wq, Wk, Wv, Wo = (w[o[n]: o[n] + 1024 * 1024] for n in ("attn_q_w", "attn_k_w", "attn_v_w", "attn_o_w"))
    rows = np.unique(np.linspace(0, 16383, 24).astype(np.int64))
    att = oracle.attention_fwd_rows(emb, Wq, Wk, Wv, Wo, rows, 16384, 1024, 8)
    ref = oracle.layernorm(att, 1024).reshape(len(rows), 1024)
    helpers.assert_close(out[rows], ref, "c3d rows")
