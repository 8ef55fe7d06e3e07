"""Top-1 MoE forward: router logits and expert choices bit-exact with the
oracle (exact and near gate-logit ties reported), outputs within tolerance,
liveness mask and the expert lifecycle against the reference fixtures, and
config 4 at full size.

The routing probability p = exp(l_best - max) / sum is an fp32 value and is
held to the fp32 tolerance: the device evaluates exp correctly rounded,
glibc's expf (the reference's) is off by one ulp on ~0.009% of inputs, so p
can differ in its last bit for a fraction of a percent of tokens."""
import os

import numpy as np
import pytest

import helpers
import oracle
from golden.make_golden import CASES, case_inputs
from neuralscript_amd import runtime, workloads

pytestmark = pytest.mark.gpu


def tie_report(logits, E):
    """(exact ties, near ties < 1e-6 relative) between the top-2 logits."""
    lg = logits.reshape(-1, E).astype(np.float64)
    top2 = np.sort(lg, axis=1)[:, -2:]
    gap = top2[:, 1] - top2[:, 0]
    exact = int((gap == 0).sum())
    near = int(((gap > 0) & (gap <= 1e-6 * np.maximum(1.0, np.abs(top2[:, 1])))).sum())
    return exact, near


@pytest.mark.parametrize("name", ["c4s", "c4k"])
def test_moe_forward_matches_reference_fixture(name):
    case = next(c for c in CASES if c[0] == name)
    net, x, _ = case_inputs(name, case[1], case[2])
    w = helpers.net_weights(name, case[2])
    lib = runtime.net_lib(name)
    m = lib.init(w)
    out = lib.eval_infer(m, x)
    g = np.load(os.path.join(helpers.GOLDEN, f"{name}.npz"))
    helpers.assert_close(out[: g["out"].size], g["out"], f"{name} forward")
    lib.free(m)


def test_moe_lifecycle_matches_reference_fixture():
    name = "c4k"
    case = next(c for c in CASES if c[0] == name)
    net, x, _ = case_inputs(name, case[1], case[2])
    lib = runtime.net_lib(name)
    m = lib.init(helpers.net_weights(name, case[2]))
    g = np.load(os.path.join(helpers.GOLDEN, f"{name}.npz"))
    assert lib.lib.ns_expert_count(m) == 4
    counts = [lib.lib.ns_expert_birth(m, 1)]
    o1 = lib.eval_infer(m, x)[: g["out"].size]
    counts.append(lib.lib.ns_expert_merge(m, 0, 1))
    o2 = lib.eval_infer(m, x)[: g["out"].size]
    counts.append(lib.lib.ns_expert_kill(m, 2))
    o3 = lib.eval_infer(m, x)[: g["out"].size]
    assert counts == list(g["life_counts"])
    assert helpers.bitwise_equal(lib.get_weights(m), g["life_w"])  # host-side edits are exact
    for o, ref in zip((o1, o2, o3), g["life_outs"]):
        helpers.assert_close(o, ref, "lifecycle forward")
    # invalid arguments leave the count unchanged
    assert lib.lib.ns_expert_kill(m, 99) == counts[-1]
    assert lib.lib.ns_expert_merge(m, 0, 0) == counts[-1]
    lib.free(m)


@pytest.mark.parametrize("M,D,E,H,mask", [(1000, 64, 8, 96, None), (3000, 128, 64, 64, None),
                                          (777, 64, 16, 32, "some"), (513, 32, 130, 16, None),
                                          (600, 32, 256, 16, "some"), (400, 32, 300, 8, "some"),
                                          (300, 16, 1000, 4, None), (700, 16, 5000, 2, "some")])
def test_moe_routing_is_bit_exact(M, D, E, H, mask):
    print(f"moe routing M={M} D={D} E={E} H={H}", flush=True)
    ir = ("ns.func @MOE {\n"
          f"  ns.tensor.alloc %moe_g_w : Tensor[{D}, {E}] float32\n"
          f"  ns.tensor.alloc %moe_e1_w : Tensor[{E}, {D * H}] float32\n"
          f"  ns.tensor.alloc %moe_e2_w : Tensor[{E}, {H * D}] float32\n"
          f"  ns.layer.moe %moe0 %x %moe_g_w %moe_e1_w %moe_e2_w : Tensor[Dynamic, {D}] float32 "
          f"// moe(x, experts={E}, ffn={H}) initial={E // 2 if mask else E}\n"
          "  ns.return %moe0\n}\n")
    plan = runtime.Plan(ir)
    from neuralscript_amd import synth
    Wg = synth.normal(M + 1, D * E, float(1 / np.sqrt(D)))
    We1 = synth.normal(M + 2, E * D * H, 0.05)
    We2 = synth.normal(M + 3, E * H * D, 0.05)
    w = np.concatenate([Wg, We1, We2])
    x = synth.normal(M + 4, M * D)
    model = runtime.Model(plan, w)
    out = model.eval_infer(x)[: M * D]
    best, prob, lg = model.last_routing(M, E)
    active = None
    if mask:
        active = np.zeros(E, np.uint8)
        active[: E // 2] = 1
    rbest, rprob, rlg = oracle.moe_route(x, Wg, active, M, D, E, want_logits=True)
    exact, near = tie_report(rlg, E)
    print(f"  exact gate-logit ties {exact}, near ties {near}")
    assert helpers.bitwise_equal(lg, rlg), "router logits differ"
    assert np.array_equal(best, rbest), f"expert choice differs at {np.flatnonzero(best != rbest)[:10]}"
    print(f"  p differs in the last bit for {int((prob != rprob).sum())} of {M} tokens")
    helpers.assert_close(prob, rprob, "routing probability")
    ref, _, _ = oracle.moe_fwd(x, Wg, We1, We2, active, M, D, H, E)
    helpers.assert_close(out, ref, "moe output")
    model.free()


def test_c4_full_size():
    """Config 4: 65536 tokens, d_model 1024, 64 experts (FFN 1024), Zipf gate
    prior.  Every expert choice and probability is compared bit-exactly; the
    outputs of 128 tokens (spread, plus the first tokens of each expert) are
    recomputed by the oracle."""
    print("c4 full size", flush=True)
    ir = helpers.ir_text("c4")
    plan = runtime.Plan(ir)
    shapes = workloads.ir_shapes(ir)
    w = workloads.weights("c4", plan.layout(), shapes)
    x = workloads.inputs("c4")
    M, D, E, H = 65536, 1024, 64, 1024
    model = runtime.Model(plan, w)
    out = model.eval_infer(x)[: M * D].reshape(M, D)
    best, prob, lg = model.last_routing(M, E)
    model.free()
    Wg = w[: D * E]
    rbest, rprob, rlg = oracle.moe_route(x, Wg, None, M, D, E, want_logits=True)
    exact, near = tie_report(rlg, E)
    hist = np.bincount(rbest, minlength=E)
    print(f"  expert histogram (first 8) {hist[:8].tolist()} max {hist.max()} min {hist.min()}; "
          f"exact ties {exact}, near ties {near}")
    assert helpers.bitwise_equal(lg, rlg)
    assert np.array_equal(best, rbest)
    print(f"  p differs in the last bit for {int((prob != rprob).sum())} of {M} tokens")
    helpers.assert_close(prob, rprob, "routing probability")
    rows = np.unique(np.concatenate([np.linspace(0, M - 1, 96).astype(np.int64),
                                     [np.flatnonzero(rbest == e)[0] for e in range(0, E, 2) if (rbest == e).any()]]))
    ref, _, _ = oracle.moe_fwd(x.reshape(M, D)[rows].ravel(), Wg, w[D * E: D * E + E * D * H],
                               w[D * E + E * D * H:], None, len(rows), D, H, E)
    helpers.assert_close(out[rows], ref.reshape(len(rows), D), "c4 rows")


def test_lifecycle_after_training_keeps_trained_weights():
    """Kill / merge / birth after device training act on the trained weights.

    Kill only flips the liveness mask (codegen.cpp:2619-2626): the trained
    weights read back before and after it are identical, and the forward
    afterwards equals the oracle's with those weights and that mask.  Merge
    and birth edit the trained blob (the host copy is refreshed from the
    device first), so their results equal the same edits replayed by the
    oracle's restatement on the trained weights."""
    name, rows, seed = "moet", 41, 109
    net, x, y = case_inputs(name, rows, seed)
    lib = runtime.net_lib(name)
    m = lib.init(helpers.net_weights(name, seed))
    for _ in range(3):
        lib.train_step(m, x, y, 0.01)
    w_trained = lib.get_weights(m)
    om = oracle.Model(net, w_trained)
    live = np.flatnonzero(om.active)
    assert len(live) >= 3
    k = int(live[-1])
    assert lib.lib.ns_expert_kill(m, k) == len(live) - 1
    assert helpers.bitwise_equal(lib.get_weights(m), w_trained), "kill changed the trained weights"
    om.active[k] = 0
    helpers.assert_close(lib.eval_infer(m, x), om.eval_infer(x), "forward after kill")
    # merge: averages expert a and b into a (host-side edit of the trained blob)
    a, b = int(live[0]), int(live[1])
    assert lib.lib.ns_expert_merge(m, a, b) == len(live) - 2
    om.expert_merge(a, b)
    assert helpers.bitwise_equal(lib.get_weights(m), om.w), "merge did not act on the trained weights"
    helpers.assert_close(lib.eval_infer(m, x), om.eval_infer(x), "forward after merge")
    # birth: a live expert (drawn from the model's mt19937) copied with noise
    # into the first dead slot
    assert lib.lib.ns_expert_birth(m, 1) == om.expert_birth(1) == len(live) - 1
    assert helpers.bitwise_equal(lib.get_weights(m), om.w), "birth did not act on the trained weights"
    helpers.assert_close(lib.eval_infer(m, x), om.eval_infer(x), "forward after birth")
    # training continues from the edited state
    l_dev = lib.train_step(m, x, y, 0.01)
    l_ref = om.train_step(x, y, 0.01)
    assert abs(l_dev - l_ref) <= 1e-5 + 1e-4 * abs(l_ref), (l_dev, l_ref)
    lib.free(m)


def test_moe_forward_with_every_expert_killed():
    """ns_expert_kill may take the live count to zero (codegen.cpp:2590-2626).
    The reference's forward then routes every token to expert -1 and reads
    outside its weights (no defined result); this backend outputs zeros and
    reports best = -1, and a later birth makes the layer route again."""
    name = "c4k"
    case = next(c for c in CASES if c[0] == name)
    net, x, _ = case_inputs(name, case[1], case[2])
    lib = runtime.net_lib(name)
    w = helpers.net_weights(name, case[2])
    m = lib.init(w)
    om = oracle.Model(net, w)
    for k in range(net.moe["E"]):
        n = lib.lib.ns_expert_kill(m, k)
        om.expert_kill(k)
    assert n == 0
    # the forward writes M x D floats (x's size); output_numel's F3 quirk
    # sizes the host buffer larger
    out = lib.eval_infer(m, x)[: x.size]
    assert np.all(out == 0.0), "no live expert: the MoE output must be zero"
    # birth finds no live source within its tries and copies the last drawn
    # slot (codegen.cpp:2565-2590), as the oracle restates
    assert lib.lib.ns_expert_birth(m, 1) == om.expert_birth(1) == 1
    assert helpers.bitwise_equal(lib.get_weights(m), om.w), "birth from no live expert"
    ref = om.eval_infer(x)
    helpers.assert_close(lib.eval_infer(m, x)[: ref.size], ref, "forward after the birth")
    lib.free(m)


def test_moe_checkpoint_tail_matches_reference(tmp_path):
    """NSM2 with the MoE tail (codegen.cpp:2501-2557) on c4k after birth,
    merge and kill: the saved file is byte-identical to the reference
    driver's; loading it restores weights and liveness; an NSM1 file loads
    with every capacity slot alive (as the reference's load does); a file
    with a wrong layer count, capacity or a short mask returns -1 and leaves
    the model as it was."""
    import hashlib
    name = "c4k"
    case = next(c for c in CASES if c[0] == name)
    net, x, _ = case_inputs(name, case[1], case[2])
    w = helpers.net_weights(name, case[2])
    g = np.load(os.path.join(helpers.GOLDEN, f"{name}.npz"))
    n_out = g["out"].size
    lib = runtime.net_lib(name)
    m = lib.init(w)
    lib.lib.ns_expert_birth(m, 1)
    lib.lib.ns_expert_merge(m, 0, 1)
    lib.lib.ns_expert_kill(m, 2)
    path = str(tmp_path / "life.nsm")
    assert lib.save(m, path) == 0
    with open(path, "rb") as f:
        raw = f.read()
    assert raw[12 + 4 * w.size:] == g["ckpt_tail"].tobytes()
    assert hashlib.sha256(raw).hexdigest() == str(g["ckpt_digest"]), "checkpoint bytes differ from the reference's"
    lib.free(m)

    m2 = lib.init(w)
    assert lib.load(m2, path) == 0
    assert lib.lib.ns_expert_count(m2) == int(g["life_counts"][-1])
    assert helpers.bitwise_equal(lib.get_weights(m2), g["life_w"])
    helpers.assert_close(lib.eval_infer(m2, x)[:n_out], g["life_outs"][-1], "forward after load")

    nsm1 = str(tmp_path / "w.nsm1")
    with open(nsm1, "wb") as f:
        f.write(np.uint32(0x4E534D31).tobytes() + np.uint64(w.size).tobytes() + w.tobytes())
    assert lib.load(m2, nsm1) == 0
    assert lib.lib.ns_expert_count(m2) == int(g["nsm1_count"]) == net.moe["E"]
    assert helpers.bitwise_equal(lib.get_weights(m2), w)
    helpers.assert_close(lib.eval_infer(m2, x)[:n_out], g["nsm1_out"], "forward after NSM1 load")

    # back to the lifecycle state, then every malformed tail is rejected
    assert lib.load(m2, path) == 0
    before = lib.eval_infer(m2, x)[:n_out]
    E = net.moe["E"]
    head = raw[: 12 + 4 * w.size]
    mask = raw[-E:]
    bad = {"cap+1": head + np.uint32(1).tobytes() + np.uint64(E + 1).tobytes() + mask + b"\x01",
           "cap-1": head + np.uint32(1).tobytes() + np.uint64(E - 1).tobytes() + mask[:-1],
           "layers=2": head + np.uint32(2).tobytes() + np.uint64(E).tobytes() + mask,
           "short mask": head + np.uint32(1).tobytes() + np.uint64(E).tobytes() + mask[:-1],
           "no tail": head}
    w_other = (w * np.float32(2)).astype(np.float32)
    for label, body in bad.items():
        # the blob in the bad file differs, so a partial load would show
        body = body[:12] + w_other.tobytes() + body[12 + 4 * w.size:]
        p = str(tmp_path / f"bad_{label.replace(' ', '_')}.nsm")
        with open(p, "wb") as f:
            f.write(body)
        assert lib.load(m2, p) == -1, label
        assert lib.lib.ns_expert_count(m2) == int(g["life_counts"][-1]), label
        assert helpers.bitwise_equal(lib.get_weights(m2), g["life_w"]), label
        assert helpers.bitwise_equal(lib.eval_infer(m2, x)[:n_out], before), label
    lib.free(m2)


def test_moe_backward_at_production_shape():
    """The four MoE gradients (codegen.cpp:1388-1579) at config 4's expert
    shape -- d_model 1024, 64 experts, FFN 1024 -- over 4096 tokens with
    Zipf-skewed routing (the embedding's last column is 1 and the router's
    last row carries log Zipf(1.1) priors, as config 4 folds its gate bias):
    every element of dx, dWg, dWe1 and dWe2 against the oracle.  One
    training step of the `moep` network (embedding -> MoE -> fc -> CE) at
    lr 0; the oracle skips its optimizer (only the gradients are compared).

    Bar: the fp32 one with its absolute term scaled to the tensor
    (|d| <= 1e-5 rms(ref) + 1e-4 |ref|; these gradients are ~1e-5 in size),
    or, where the reference itself is that sensitive (a dx element is a sum
    over 1024 + 64 terms that can cancel), at least the reference's own
    accuracy against the same formulas evaluated in float64 (oracle/f64.py,
    the reference's expert choices): rms and max error no larger than the
    reference's, scale error within max(2e-4, the reference's)."""
    name, M = "moep", 4096
    ir = helpers.ir_text(name)
    net = oracle.Net(ir)
    D, E, H = 1024, 64, 1024
    w, x, y = workloads.moe_training_workload(M)
    assert w.size == net.total
    Wg = w[8192 * D: 8192 * D + D * E]
    print(f"moe backward D={D} E={E} H={H} tokens={M}", flush=True)

    def oracle_run(weights):
        om = oracle.Model(net, weights)
        om._opt_step = lambda *a, **k: None
        rec = {}
        om.train_step(x, y, 0.0, rec)
        return rec

    rec = oracle_run(w)
    ref_buf = rec["buf"]
    rng = np.random.default_rng(5)
    wp = (w * (1 + np.float32(2.0 ** -23) * rng.choice(np.array([-1, 1], np.float32), w.size))).astype(np.float32)
    pert_buf = oracle_run(wp)["buf"]
    import f64
    vals64, _ = f64.train_values(net, w, x, y, moe_best=rec["moe_best"])
    best, _, lg = oracle.moe_route(ref_buf["emb3"], Wg, None, M, D, E, want_logits=True)
    hist = np.bincount(best, minlength=E)
    exact, near = tie_report(lg, E)
    print(f"  routing: busiest expert {hist.max()} tokens, {int((hist > 0).sum())} experts used, "
          f"rarest used {hist[hist > 0].min()}; exact ties {exact}, near ties {near}")
    model = runtime.Model(runtime.Plan(ir), w)
    model.train_step(x, y, 0.0)
    bad = []
    for ins in net.train.instrs:
        if not ins.op.startswith("ns.grad.moe."):
            continue
        ref = ref_buf[ins.result]
        got = model.read_value(ins.result, ref.size)
        atol = 1e-5 * float(np.sqrt(np.mean(ref.astype(np.float64) ** 2)))
        viol = helpers.violation(got, ref, atol=atol, rtol=1e-4)
        floor = helpers.violation(pert_buf[ins.result], ref, atol=atol, rtol=1e-4)
        a = helpers.accuracy_vs_f64(got, vals64[ins.result])
        o = helpers.accuracy_vs_f64(ref, vals64[ins.result])
        f64_fails = helpers.f64_accuracy_failures(got, ref, vals64[ins.result], ins.op)
        print(f"  {ins.op:18s} n={ref.size:9d} violation x{viol:.3g} (1-ulp weight noise: x{floor:.3g}); "
              f"vs float64: rms {a['rms']:.3g} max {a['max']:.3g} scale {a['scale']:+.2g} (reference rms "
              f"{o['rms']:.3g} max {o['max']:.3g} scale {o['scale']:+.2g})")
        if not np.all(np.isfinite(got)) or (viol > 1.0 and f64_fails):
            bad.append((ins.op, viol, f64_fails))
    model.free()
    assert not bad, bad


@pytest.mark.parametrize("E,rows", [(300, 300), (1000, 257), (6000, 700)])
def test_moe_training_step_with_many_experts(E, rows):
    """More than 256 experts (the router's logits by expert tiles, routing
    from them, the dispatch scan's tables in dynamic LDS -- in the ints
    workspace above 4096 experts --, the backward's routing probabilities
    per lane): moet's network with E experts (three quarters live), one
    training step against the oracle -- expert choices bit-exact, every MoE
    gradient and the loss at the fp32 bar."""
    print(f"moe training E={E} rows={rows}", flush=True)
    ir = (helpers.ir_text("moet").replace("Tensor[32, 8]", f"Tensor[32, {E}]")
          .replace("Tensor[8, 1536]", f"Tensor[{E}, 1536]").replace("experts=8", f"experts={E}")
          .replace("initial=6", f"initial={3 * E // 4}"))
    net = oracle.Net(ir)
    assert net.moe["E"] == E and net.moe["K0"] == 3 * E // 4
    seed = 700 + E
    x = helpers.net_inputs(net, "moet", seed, rows)
    y = helpers.net_labels(net, seed, rows)
    w = helpers.net_weights_for(net, seed)
    om = oracle.Model(net, w)
    rec = {}
    ref_loss = om.train_step(x, y, 0.02, rec)
    model = runtime.Model(runtime.Plan(ir), w)
    loss = model.train_step(x, y, 0.02)
    best, _, _ = model.last_routing(rows, E)
    assert np.array_equal(best, rec["moe_best"]), "expert choice differs"
    helpers.assert_close(np.float32(loss), ref_loss, "loss")
    for ins in net.train.instrs:
        if ins.op.startswith("ns.grad.moe."):
            ref = rec["buf"][ins.result]
            helpers.assert_close(model.read_value(ins.result, ref.size), ref, f"{ins.op} E={E}")
    model.free()


def test_expert_gradients_after_a_step_that_routed_elsewhere():
    """The expert weight gradients of an expert without tokens are zeros,
    written only when that expert's slices may hold something (a per-expert
    flag kept with the gradient buffers).  A step on a 3-token batch right
    after a step on 64 tokens that used other experts must give exactly the
    gradients of the same 3-token step on a fresh model (lr 0: the weights do
    not move), the stale slices of the first step's experts cleared."""
    name = "moet"
    print(f"moe gradients after rerouting ({name})", flush=True)
    ir = helpers.ir_text(name)
    net = oracle.Net(ir)
    E = net.moe["E"]
    w = helpers.net_weights_for(net, 811)
    xa, ya = helpers.net_inputs(net, name, 812, 64), helpers.net_labels(net, 812, 64)
    xb, yb = helpers.net_inputs(net, name, 813, 3), helpers.net_labels(net, 813, 3)
    plan = runtime.Plan(ir)
    grads = [i.result for i in net.train.instrs if i.op.startswith("ns.grad.moe.")]
    sizes = {i.result: i for i in net.train.instrs if i.op.startswith("ns.grad.moe.")}
    om = oracle.Model(net, w)
    om._opt_step = lambda *a, **k: None
    rec = {}
    om.train_step(xb, yb, 0.0, rec)
    m1 = runtime.Model(plan, w)
    m1.train_step(xa, ya, 0.0)
    used_a = set(m1.last_routing(64, E)[0].tolist())
    m1.train_step(xb, yb, 0.0)
    used_b = set(m1.last_routing(3, E)[0].tolist())
    assert used_a - used_b, "the first batch must use experts the second does not"
    m2 = runtime.Model(plan, w)
    m2.train_step(xb, yb, 0.0)
    try:
        for g in grads:
            n = rec["buf"][g].size
            a, b = m1.read_value(g, n), m2.read_value(g, n)
            assert helpers.bitwise_equal(a, b), f"{sizes[g].op} after rerouting differs from a fresh model's"
            helpers.assert_close(a, rec["buf"][g], sizes[g].op)
    finally:
        m1.free()
        m2.free()
