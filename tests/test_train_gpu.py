"""AOT training through ns_runtime_train_step on the GPU against the
reference: per-step losses and trained weights (fixtures written by the
reference build), every gradient of a step against the oracle, the Muon
update on its determined part, the objective's purity, and 100-step loss
curves with the cosine warmup schedule applied by the host.

Loss tolerance.  Muon orthonormalises the gradient with modified
Gram-Schmidt and its +1e-30 guard turns the rounding residue of every
rank-deficient direction into a unit vector (LayerNorm outputs and
softmax-minus-one-hot rows sum to zero, small batches have low rank), so the
reference's own trajectory moves under a mere change of summation order.
Each fixture records that movement (`band`: the largest deviation of the
reference restatement with its MGS dot products summed in ten other orders:
2..8 interleaved partial sums, 2, 4 or 8 contiguous blocks,
tests/golden/make_band.py); a loss at step t must
be within 1e-3 + 2 * max(band[:t+1]) of the reference.  AdamW-only
networks have band 0, i.e. plain 1e-3, and their weights are compared too."""
import os

import numpy as np
import pytest

import helpers
import oracle
from golden.make_golden import CASES, CURVES, case_inputs, curve_lrs
from neuralscript_amd import runtime

pytestmark = pytest.mark.gpu

TRAIN = [c for c in CASES if c[3]]
LOSS_TOL = 1e-3


def loss_tol(band):
    return LOSS_TOL + 2.0 * np.maximum.accumulate(np.asarray(band, np.float64))


def golden(name):
    return np.load(os.path.join(helpers.GOLDEN, f"{name}.npz"))


@pytest.mark.parametrize("case", TRAIN, ids=lambda c: c[0])
def test_train_steps_match_reference_fixture(case):
    name, rows, seed, steps, lr, _ = case
    print(f"train {name} rows={rows} steps={steps}", flush=True)
    net, x, y = case_inputs(name, rows, seed)
    lib = runtime.net_lib(name)
    m = lib.init(helpers.net_weights(name, seed))
    g = golden(name)
    losses = np.array([lib.train_step(m, x, y, lr) for _ in range(steps)], dtype=np.float32)
    tol = loss_tol(g["band"])
    print(f"  losses {losses} reference {g['losses']} tolerance {tol}")
    assert np.all(np.abs(losses - g["losses"]) <= tol), (losses, g["losses"], tol)
    # the first loss is a pure forward: fp32 tolerance
    helpers.assert_close(losses[:1], g["losses"][:1], f"{name} first loss")
    obj = lib.objective_loss(m, x, y)
    assert abs(obj - g["objective"]) <= tol[-1] + 2.0 * np.max(g["band"])
    if not np.any(g["band"]):  # no Muon matrix: weights and outputs are determined
        print(f"  trained weights violation x{helpers.violation(lib.get_weights(m), g['w_final']):.3g}, forward "
              f"after x{helpers.violation(lib.eval_infer(m, x)[: g['out_after'].size], g['out_after']):.3g}")
        helpers.assert_close(lib.get_weights(m), g["w_final"], f"{name} trained weights")
        helpers.assert_close(lib.eval_infer(m, x)[: g["out_after"].size], g["out_after"], f"{name} forward after")
    lib.free(m)


@pytest.mark.parametrize("name", ["mlpt", "c5s", "moet", "moeb", "drp", "c5a"])
def test_train_step_on_an_empty_batch(name):
    """Zero rows: the reference's loss is 0/0 (NaN) and every gradient an
    empty sum, so the optimizer step applies only its decay terms (Muon of a
    zero matrix gives Q = 0; AdamW of g = 0 moves nothing but the decay)."""
    print(f"empty train step {name}", flush=True)
    net = oracle.Net(helpers.ir_text(name))
    w = helpers.net_weights(name, 3)
    lib = runtime.net_lib(name)
    m = lib.init(w)
    om = oracle.Model(net, w)
    empty = np.zeros(0, np.float32)
    loss = lib.train_step(m, empty, empty, 0.02)
    ref = om.train_step(empty, empty, 0.02)
    assert np.isnan(loss) and np.isnan(ref), (loss, ref)
    got = lib.get_weights(m)
    print(f"  weights bit-identical to the oracle's: {helpers.bitwise_equal(got, om.w)}")
    helpers.assert_close(got, np.asarray(om.w, np.float32), f"{name} weights after an empty step")
    lib.free(m)


def test_objective_does_not_mutate_weights():
    name, rows, seed = "c5t", 33, 108
    net, x, y = case_inputs(name, rows, seed)
    lib = runtime.net_lib(name)
    m = lib.init(helpers.net_weights(name, seed))
    lib.train_step(m, x, y, 0.01)
    w0 = lib.get_weights(m)
    lib.objective_loss(m, x, y)
    lib.objective_loss(m, x, y)
    assert helpers.bitwise_equal(lib.get_weights(m), w0)
    lib.free(m)


def test_adamw_training_matches_oracle_step_by_step():
    """AdamW network (xor): after every step the weights stay within the
    fp32 bar (1e-5 + 1e-4 |ref|) of the oracle's (no drift accumulation)."""
    name, rows, seed = "xor", 4, 103
    net, x, y = case_inputs(name, rows, seed)
    w = helpers.net_weights(name, seed)
    om = oracle.Model(net, w)
    lib = runtime.net_lib(name)
    m = lib.init(w)
    for step in range(8):
        lg = lib.train_step(m, x, y, 0.3)
        lo = om.train_step(x, y, 0.3)
        assert abs(lg - lo) <= 1e-5 + 1e-4 * abs(lo), (step, lg, lo)
        print(f"  xor step {step}: violation x{helpers.violation(lib.get_weights(m), om.w):.3g}")
        helpers.assert_close(lib.get_weights(m), om.w, f"xor step {step}")
    lib.free(m)


@pytest.mark.parametrize("curve", CURVES, ids=lambda c: f"{c[0]}-{c[2]}")
def test_100_step_loss_curve_matches_reference(curve):
    name, rows, seed, base = curve
    print(f"curve {name} tokens={rows} lr={base}", flush=True)
    g = np.load(os.path.join(helpers.GOLDEN, f"curve_{name}_{seed}.npz"))
    net = oracle.Net(helpers.ir_text(name))
    x = helpers.net_inputs(net, name, seed, rows)
    y = helpers.net_labels(net, seed, rows)
    lib = runtime.net_lib(name)
    m = lib.init(helpers.net_weights(name, seed, std=0.1))
    losses = np.array([lib.train_step(m, x, y, lr) for lr in curve_lrs(base)], dtype=np.float32)
    lib.free(m)
    dev = np.abs(losses - g["losses"])
    tol = loss_tol(g["band"])
    print(f"  max |loss - reference| = {dev.max():.3g} at step {int(dev.argmax())}; "
          f"reordering band max {g['band'].max():.3g}; worst ratio to tolerance {np.max(dev / tol):.3g}")
    assert np.all(dev <= tol), (dev, tol)


@pytest.mark.parametrize("name,rows", [("c5t", 40), ("mlpt", 17), ("c5s", 64), ("c5s", 2048), ("c5h", 192),
                                       ("c5h", 100), ("moet", 41), ("moet", 300), ("moeb", 4096),
                                       ("smt", 64), ("drp", 64), ("drp", 29), ("c5w", 400), ("c5w", 130),
                                       ("embw", 40), ("embw", 400), ("embw", 3000)])
def test_every_value_of_one_train_step_matches_oracle(name, rows):
    """Each intermediate and gradient of one training step (read back from
    the device by IR value name) against the oracle's value of the same
    name; the weights after the optimizer last.

    A value passes at the north star's bar, |d| <= 1e-5 + 1e-4 |ref|, or,
    where the network amplifies rounding beyond it, by being at least half
    as accurate as the reference itself against the same formulas evaluated
    in float64 (oracle/f64.py; violations at the same bar): at 2048 tokens
    the attention output is an average over 2048 rows (rms 0.025) that
    LayerNorm rescales by ~40, so the reference's own float32 logits sit
    beyond the bar from the float64 ones.  Networks with operations the
    float64 evaluation does not cover (softmax, dropout, MoE) fall back to
    4x the movement that a random 1-ulp perturbation of the weights causes
    in the reference, measured at the same bar.  embw (a 4096-row
    embedding) at 40 and 400 tokens runs its Muon MGS on the gradient's
    live rows only (compacted vectors); at 3000 tokens at full length."""
    ir = helpers.ir_text(name)
    net = oracle.Net(ir)
    seed = 400 + rows
    x = helpers.net_inputs(net, name, seed, rows)
    y = helpers.net_labels(net, seed, rows)
    w = helpers.net_weights(name, seed)
    om = oracle.Model(net, w)
    rec = {}
    om.train_step(x, y, 0.02, rec)
    rng = np.random.default_rng(seed)
    wp = (w * (1 + np.float32(2.0 ** -23) * rng.choice(np.array([-1, 1], np.float32), w.size))).astype(np.float32)
    rec_p = {}
    oracle.Model(net, wp).train_step(x, y, 0.02, rec_p)
    import f64
    try:
        vals64, _ = f64.train_values(net, w, x, y)
    except NotImplementedError:
        vals64 = None
    model = runtime.Model(runtime.Plan(ir), w)
    model.train_step(x, y, 0.02)
    bad = []
    # a MATMUL_GRAD_A result whose only use is an ACTIVATION_GRAD is folded
    # into that GEMM's epilogue and never stored; the activation gradient
    # computed from it is checked instead
    uses = {}
    for ins in net.train.instrs:
        for o in ins.operands:
            uses[o] = uses.get(o, 0) + 1
    folded = {i.operands[0] for i in net.train.instrs
              if i.op == "ns.grad.activation" and "dropout_mask" not in i.comment and uses.get(i.operands[0]) == 1}
    for ins in net.train.instrs:
        v = ins.result
        if v is None or v not in rec["buf"] or ins.op in ("ns.cross_entropy",):
            continue
        if ins.op == "ns.grad.matmul.a" and v in folded:
            print(f"  {ins.op:24s} {v:8s} folded into its activation gradient's GEMM epilogue")
            continue
        ref = rec["buf"][v]
        got = model.read_value(v, ref.size)
        viol = helpers.violation(got, ref)
        if vals64 is not None and v in vals64:
            # at least half as accurate as the reference against float64
            v64, o64 = helpers.violation(got, vals64[v]), helpers.violation(ref, vals64[v])
            print(f"  {ins.op:24s} {v:8s} n={ref.size:7d} violation x{viol:.3g}; vs float64 x{v64:.3g} "
                  f"(the reference x{o64:.3g})")
            if viol > 1.0 and v64 > max(1.0, 2.0 * o64):
                bad.append((ins.op, v, viol, v64, o64))
            continue
        floor = helpers.violation(rec_p["buf"][v], ref)
        print(f"  {ins.op:24s} {v:8s} n={ref.size:7d} violation x{viol:.3g} (1-ulp weight noise: x{floor:.3g})")
        if viol > max(1.0, 4.0 * floor):
            bad.append((ins.op, v, viol, floor))
    # Weights after the optimizer.  AdamW: the whole update.  Muon: the update
    # is lr*sqrt(min(r,c))*Q + 0.01*lr*W with Q = MGS(grad); only the Q
    # vectors of the determined prefix (rank of the gradient's vector set)
    # are implementation-independent, the rest normalise rounding residue.
    grads = {}
    for ins in net.train.instrs:
        if ins.op == "ns.opt.step":
            grads = {ins.operands[k]: ins.operands[k + 1] for k in range(0, len(ins.operands) - 1, 2)}
    lr = np.float32(0.02)
    for n_, r, c in net.weights:
        o = net.offsets[n_]
        w0, wg, wo = w[o:o + r * c], model.read_value(n_, r * c), om.w[o:o + r * c]
        if not oracle.use_muon(r, c):
            v = helpers.violation(wg, wo)
            print(f"  weight {n_} [{r}x{c}] AdamW violation x{v:.3g}")
            assert v <= 1, n_
            continue
        le = np.float64(lr) * np.sqrt(np.float32(min(r, c)))
        decay = 0.01 * np.float64(lr)
        qg = ((w0.astype(np.float64) - wg) - decay * w0) / le
        qo = ((w0.astype(np.float64) - wo) - decay * w0) / le
        G = rec["buf"][grads[n_]].reshape(r, c).astype(np.float64)
        vecs = G if r < c else G.T           # one vector per row of `vecs`
        qg = qg.reshape(r, c) if r < c else qg.reshape(r, c).T
        qo = qo.reshape(r, c) if r < c else qo.reshape(r, c).T
        # determined prefix: vectors whose Gram-Schmidt residual keeps > 1e-3
        # of their norm, in order
        basis, k = [], 0
        for vj in vecs:
            res = vj.copy()
            for b in basis:
                res -= (b @ res) * b
            if np.linalg.norm(res) <= 1e-3 * max(np.linalg.norm(vj), 1e-30):
                break
            basis.append(res / np.linalg.norm(res))
            k += 1
        d = np.max(np.abs(qg[:k] - qo[:k])) if k else 0.0
        print(f"  weight {n_} [{r}x{c}] Muon: determined vectors {k}/{vecs.shape[0]}, max |dQ| {d:.3g}")
        assert d <= 2e-3, n_
    assert not bad, bad
    model.free()


def test_c5_full_size_100_step_loss_curve():
    """Config c5 at full size (one 16384-token sequence, vocab 8192, Muon on
    every matrix): 100 device-resident training steps with the host's cosine
    warmup lr (3e-4 x lr_scale(t)) against the oracle's curve, which is
    bit-identical to the reference's emitted driver (written by
    tests/golden/make_c5_curve.py): every loss within 1e-3, the first (a pure
    forward) within fp32 tolerance."""
    from golden.make_golden import digest
    from neuralscript_amd import workloads
    print("c5 full-size curve: 100 steps", flush=True)
    g = np.load(os.path.join(helpers.GOLDEN, "curve_c5_full.npz"))
    assert int(g["steps_done"]) == 100
    plan = runtime.Plan.load("c5")
    w = workloads.weights("c5", plan.layout(), workloads.ir_shapes(plan.ir))
    x, y = workloads.inputs("c5"), workloads.labels("c5")
    assert digest(x) == str(g["x_digest"]) and digest(w) == str(g["w_digest"]), "input generator drifted"
    model = runtime.Model(plan, w)
    dx, dy = runtime.DeviceArray.from_host(x), runtime.DeviceArray.from_host(y)
    losses = np.array([model.train_step_device(dx, dy, lr) for lr in curve_lrs(3e-4, 100)], dtype=np.float32)
    model.free()
    dev = np.abs(losses.astype(np.float64) - g["losses"])
    print(f"  max |loss - reference| = {dev.max():.3g} at step {int(dev.argmax())}; "
          f"losses {losses[0]:.6f} .. {losses[-1]:.6f}")
    helpers.assert_close(losses[:1], g["losses"][:1], "c5 first loss")
    assert np.all(dev <= LOSS_TOL), dev


def test_adamw_variant_100_step_curve_and_weights():
    """The AdamW variant of c5 (c5sa: c5's network at the reduced shape with
    `optimizer=adamw` on its step -- a build knob of this backend, not
    something the reference emits; AdamW rule codegen.cpp:3108-3119, pinned
    bit for bit by the AdamW fixtures) over 100 steps of the host's
    cosine-warmup lr (base 1e-3): every loss within plain 1e-3 on a curve
    that falls from 6.43 to 5.20, the weights after 20 steps within the fp32
    bar.  AdamW has a band of its own: a gradient element that cancels to ~0
    becomes a +-lr step whose sign follows rounding, and the oracle started
    from 1-ulp-perturbed weights ends 100 steps up to 0.053 away in some
    weights (loss within 2.3e-4, weights after 20 steps within 6.4e-7); the
    final weights are held to twice that measured spread."""
    g = np.load(os.path.join(helpers.GOLDEN, "curve_c5sa_206.npz"))
    from golden.make_golden import digest
    name, rows, seed = "c5sa", int(g["rows"]), 206
    net = oracle.Net(helpers.ir_text(name))
    x = helpers.net_inputs(net, name, seed, rows)
    y = helpers.net_labels(net, seed, rows)
    w = helpers.net_weights(name, seed, std=0.1)
    assert digest(x) == str(g["x_digest"]) and digest(w) == str(g["w_digest"]), "input generator drifted"
    lib = runtime.net_lib(name)
    m = lib.init(w)
    losses, w20 = [], None
    for t, lr in enumerate(curve_lrs(float(g["base"]))):
        losses.append(lib.train_step(m, x, y, lr))
        if t + 1 == 20:
            w20 = lib.get_weights(m)
    losses = np.array(losses, dtype=np.float32)
    wf = lib.get_weights(m)
    lib.free(m)
    dev = np.abs(losses.astype(np.float64) - g["losses"])
    d100 = float(np.max(np.abs(wf.astype(np.float64) - g["w_final"])))
    print(f"  losses {losses[0]:.4f} .. {losses[-1]:.4f}; max |loss - oracle| {dev.max():.3g} at step "
          f"{int(dev.argmax())} (1-ulp band {g['band'].max():.3g}); weights after 20 steps violation "
          f"x{helpers.violation(w20, g['w20']):.3g}; after 100 max |dw| {d100:.3g} (1-ulp spread "
          f"{float(g['spread_w100']):.3g})")
    assert np.all(dev <= LOSS_TOL), dev
    helpers.assert_close(w20, g["w20"], "c5sa weights after 20 AdamW steps")
    assert d100 <= 2.0 * float(g["spread_w100"]), d100


def _c5_full(name):
    from golden.make_golden import digest
    from neuralscript_amd import workloads
    plan = runtime.Plan.load(name)
    net = oracle.Net(plan.ir)
    w = workloads.weights("c5", plan.layout(), workloads.ir_shapes(plan.ir))
    x, y = workloads.inputs("c5"), workloads.labels("c5")
    return plan, net, w, x, y, digest


def test_c5_full_size_first_muon_update_matches_oracle():
    """Config c5 at full size, one training step at lr 3e-4 from the seeded
    weights.  At 16384 tokens the forward is ill-conditioned (the attention
    averages nearly identical rows that LayerNorm rescales), so the
    reference's own float32 gradients are off by up to a few % of their rms
    from the same formulas evaluated in float64 (tests/golden/
    make_c5_full_checks.py float64; oracle/f64.py).  Against those float64
    values every one of the eight sampled gradients must be at least as
    accurate as the reference's (rms and max error, and a least-squares
    scale error within max(2e-4, the reference's): a gradient scaled by
    1.001 fails, test_full_size_gradient_check_rejects_scaled_and_broken_
    gradients).  The update: its Frobenius norm within 1e-3 of the oracle's
    (lr * min(r, c) for any summation order, so a no-op optimizer, a doubled
    lr or a wrong sqrt(min(r, c)) factor fail) and Q, on the vectors that
    keep >= 5% of their norm in Gram-Schmidt, at least as close (rms, max)
    to the float64 MGS of the GPU's own gradient as the reference's Q is to
    the float64 MGS of the reference's gradient.  The step's loss (a pure
    forward) within the fp32 bar of the oracle's."""
    g = np.load(os.path.join(helpers.GOLDEN, "c5_full_update.npz"))
    plan, net, w, x, y, digest = _c5_full("c5")
    assert digest(x) == str(g["x_digest"]) and digest(w) == str(g["w_digest"]), "input generator drifted"
    print("c5 full size: one step", flush=True)
    model = runtime.Model(plan, w)
    dx, dy = runtime.DeviceArray.from_host(x), runtime.DeviceArray.from_host(y)
    loss = model.train_step_device(dx, dy, float(g["lr"]))
    w1 = model.get_weights()
    full = {n: model.read_value(str(g[n + ":grad"]), r * c) for n, r, c in net.weights}
    model.free()
    grads = {n: full[n][g[n + ":gi"]] for n in full}
    own = {n: helpers.own_mgs(full[n], n, r, c, g) for n, r, c in net.weights}
    stats = helpers.muon_update_stats(w, w1, float(g["lr"]), net.weights, net.offsets, g)
    fails = helpers.muon_update_failures(stats, g, own) + helpers.full_gradient_failures(grads, g)
    print(f"  loss {loss:.7f} (oracle {float(g['loss']):.7f}, float64 {float(g['loss64']):.7f})")
    for name, (norm, q) in stats.items():
        a = helpers.accuracy_vs_f64(grads[name], g[name + ":g64"])
        o = helpers.accuracy_vs_f64(g[name + ":g"], g[name + ":g64"])
        b_rms, b_max = helpers.muon_q_bounds(g, name)
        sel = own[name][1] >= helpers.MUON_Q_RATIO
        dq = np.asarray(q, np.float64)[sel] - own[name][0][sel]
        print(f"  {name}: gradient vs float64 rms {a['rms']:.3g} max {a['max']:.3g} scale {a['scale']:+.2g} "
              f"(reference rms {o['rms']:.3g} max {o['max']:.3g} scale {o['scale']:+.2g}); |dW| {norm:.6g} "
              f"(oracle {float(g[name + ':norm']):.6g}); Q vs float64 MGS of its gradient on {int(sel.sum())} "
              f"samples rms {np.sqrt(np.mean(dq ** 2)):.3g} max {np.max(np.abs(dq)):.3g} (bounds {b_rms:.3g}, "
              f"{b_max:.3g}); vs the float64 gradient's MGS max {np.max(np.abs(q - g[name + ':q64'])[sel]):.3g}")
    helpers.assert_close(np.float32(loss), g["loss"], "c5 first loss")
    assert not fails, fails


def test_c5_full_size_adamw_variant_ten_steps():
    """c5a (c5 with `optimizer=adamw`, a build knob, not reference-emitted)
    at full size: 10 steps at lr 3e-4 against the oracle -- every loss within
    plain 1e-3 (the curve falls 0.21 over the 10 steps, so a no-op optimizer
    or a doubled lr fails), the per-matrix norm of W10 - W0 within 2%, and
    the 65536 sampled weights at least as accurate as the reference's against
    the same 10 steps evaluated in float64 (oracle/f64.py; helpers.
    adamw_f64_failures): as large a fraction within the fp32 bar and no
    larger an rms distance.  AdamW turns a gradient element that cancels to
    ~0 into a +-lr step whose sign follows rounding, and at this sequence
    length the gradients themselves are ill-conditioned (see the
    first-update test): the reference's own float32 run keeps only ~77% of
    the samples within the bar of the float64 one, while a wrong step size
    leaves only the weights whose 10-step update is itself below the bar:
    11% for no step or a doubled lr, 15% for lr x 1.1 (checked here as
    `noop`)."""
    g = np.load(os.path.join(helpers.GOLDEN, "c5a_full.npz"))
    plan, net, w, x, y, digest = _c5_full("c5a")
    assert digest(x) == str(g["x_digest"]) and digest(w) == str(g["w0_digest"]), "input generator drifted"
    print("c5a full size: 10 AdamW steps", flush=True)
    model = runtime.Model(plan, w)
    dx, dy = runtime.DeviceArray.from_host(x), runtime.DeviceArray.from_host(y)
    losses = np.array([model.train_step_device(dx, dy, float(g["lr"])) for _ in range(int(g["steps"]))], np.float32)
    w10 = model.get_weights()
    model.free()
    dev = np.abs(losses.astype(np.float64) - g["losses"])
    ws, wr = w10[g["idx"]].astype(np.float64), g["w_sample"].astype(np.float64)
    within = float(np.mean(np.abs(ws - wr) <= 1e-5 + 1e-4 * np.abs(wr)))
    noop = float(np.mean(np.abs(w[g["idx"]].astype(np.float64) - wr) <= 1e-5 + 1e-4 * np.abs(wr)))
    a64, o64 = helpers.adamw_f64_stats(ws, g), helpers.adamw_f64_stats(wr, g)
    print(f"  losses {losses[0]:.6f} .. {losses[-1]:.6f}; max |loss - oracle| {dev.max():.3g}; sampled weights "
          f"within the fp32 bar of the oracle's: {100 * within:.2f}% (no optimizer step {100 * noop:.2f}%), "
          f"max |d| {np.max(np.abs(ws - wr)):.3g}; against the float64 trajectory: within the bar "
          f"{100 * a64['within']:.2f}%, rms |d| {a64['rms']:.3g} (the reference: {100 * o64['within']:.2f}%, "
          f"{o64['rms']:.3g})")
    fails = helpers.adamw_f64_failures(ws, g)
    norms = []
    for name, r, c in net.weights:
        o = net.offsets[name]
        n = float(np.linalg.norm(w10[o:o + r * c].astype(np.float64) - w[o:o + r * c]))
        norms.append((name, n, float(g[name + ":norm"])))
    print("  |W10 - W0| vs oracle:", [(a, round(b / c, 5)) for a, b, c in norms])
    assert np.all(dev <= LOSS_TOL), dev
    assert noop < 0.2, noop
    assert not fails, fails
    for name, n, ref in norms:
        assert abs(n - ref) <= 0.02 * ref, (name, n, ref)
