"""Full-size c5 fixtures that make the optimizer observable (written by the
oracle, which is pinned bitwise to the reference's emitted drivers):

* c5_full_update.npz -- the reference network (Muon on all 8 matrices), ONE
  training step at lr 3e-4 from the seeded weights: per matrix the Frobenius
  norm of the update W1 - W0, each gradient vector's Gram-Schmidt residual
  ratio (the fraction of its norm left after projecting out the vectors
  before it; the leading vectors with ratio > 1e-3 form the determined
  prefix), 4096 sampled entries of Q = (W0 - W1 - 0.01 lr W0) / (lr
  sqrt(min(r, c))) on that prefix and 4096 sampled gradient entries; plus
  the step's loss; (float64) the same gradient entries and loss evaluated in
  float64 by oracle/f64.py, and the float64 MGS of the float64 gradient at
  the sampled Q entries; (mgs_own) the float64 MGS of the oracle's own
  gradient at the same entries.
* c5a_full.npz -- the AdamW variant (c5a: `optimizer=adamw` on the step, a
  build knob, not reference-emitted), 10 steps at lr 3e-4: the losses, the
  per-matrix norms of W10 - W0, 65536 sampled entries of W10 and its digest;
  and (adamw_sensitivity) the same 10 steps from 1-ulp-perturbed weights;
  (adamw_float64) the same 10 steps in float64 by oracle/f64.py.
* curve_c5sa_206.npz -- the AdamW variant at the reduced c5 shape, 100 steps
  under the host's cosine-warmup lr: losses, weights after 20 and 100 steps,
  and the trajectory's own spread under 1-ulp weight noise.

    OMP_NUM_THREADS=6 python tests/golden/make_c5_full_checks.py \
        [update|sensitivity|float64|mgs_own|adamw|adamw_sensitivity|adamw_float64|curve]
"""
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [ROOT, os.path.join(ROOT, "oracle"), os.path.join(ROOT, "tests")]

import helpers  # noqa: E402
import oracle  # noqa: E402
from golden.make_golden import digest  # noqa: E402
from neuralscript_amd import workloads  # noqa: E402

LR = 3e-4


def setup(name):
    ir = helpers.ir_text(name)
    net = oracle.Net(ir)
    layout = [(n, net.offsets[n], r * c) for n, r, c in net.weights]
    w = workloads.weights("c5", layout, workloads.ir_shapes(ir))
    return net, w, workloads.inputs("c5"), workloads.labels("c5")


def residual_ratios(G, r, c):
    """Per vector (rows when r < c, else columns), in order: the fraction of
    its norm that survives modified Gram-Schmidt against the vectors before
    it (float64).  Q_j's sensitivity to a relative change e of the gradient
    is about e / ratio_j."""
    vecs = (G.reshape(r, c) if r < c else G.reshape(r, c).T).astype(np.float64)
    Q = np.zeros_like(vecs)
    out = np.zeros(vecs.shape[0])
    for j, v in enumerate(vecs):
        res = v.copy()
        for i in range(j):
            res -= (Q[i] @ res) * Q[i]
        n = np.linalg.norm(res)
        out[j] = n / max(np.linalg.norm(v), 1e-300)
        Q[j] = res / n if n > 0 else 0.0
    return out


def determined_prefix(ratios, tau=1e-3):
    """Leading vectors whose residual keeps more than tau of their norm."""
    bad = np.flatnonzero(ratios <= tau)
    return int(bad[0]) if bad.size else ratios.size


def update_sensitivity():
    """Adds to c5_full_update.npz what the same step gives from weights
    perturbed by one ulp (random sign per element): the sampled Q entries,
    the sampled gradient entries and the loss.  At 16384 tokens the
    attention averages nearly identical rows that LayerNorm then rescales,
    so the reference's own gradients move far more than fp32 rounding under
    such noise; the GPU test holds its differences to a multiple of this
    movement where it exceeds the plain bar."""
    path = os.path.join(HERE, "c5_full_update.npz")
    with np.load(path) as f:
        out = {k: f[k] for k in f.files}
    net, w0, x, y = setup("c5")
    rng = np.random.default_rng(7)
    wp = (w0 * (1 + np.float32(2.0 ** -23) * rng.choice(np.array([-1, 1], np.float32), w0.size))).astype(np.float32)
    m = oracle.Model(net, wp)
    rec = {}
    t0 = time.time()
    out["loss_ulp"] = np.float32(m.train_step(x, y, LR, rec))
    print(f"c5 perturbed step: {time.time() - t0:.0f} s", flush=True)
    lr = np.float32(LR)
    for n_, r, c in net.weights:
        o = net.offsets[n_]
        a, b = wp[o:o + r * c].astype(np.float64), m.w[o:o + r * c].astype(np.float64)
        le = np.float64(lr) * np.sqrt(np.float32(min(r, c)))
        q = ((a - b) - 0.01 * np.float64(lr) * a) / le
        q = q.reshape(r, c) if r < c else q.reshape(r, c).T
        out[f"{n_}:q_ulp"] = q[out[f"{n_}:vi"], out[f"{n_}:ei"]]
        out[f"{n_}:g_ulp"] = rec["buf"][str(out[f"{n_}:grad"])][out[f"{n_}:gi"]].copy()
        print(f"  {n_}: max |dQ| under 1-ulp noise {np.max(np.abs(out[f'{n_}:q_ulp'] - out[f'{n_}:q'])):.3g}, "
              f"gradient max |d| / rms {np.max(np.abs(out[f'{n_}:g_ulp'] - out[f'{n_}:g'])) / out[f'{n_}:grms']:.3g}",
              flush=True)
    np.savez_compressed(path, **out)


def update():
    net, w0, x, y = setup("c5")
    m = oracle.Model(net, w0)
    rec = {}
    t0 = time.time()
    loss = m.train_step(x, y, LR, rec)
    print(f"c5 step: {time.time() - t0:.0f} s, loss {loss}", flush=True)
    grads = {}
    for ins in net.train.instrs:
        if ins.op == "ns.opt.step":
            grads = {ins.operands[k]: ins.operands[k + 1] for k in range(0, len(ins.operands) - 1, 2)}
    out = {"loss": np.float32(loss), "lr": np.float32(LR), "x_digest": np.array(digest(x)),
           "w_digest": np.array(digest(w0))}
    rng = np.random.default_rng(2024)
    lr = np.float32(LR)
    for n_, r, c in net.weights:
        o = net.offsets[n_]
        a, b = w0[o:o + r * c].astype(np.float64), m.w[o:o + r * c].astype(np.float64)
        le = np.float64(lr) * np.sqrt(np.float32(min(r, c)))
        q = ((a - b) - 0.01 * np.float64(lr) * a) / le
        q = q.reshape(r, c) if r < c else q.reshape(r, c).T  # one vector per row
        G = rec["buf"][grads[n_]]
        ratios = residual_ratios(G, r, c)
        k = determined_prefix(ratios)
        vi = rng.integers(0, k, 4096)
        ei = rng.integers(0, q.shape[1], 4096)
        gi = rng.integers(0, r * c, 4096)
        out[f"{n_}:norm"] = np.float64(np.linalg.norm(b - a))
        out[f"{n_}:k"] = np.int64(k)
        out[f"{n_}:ratio"] = ratios
        out[f"{n_}:vi"], out[f"{n_}:ei"], out[f"{n_}:q"] = vi, ei, q[vi, ei]
        out[f"{n_}:grad"] = np.array(grads[n_])
        out[f"{n_}:gi"], out[f"{n_}:g"] = gi, G[gi].copy()
        out[f"{n_}:grms"] = np.float64(np.sqrt(np.mean(G.astype(np.float64) ** 2)))
        print(f"  {n_} [{r}x{c}] determined {k}/{q.shape[0]} |dW| {out[f'{n_}:norm']:.6g} "
              f"ratios {np.round(ratios[:4], 4)} min over prefix {ratios[:k].min():.3g}", flush=True)
    np.savez_compressed(os.path.join(HERE, "c5_full_update.npz"), **out)


def float64():
    """Adds to c5_full_update.npz the float64 evaluation of the same step's
    gradients (oracle/f64.py: the reference's formulas in float64) at the
    sampled entries (`<matrix>:g64`) and the float64 loss (`loss64`): the
    yardstick against which the oracle's float32 rounding and the GPU's are
    both measured."""
    import f64
    path = os.path.join(HERE, "c5_full_update.npz")
    with np.load(path) as f:
        out = {k: f[k] for k in f.files}
    net, w0, x, y = setup("c5")
    t0 = time.time()
    vals, loss = f64.train_values(net, w0, x, y)
    print(f"c5 float64 step: {time.time() - t0:.0f} s, loss {loss!r} (float32 oracle {float(out['loss'])!r})",
          flush=True)
    out["loss64"] = np.float64(loss)
    for n_, r, c in net.weights:
        g64 = vals[str(out[f"{n_}:grad"])]
        out[f"{n_}:g64"] = g64[out[f"{n_}:gi"]].copy()
        out[f"{n_}:g64rms"] = np.float64(np.sqrt(np.mean(g64 ** 2)))
        # Q of the float64 gradient (MGS in float64) at the sampled entries,
        # and the float64 gradient's own residual ratios
        k = int(out[f"{n_}:k"])
        q64, ratio64 = helpers.mgs64(g64, r, c, k)
        out[f"{n_}:q64"] = q64[out[f"{n_}:vi"], out[f"{n_}:ei"]]
        out[f"{n_}:ratio64"] = ratio64
        d = np.abs(out[f"{n_}:g"].astype(np.float64) - out[f"{n_}:g64"])
        print(f"  {n_}: oracle vs float64 max |d| / rms {d.max() / out[f'{n_}:g64rms']:.3g}, "
              f"median {np.median(d) / out[f'{n_}:g64rms']:.3g}", flush=True)
    np.savez_compressed(path, **out)


def mgs_own():
    """Adds to c5_full_update.npz the float64 MGS of the oracle's own
    float32 gradients on their determined prefix, at the sampled entries
    (`<matrix>:q64own`): the yardstick of the reference's Q, against which
    the GPU test measures how far its own Q is from the float64 MGS of its
    own gradient."""
    path = os.path.join(HERE, "c5_full_update.npz")
    with np.load(path) as f:
        out = {k: f[k] for k in f.files}
    net, w0, x, y = setup("c5")
    rec = {}
    t0 = time.time()
    oracle.Model(net, w0).train_step(x, y, LR, rec)
    print(f"c5 step: {time.time() - t0:.0f} s", flush=True)
    for n_, r, c in net.weights:
        G = rec["buf"][str(out[f"{n_}:grad"])]
        assert np.array_equal(G[out[f"{n_}:gi"]], out[f"{n_}:g"]), "oracle drifted from the fixture"
        q64own, ratio = helpers.own_mgs(G, n_, r, c, out)
        out[f"{n_}:q64own"] = q64own
        d = out[f"{n_}:q"] - q64own
        print(f"  {n_}: reference Q vs float64 MGS of its gradient: rms {np.sqrt(np.mean(d ** 2)):.3g} "
              f"max {np.max(np.abs(d)):.3g}", flush=True)
    np.savez_compressed(path, **out)


def adamw(steps=10):
    net, w0, x, y = setup("c5a")
    m = oracle.Model(net, w0)
    losses = []
    for s in range(steps):
        t0 = time.time()
        losses.append(m.train_step(x, y, LR))
        print(f"c5a step {s}: loss {losses[-1]:.7f} ({time.time() - t0:.0f} s)", flush=True)
    rng = np.random.default_rng(2025)
    idx = np.sort(rng.choice(w0.size, 65536, replace=False))
    out = {"losses": np.array(losses, np.float32), "lr": np.float32(LR), "steps": np.int64(steps),
           "idx": idx, "w_sample": m.w[idx].copy(), "w_digest": np.array(digest(m.w)),
           "x_digest": np.array(digest(x)), "w0_digest": np.array(digest(w0))}
    for n_, r, c in net.weights:
        o = net.offsets[n_]
        out[f"{n_}:norm"] = np.float64(np.linalg.norm(m.w[o:o + r * c].astype(np.float64) - w0[o:o + r * c]))
    np.savez_compressed(os.path.join(HERE, "c5a_full.npz"), **out)



def adamw_float64():
    """Adds to c5a_full.npz the same 10 AdamW steps evaluated in float64
    (oracle/f64.py: gradients and updates by the reference's formulas) at
    the sampled weights (`w64_sample`) and its losses (`losses64`)."""
    import f64
    path = os.path.join(HERE, "c5a_full.npz")
    with np.load(path) as f:
        out = {k: f[k] for k in f.files}
    net, w0, x, y = setup("c5a")
    w = w0.astype(np.float64)
    state = {n_: (np.zeros(r * c), np.zeros(r * c)) for n_, r, c in net.weights}
    grads = {}
    for ins in net.train.instrs:
        if ins.op == "ns.opt.step":
            grads = {ins.operands[k]: ins.operands[k + 1] for k in range(0, len(ins.operands) - 1, 2)}
    losses = []
    for s in range(int(out["steps"])):
        t0 = time.time()
        vals, loss = f64.train_values(net, w, x, y)
        losses.append(loss)
        for n_, r, c in net.weights:
            o = net.offsets[n_]
            m, v = state[n_]
            f64.adamw_step(w[o:o + r * c], vals[grads[n_]], m, v, s + 1, float(out["lr"]))
        print(f"float64 c5a step {s}: loss {loss:.7f} ({time.time() - t0:.0f} s)", flush=True)
    out["losses64"] = np.array(losses, np.float64)
    out["w64_sample"] = w[out["idx"]].copy()
    np.savez_compressed(path, **out)


def adamw_sensitivity(seed=8):
    """Adds to c5a_full.npz the oracle's own 10 steps from the initial
    weights perturbed by one ulp (random sign per element): its losses
    (`ulp_losses`), the fraction of the sampled weights within the fp32 bar
    of the unperturbed run (`ulp_within`) and the largest deviation
    (`ulp_maxdev`) -- how far rounding alone moves this trajectory."""
    path = os.path.join(HERE, "c5a_full.npz")
    with np.load(path) as f:
        out = {k: f[k] for k in f.files}
    net, w0, x, y = setup("c5a")
    rng = np.random.default_rng(seed)
    wp = (w0 * (1 + np.float32(2.0 ** -23) * rng.choice(np.array([-1, 1], np.float32), w0.size))).astype(np.float32)
    m = oracle.Model(net, wp)
    losses = []
    for s in range(int(out["steps"])):
        t0 = time.time()
        losses.append(m.train_step(x, y, float(out["lr"])))
        print(f"perturbed c5a step {s}: {losses[-1]:.7f} ({time.time() - t0:.0f} s)", flush=True)
    ws = m.w[out["idx"]].astype(np.float64)
    wr = out["w_sample"].astype(np.float64)
    out["ulp_losses"] = np.array(losses, np.float32)
    out["ulp_within"] = np.float64(np.mean(np.abs(ws - wr) <= 1e-5 + 1e-4 * np.abs(wr)))
    out["ulp_maxdev"] = np.float64(np.max(np.abs(ws - wr)))
    np.savez_compressed(path, **out)


def adamw_curve(rows=256, seed=206, base=1e-3, trials=4):
    """curve_c5sa_206.npz: the AdamW variant at the reduced c5 shape (c5sa),
    100 steps under the host's cosine-warmup lr: the losses, the weights
    after 20 steps and after 100, and the trajectory's own sensitivity --
    the same steps from weights perturbed by one ulp (random sign per
    element), `trials` times: per-step loss spread, the weight spread after
    20 and after 100 steps.  AdamW turns a gradient element that cancels to
    ~0 into a +-lr step whose sign follows rounding; such flips stay rare for
    the first 20 steps here and have spread over most weights by step 100,
    while the loss curve stays within a few 1e-4."""
    from golden.make_golden import curve_lrs
    net = oracle.Net(helpers.ir_text("c5sa"))
    x = helpers.net_inputs(net, "c5sa", seed, rows)
    y = helpers.net_labels(net, seed, rows)
    w = helpers.net_weights("c5sa", seed, std=0.1)

    def run(w0):
        m = oracle.Model(net, w0)
        losses, w20 = [], None
        for t, lr in enumerate(curve_lrs(base)):
            losses.append(m.train_step(x, y, lr))
            if t + 1 == 20:
                w20 = m.w.copy()
        return np.array(losses, np.float32), w20, m.w.copy()

    losses, w20, w100 = run(w)
    band, s20, s100 = np.zeros(100), 0.0, 0.0
    for trial in range(trials):
        rng = np.random.default_rng(trial)
        wp = (w * (1 + np.float32(2.0 ** -23) * rng.choice(np.array([-1, 1], np.float32), w.size))).astype(np.float32)
        lp, p20, p100 = run(wp)
        band = np.maximum(band, np.abs(lp.astype(np.float64) - losses))
        s20 = max(s20, float(np.max(np.abs(p20.astype(np.float64) - w20))))
        s100 = max(s100, float(np.max(np.abs(p100.astype(np.float64) - w100))))
    np.savez_compressed(os.path.join(HERE, f"curve_c5sa_{seed}.npz"), losses=losses, w20=w20, w_final=w100,
                        x_digest=np.array(digest(x)), w_digest=np.array(digest(w)), base=np.float32(base),
                        rows=np.int64(rows), band=band, spread_w20=np.float64(s20), spread_w100=np.float64(s100))
    print("c5sa curve", losses[[0, 1, 50, 99]], f"1-ulp loss band {band.max():.3g}, weight spread after 20 "
          f"steps {s20:.3g}, after 100 {s100:.3g}", flush=True)

if __name__ == "__main__":
    what = sys.argv[1:] or ["update", "sensitivity", "float64", "mgs_own", "adamw", "adamw_sensitivity",
                            "adamw_float64", "curve"]
    for wname in what:
        {"update": update, "sensitivity": update_sensitivity, "float64": float64, "mgs_own": mgs_own,
         "adamw": adamw, "adamw_sensitivity": adamw_sensitivity, "adamw_float64": adamw_float64,
         "curve": adamw_curve}[wname]()
