"""Add the reordering drift band to the training fixtures of tests/golden.

For every fixture that holds a loss trajectory, rerun the same training with
the oracle set to sum each modified-Gram-Schmidt dot product in another
order -- P interleaved partial sums (P = 2..8) or P contiguous blocks
(P = 2, 4, 8); otherwise identical to the reference -- and store `band` =
max over these orders of |losses_P - losses|.
Muon normalises the rounding noise of rank-deficient gradient directions
(ns_orthonom's +1e-30 guard), so the reference's own trajectory moves this
much under a mere change of summation order; a GPU implementation is held to
1e-3 plus a small multiple of this band.

    python tests/golden/make_band.py [net ...]    (default: every net)
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [ROOT, os.path.join(ROOT, "oracle"), os.path.join(ROOT, "tests")]

import helpers  # noqa: E402
import oracle  # noqa: E402
from golden.make_golden import CASES, CURVES, case_inputs, curve_lrs  # noqa: E402


def update(path, **extra):
    d = dict(np.load(path))
    d.update(extra)
    np.savez_compressed(path, **d)


PARTIALS = (2, 3, 4, 5, 6, 7, 8, -2, -4, -8)


def spread(run, ref):
    out = np.zeros_like(ref)
    for p in PARTIALS:
        oracle.set_mgs_partials(p)
        out = np.maximum(out, np.abs(run() - ref))
    oracle.set_mgs_partials(1)
    return out


def main(names=()):
    for name, rows, seed, steps, lr, _ in CASES:
        if not steps or (names and name not in names):
            continue
        net, x, y = case_inputs(name, rows, seed)

        def run():
            m = oracle.Model(net, helpers.net_weights(name, seed))
            return np.array([m.train_step(x, y, lr) for _ in range(steps)], np.float32)

        path = os.path.join(HERE, f"{name}.npz")
        band = spread(run, np.load(path)["losses"])
        update(path, band=band)
        print(name, "band", band)
    for name, rows, seed, base in CURVES:
        if names and name not in names:
            continue
        net = oracle.Net(helpers.ir_text(name))
        x = helpers.net_inputs(net, name, seed, rows)
        y = helpers.net_labels(net, seed, rows)

        def run():
            m = oracle.Model(net, helpers.net_weights(name, seed, std=0.1))
            return np.array([m.train_step(x, y, lr) for lr in curve_lrs(base)], np.float32)

        path = os.path.join(HERE, f"curve_{name}_{seed}.npz")
        band = spread(run, np.load(path)["losses"])
        update(path, band=band)
        print(name, seed, "max band", band.max())


if __name__ == "__main__":
    main(sys.argv[1:])
