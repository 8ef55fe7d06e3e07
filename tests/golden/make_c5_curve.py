"""Full-size config-5 loss curve for the parity test (tests/golden/curve_c5_full.npz).

100 ns_runtime_train_step calls of the c5 network (emb 8192x512 -> attention
512/8 -> LayerNorm -> MLP 512-2048-512 ReLU -> fc 8192, CE) on one sequence of
32x512 = 16384 tokens, lr = 3e-4 * cosine-warmup multiplier applied by the
host, computed by the oracle restatement (bit-identical to the reference's
emitted CPU driver, tests/test_oracle.py pins it), because the reference's
own single-threaded driver would need hours per step at this size.
Run in the build container (about 5 h on 6 cores):
    OMP_NUM_THREADS=6 python tests/golden/make_c5_curve.py
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
from neuralscript_amd import workloads  # noqa: E402
from golden.make_golden import curve_lrs, digest  # noqa: E402

STEPS = 100
BASE_LR = 3e-4


def main():
    ir = helpers.ir_text("c5")
    net = oracle.Net(ir)
    shapes = workloads.ir_shapes(ir)
    lay = [(n, net.offsets[n], r * c) for n, r, c in net.weights]
    w = workloads.weights("c5", lay, shapes)
    x = workloads.inputs("c5")
    y = workloads.labels("c5")
    m = oracle.Model(net, w)
    out = os.path.join(HERE, "curve_c5_full.npz")
    losses = []
    for t, lr in enumerate(curve_lrs(BASE_LR, STEPS)):
        t0 = time.time()
        losses.append(m.train_step(x, y, lr))
        print(f"step {t} lr {lr:.3e} loss {losses[-1]:.7f} ({time.time() - t0:.1f} s)", flush=True)
        np.savez_compressed(out, losses=np.array(losses, np.float32), x_digest=np.array(digest(x)),
                            w_digest=np.array(digest(w)), steps_done=np.array(len(losses)))


if __name__ == "__main__":
    main()
