"""Write the golden fixtures of tests/golden/*.npz from the REFERENCE itself.

Each case runs a network driver emitted by the reference compiler
(`nsc <net>.ns --cpp --runtime`, compiled by oracle/Makefile into
oracle/_ref/lib<net>.so exactly as the reference tests compile it) through
its C-ABI on seeded inputs, and stores what it returned: the forward output,
and for training cases the per-step losses, the objective loss and the final
weight blob.  Inputs are not stored; they are regenerated from the seeds
(SplitMix64, neuralscript_amd/synth.py) and checked against a stored digest.

Run in the build container (needs /root/reference built by oracle/Makefile):
    python tests/golden/make_golden.py [net ...]    (default: every net)
then tests/golden/make_band.py, which adds the reordering band to the
training fixtures.
"""
import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [ROOT, os.path.join(ROOT, "oracle"), os.path.join(ROOT, "tests")]

import helpers  # noqa: E402
import oracle  # noqa: E402
from neuralscript_amd.abi import NsLib, _fp  # noqa: E402

XOR_X = np.array([0, 0, 0, 1, 1, 0, 1, 1], dtype=np.float32)
XOR_Y = np.array([1, 0, 0, 1, 0, 1, 1, 0], dtype=np.float32)

# name, rows, seed, train steps, lr, lifecycle
CASES = [
    ("c1", 64, 101, 0, 0.0, False),
    ("c2s", 29, 102, 0, 0.0, False),
    ("xor", 4, 103, 6, 0.3, False),
    ("mlpt", 17, 104, 3, 0.01, False),
    ("c3s", 45, 105, 0, 0.0, False),
    ("c4s", 50, 106, 0, 0.0, False),
    ("c4k", 40, 107, 0, 0.0, True),
    ("c5t", 33, 108, 3, 0.01, False),
    ("moet", 41, 109, 3, 0.01, False),
    ("c5s", 64, 110, 2, 0.003, False),
    ("moeb", 300, 111, 3, 0.01, False),
    ("dmv", 37, 112, 0, 0.0, False),
    ("dmw", 29, 113, 0, 0.0, False),
    ("bop", 41, 114, 0, 0.0, False),
    ("dmx", 23, 115, 0, 0.0, False),
    ("smt", 33, 116, 3, 0.05, False),
    ("drp", 37, 117, 4, 0.05, False),
    ("c5w", 400, 118, 2, 0.003, False),
]


def case_inputs(name, rows, seed):
    net = oracle.Net(helpers.ir_text(name))
    if name == "xor":
        return net, XOR_X.copy(), XOR_Y.copy()
    x = helpers.net_inputs(net, name, seed, rows)
    y = helpers.net_labels(net, seed, rows) if net.train else None
    return net, x, y


# 100-step loss curves, host-side cosine warmup schedule (lr * lr_scale(t),
# t = 0..99, so the first step has lr 0), on reduced c5 twins:
# name, tokens, seed, base lr
CURVES = [("c5s", 256, 201, 3e-4), ("c5s", 256, 202, 0.02), ("c5t", 96, 203, 0.05), ("moeb", 512, 204, 0.01),
          ("drp", 128, 205, 0.01)]


def curve_lrs(base, steps=100):
    return [np.float32(base) * np.float32(oracle.lr_scale_cosine(t)) for t in range(steps)]


def written(lib, m, x):
    """ns_eval_infer's output, cut to the prefix the driver wrote: it copies
    its result buffer, which for some data-movement programs is shorter than
    ns_model_output_numel (two runs over differently pre-filled outputs)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    outs = []
    for fill in (np.float32(-7.5e37), np.float32(3.25e37)):
        o = np.full(lib.output_numel(m, x.size), fill, dtype=np.float32)
        assert lib.lib.ns_eval_infer(m, _fp(x), _fp(o), x.size) == 0
        outs.append(o)
    diff = np.nonzero(outs[0].view(np.uint32) != outs[1].view(np.uint32))[0]
    return outs[0][: diff[0]] if diff.size else outs[0]


def digest(a):
    return hashlib.sha256(np.ascontiguousarray(a, dtype=np.float32).tobytes()).hexdigest()[:16]


def main(names=()):
    for name, rows, seed, steps, lr, life in CASES:
        if names and name not in names:
            continue
        net, x, y = case_inputs(name, rows, seed)
        w = helpers.net_weights(name, seed)
        lib = NsLib(os.path.join(helpers.REF, f"lib{name}.so"))
        m = lib.init(w)
        out = written(lib, m, x)[: net.output_numel(x.size) if net.moe is None else rows * net.moe["D"]]
        rec = dict(out=out, x_digest=np.array(digest(x)), w_digest=np.array(digest(w)))
        if steps:
            rec["losses"] = np.array([lib.train_step(m, x, y, lr) for _ in range(steps)], dtype=np.float32)
            rec["objective"] = np.float32(lib.objective_loss(m, x, y))
            rec["w_final"] = lib.get_weights(m)
            rec["out_after"] = lib.eval_infer(m, x)[: out.size]
        if life:
            outs, counts = [], []
            counts.append(lib.lib.ns_expert_birth(m, 1))
            outs.append(lib.eval_infer(m, x)[: out.size])
            counts.append(lib.lib.ns_expert_merge(m, 0, 1))
            outs.append(lib.eval_infer(m, x)[: out.size])
            counts.append(lib.lib.ns_expert_kill(m, 2))
            outs.append(lib.eval_infer(m, x)[: out.size])
            rec["life_counts"] = np.array(counts, dtype=np.int64)
            rec["life_outs"] = np.stack(outs)
            rec["life_w"] = lib.get_weights(m)
            # the reference's NSM2 file after the lifecycle (codegen.cpp:2505-2528):
            # digest of every byte, and the MoE tail after the blob
            import tempfile
            with tempfile.TemporaryDirectory() as d:
                path = os.path.join(d, "life.nsm")
                assert lib.save(m, path) == 0
                with open(path, "rb") as f:
                    raw = f.read()
                rec["ckpt_digest"] = np.array(hashlib.sha256(raw).hexdigest())
                rec["ckpt_tail"] = np.frombuffer(raw[12 + 4 * rec["life_w"].size:], dtype=np.uint8).copy()
                # an NSM1 file of the initial weights loads with every slot alive
                # (codegen.cpp:2549-2551); the forward after that load
                nsm1 = os.path.join(d, "w.nsm1")
                with open(nsm1, "wb") as f:
                    f.write(np.uint32(0x4E534D31).tobytes() + np.uint64(w.size).tobytes() + w.tobytes())
                m1 = lib.init(w)
                assert lib.load(m1, nsm1) == 0
                rec["nsm1_count"] = np.int64(lib.lib.ns_expert_count(m1))
                rec["nsm1_out"] = lib.eval_infer(m1, x)[: out.size]
                lib.free(m1)
        lib.free(m)
        np.savez_compressed(os.path.join(HERE, f"{name}.npz"), **rec)
        print(name, {k: getattr(v, "shape", None) for k, v in rec.items()})


def curves(names=()):
    for name, rows, seed, base in CURVES:
        if names and name not in names:
            continue
        net = oracle.Net(helpers.ir_text(name))
        x = helpers.net_inputs(net, name, seed, rows)
        y = helpers.net_labels(net, seed, rows)
        w = helpers.net_weights(name, seed, std=0.1)
        lib = NsLib(os.path.join(helpers.REF, f"lib{name}.so"))
        m = lib.init(w)
        losses = np.array([lib.train_step(m, x, y, lr) for lr in curve_lrs(base)], dtype=np.float32)
        wf = lib.get_weights(m)
        lib.free(m)
        tag = f"curve_{name}_{seed}"
        np.savez_compressed(os.path.join(HERE, tag + ".npz"), losses=losses, x_digest=np.array(digest(x)),
                            w_final_digest=np.array(digest(wf)))
        print(tag, losses[[0, 1, 50, 99]])


def config_c1():
    """c1_workload.npz: configuration c1 exactly as stated (batch 256,
    Xavier-uniform weights and U[-1,1] inputs from the workload generator),
    forward through the reference's own emitted driver."""
    from neuralscript_amd import workloads
    ir = helpers.ir_text("c1")
    net = oracle.Net(ir)
    layout = [(n, net.offsets[n], r * c) for n, r, c in net.weights]
    w = workloads.weights("c1", layout, workloads.ir_shapes(ir))
    x = workloads.inputs("c1")
    lib = NsLib(os.path.join(helpers.REF, "libc1.so"))
    m = lib.init(w)
    out = lib.eval_infer(m, x)
    lib.free(m)
    np.savez_compressed(os.path.join(HERE, "c1_workload.npz"), out=out, x_digest=np.array(digest(x)),
                        w_digest=np.array(digest(w)))
    print("c1_workload", out.shape)


if __name__ == "__main__":
    if sys.argv[1:] == ["c1_workload"]:
        config_c1()
    else:
        main(sys.argv[1:])
        curves(sys.argv[1:])
