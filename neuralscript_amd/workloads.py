"""The benchmark configurations (BASELINE.json `configs`) as synthetic workloads.

Each config names a bundled network plan (neuralscript_amd/nets/<net>.mlir,
printed by the reference compiler from oracle/nets/<net>.ns) and builds its
weight blob (TENSOR_ALLOC order) and inputs from seeded SplitMix64 streams
(synth.py), so every consumer -- tests, bench, oracle -- sees the same bits.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from . import synth


@dataclass(frozen=True)
class Workload:
    key: str
    net: str
    rows: int          # tokens (M) per call
    seed: int
    desc: str


CONFIGS = {
    "c1": Workload("c1", "c1", 256, 0x5EED0001,
                   "fp32 MLP 64->256 ReLU->256 ReLU->10, batch 256, U[-1,1] inputs, Xavier-uniform weights"),
    "c2": Workload("c2", "c2", 8192, 0x5EED0002,
                   "fp32 MLP 1024->4096 GELU->4096 GELU->1024, batch 8192, N(0,1) inputs, Xavier-uniform weights"),
    "c3": Workload("c3", "c3", 16384, 0x5EED0003,
                   "fp32 Embedding(32000,1024)->Attention(1024,16)->LayerNorm, 8x2048 ids as one 16384-token sequence, N(0,0.02) weights"),
    # not a BASELINE config: c3 with 8 heads of 128 (Attention(1024, 8)), the
    # head size of the flash kernels' DK = 128 instantiation
    "c3d": Workload("c3d", "c3d", 16384, 0x5EED0003,
                    "fp32 Embedding(32000,1024)->Attention(1024,8)->LayerNorm (head size 128), c3's 16384-token "
                    "sequence and weights"),
    "c4": Workload("c4", "c4", 65536, 0x5EED0004,
                   "fp32 top-1 MoE, 65536 tokens, d_model 1024, 64 experts (FFN 1024), Zipf(1.1) gate bias folded into Wg"),
    "c5": Workload("c5", "c5", 16384, 0x5EED0005,
                   "fp32 train step emb(8192,512)->attn(512,8)->LN->MLP 512->2048 ReLU->512->fc 8192, CE, 32x512 tokens"),
}


def weights(key, layout, shapes):
    """Weight blob of config `key`.  `shapes`: name -> (rows, cols)."""
    wl = CONFIGS[key]
    out = []
    for name, off, count in layout:
        r, c = shapes[name]
        s = synth.stream_seed(wl.seed, "w:" + name)
        if key in ("c1", "c2"):
            out.append(synth.xavier_uniform(s, r, c))
        elif key == "c4":
            out.append(_moe_weight(name, r, c, s))
        else:
            out.append(synth.normal(s, count, 0.02))
    return np.concatenate(out)


def zipf_probs(E, s=1.1):
    p = (np.arange(1, E + 1, dtype=np.float64)) ** (-s)
    return p / p.sum()


def _moe_weight(name, r, c, s):
    if name.endswith("_g_w"):
        # Router [D, E]: N(0, 1/D) except the last row, which carries the Zipf
        # log-prior (the reference has no gate bias; x[:, D-1] = 1 feeds it).
        D, E = r, c
        w = synth.normal(s, D * E, float(np.sqrt(1.0 / D))).reshape(D, E)
        w[D - 1, :] = np.log(zipf_probs(E)).astype(np.float32)
        return w.ravel()
    return synth.normal(s, r * c, 0.02)


def inputs(key, rows=None, in_cols=None, vocab=None, D=None):
    """Input of config `key` for `rows` tokens."""
    wl = CONFIGS[key]
    rows = wl.rows if rows is None else rows
    s = synth.stream_seed(wl.seed, "x")
    if key == "c1":
        return synth.uniform(s, rows * 64, -1.0, 1.0)
    if key == "c2":
        return synth.normal(s, rows * 1024)
    if key in ("c3", "c3d"):
        return synth.token_ids(s, rows, 32000)
    if key == "c4":
        x = synth.normal(s, rows * 1024).reshape(rows, 1024)
        x[:, 1023] = 1.0
        return x.ravel()
    if key == "c5":
        return synth.token_ids(s, rows, 8192)
    raise KeyError(key)


def labels(key, rows=None, classes=8192):
    wl = CONFIGS[key]
    rows = wl.rows if rows is None else rows
    ids = synth.token_ids(synth.stream_seed(wl.seed, "y"), rows, classes)
    return synth.one_hot(ids, classes)


def generic_weights(layout, shapes, seed, std=0.2):
    """Test-net blob: N(0, std) per weight, one stream per weight name."""
    return np.concatenate([synth.normal(synth.stream_seed(seed, "w:" + n), cnt, std)
                           for n, off, cnt in layout])


def ir_shapes(ir_text):
    """name -> (rows, cols) of every weight allocated in an IR text."""
    shapes = {}
    for line in ir_text.splitlines():
        line = line.strip()
        if not line.startswith("ns.tensor.alloc"):
            continue
        name = line.split()[1][1:]
        dims = line[line.index("[") + 1:line.index("]")].split(",")
        r = int(dims[0])
        c = int(dims[1]) if len(dims) > 1 else 1
        shapes[name] = (r, c)
    return shapes


def moe_training_workload(tokens=4096, V=8192, D=1024, E=64, H=1024, classes=16):
    """The `moep` network (embedding -> top-1 MoE -> fc -> CE) at config 4's
    expert shape, for the MoE backward at production size (not a BASELINE
    config): the embedding's last column is 1 and the router's last row holds
    log Zipf(1.1) priors, so routing is Zipf-skewed as in config 4.  Returns
    (weights in TENSOR_ALLOC order, token ids, one-hot labels)."""
    emb = synth.normal(71, V * D).reshape(V, D)
    emb[:, D - 1] = 1.0
    Wg = synth.normal(72, D * E, float(np.sqrt(1.0 / D))).reshape(D, E)
    Wg[D - 1, :] = np.log(zipf_probs(E)).astype(np.float32)
    w = np.concatenate([emb.ravel(), Wg.ravel(), synth.normal(73, E * D * H, 0.02), synth.normal(74, E * H * D, 0.02),
                        synth.normal(75, D * classes, 0.05)])
    x = synth.token_ids(synth.stream_seed(76, "x"), tokens, V)
    y = synth.one_hot(synth.token_ids(synth.stream_seed(77, "y"), tokens, classes), classes)
    return w, x, y
