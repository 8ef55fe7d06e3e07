"""Benchmark of the NeuralScript HIP backend on one MI355X.

`python bench.py` runs every GPU configuration of BASELINE.json and prints ONE
JSON line.  The headline (`value`) is config c5 -- the largest single-GPU
workload and the metric's "train steps/s" half: device-resident
`ns_runtime_train_step` (nsh_train_step_device) of the emb->attn->LN->MLP->CE
transformer on one 16384-token sequence, steps/s.  c2, c3 (ns_eval_infer
forward, tokens/s) and c4 (MoE forward, tokens/s) are nested under
`configs`, each with the same fields.  Inputs and weights are synthetic
(seeded SplitMix64 streams, neuralscript_amd/workloads.py) and already in HBM
when a timed region starts.

Each config carries
  roofline     -- its dominant kernel: algorithmic FLOP per launch / average
                  launch time, from HIP events recorded on the model's stream
                  around every launch in the timed region; `traffic` = HBM
                  bytes per launch measured with rocprofv3 --pmc (profiles/);
  cpu_baseline -- the reference's CPU path in the reference's own loop nests
                  (oracle/ns_refloop.c, gcc -O2, one thread; pinned bitwise to
                  the reference's emitted drivers) on a bounded sample of the
                  same workload, extrapolated to the whole call as the
                  `sample` field states.
--config c2|c3|c4|c5 runs one config (profiling runs); --config peak and copy
run the attainable-peak microbenchmarks and the rocprof calibration copy.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import platform
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "ns_eval_infer tokens/s + % of fp32-MFMA/HBM roofline; train steps/s"
MFMA_F32_PEAK_TFLOPS = 157.3   # MI355X dense fp32 MFMA
HBM_PEAK_GBS = 8000.0
CPU_ORDER = "reference loop nests (oracle/ns_refloop.c, gcc -O2, no FMA, one thread)"


def load_traffic(kernel):
    """HBM bytes per launch measured with rocprofv3 --pmc (profiles/), if any."""
    p = os.path.join(ROOT, "profiles", "traffic.json")
    if not os.path.exists(p):
        return None
    with open(p) as f:
        return json.load(f).get(kernel)


def host_info():
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"cpu": model, "nproc": os.cpu_count(), "glibc": "-".join(platform.libc_ver())}


# ---------------------------------------------------------------------------
# algorithmic work
# ---------------------------------------------------------------------------

def c2_work(M=8192):
    return {"gemm": 2.0 * M * (1024 * 4096 + 4096 * 4096 + 4096 * 1024)}


def c3_work(M=16384, D=1024):
    # gemm: the 4 projections; attention: QK^T + PV over all heads;
    # embedding / layernorm: bytes (one read + one write of [M, D] fp32)
    return {"gemm": 2.0 * M * D * D * 4, "attention_fwd": 4.0 * M * M * D,
            "embedding": 2.0 * M * D * 4, "layernorm": 2.0 * M * D * 4}


def c4_work(M=65536, D=1024, E=64, H=1024):
    return {"moe_route": 2.0 * M * D * E, "moe_experts": 4.0 * M * D * H}


def c5_work(M=16384, D=512, FF=2048, C=8192):
    """Algorithmic FLOP of one c5 training step (attention counted once: its
    forward QK^T + PV, its backward dV, dP, dQ, dK)."""
    dense_fwd = 2.0 * M * (4 * D * D + D * FF + FF * D + D * C)
    return {"dense": 3 * dense_fwd, "attention_fwd": 4.0 * M * M * D, "attention_bwd": 8.0 * M * M * D,
            "total": 3 * dense_fwd + 12.0 * M * M * D}


def c5_hbm_bytes(n_muon, M=16384, D=512, C=8192, V=8192):
    """Algorithmic HBM bytes per step of c5's bandwidth-bound regions: CE reads
    the logits and the one-hot labels and writes the gradient ([M, C] each);
    the Muon gather reads g and writes its transpose, the update reads the q
    vectors and w and writes w (n_muon elements each); embedding and LayerNorm
    read and write [M, D] (LayerNorm's gradient also reads x); the embedding
    gradient as emb_grad_bytes."""
    return {"softmax_xent": 3.0 * M * C * 4, "muon_gather": 2.0 * n_muon * 4, "muon_update": 3.0 * n_muon * 4,
            "embedding": 2.0 * M * D * 4, "layernorm": 2.0 * M * D * 4, "layernorm_grad": 3.0 * M * D * 4,
            "embedding_grad": emb_grad_bytes(M, V, D)}


def emb_grad_bytes(M, V, D):
    """The embedding gradient reads the [M, D] gradient rows and the M ids
    and writes the whole [V, D] table once."""
    return (M * D + M + V * D) * 4.0


HBM_REGIONS = ("embedding", "layernorm", "layernorm_grad", "softmax_xent", "muon_gather", "muon_update",
               "embedding_grad")

# Dominant kernel of each config: (profile region, kernel name, bound).
DOMINANT = {"c2": ("gemm", "gemm_f32_kernel", "mfma"),
            "c3": ("attention_fwd", "flash_fwd_kernel<64>", "mfma"),
            "c3d": ("attention_fwd", "flash_fwd_kernel<128>", "mfma"),
            "c4": ("moe_experts", "gemm_f32_kernel (grouped by expert, gather/scatter rows)", "mfma"),
            "c5": ("attention_bwd", "flash_bwd_dkdv_kernel<64,true> + flash_bwd_dq_ds_kernel<64>", "mfma")}
TRAFFIC_KEY = {"c2": "gemm_f32_kernel", "c3": "c3:attention_fwd", "c3d": "c3d:attention_fwd", "c4": "c4:moe_experts",
               "c5": "c5:attention_bwd"}


# Profile regions that are variants of one kernel: `gemm_act` is the GEMM
# with the fused activation epilogue.
REGION_VARIANTS = {"gemm": ("gemm", "gemm_act")}


def _group(prof, region):
    """Profile entries of a region: `region` itself and its variants."""
    return [k for k in REGION_VARIANTS.get(region, (region,)) if k in prof]


def roofline_of(key, work, prof):
    """Roofline object of the dominant kernel: algorithmic FLOP of one launch
    over its average HIP-event time in the timed region."""
    region, kernel, bound = DOMINANT[key]
    members = _group(prof, region)
    calls = sum(prof[k]["calls"] for k in members)
    ms = sum(prof[k]["ms"] for k in members)
    per_launch_ms = ms / calls
    flop = work[region] / (calls / prof["_steps"])  # work per step / launches per step
    achieved = flop / (per_launch_ms * 1e-3) / 1e12
    return {"bound": bound, "kernel": kernel, "region": region, "achieved": achieved, "peak": MFMA_F32_PEAK_TFLOPS,
            "unit": "TFLOP/s", "frac": achieved / MFMA_F32_PEAK_TFLOPS, "flop_per_launch": flop,
            "avg_launch_ms": per_launch_ms, "launches": calls, "profile_regions": members,
            "traffic": load_traffic(TRAFFIC_KEY[key])}


def kernel_table(prof, steps, work, hbm):
    """Per profile region: ms and launches per step, and the achieved rate
    of the regions whose algorithmic work is known (a region's variants are
    summed, e.g. gemm + gemm_act)."""
    out = {}
    for k, v in prof.items():
        if k.startswith("_"):
            continue
        out[k] = {"ms_per_step": v["ms"] / steps, "calls_per_step": v["calls"] / steps}
    for k, amount in list(work.items()) + list(hbm.items()):
        members = _group(prof, k)
        if not members:
            continue
        ms = sum(prof[m]["ms"] for m in members) / steps
        e = out[k] if members == [k] else out.setdefault(k + " (all variants)", {"ms_per_step": ms})
        if k in hbm:
            e["GB/s"] = amount / (ms * 1e-3) / 1e9
            e["hbm_frac"] = e["GB/s"] / HBM_PEAK_GBS
        else:
            e["TFLOP/s"] = amount / (ms * 1e-3) / 1e12
    return out


# ---------------------------------------------------------------------------
# GPU legs (device-resident inputs)
# ---------------------------------------------------------------------------

def _setup(key):
    from neuralscript_amd import runtime, workloads
    if not runtime.has_gpu():
        raise SystemExit("bench.py: no GPU visible to libnship")
    wl = workloads.CONFIGS[key]
    plan = runtime.Plan.load(wl.net)
    w = workloads.weights(key, plan.layout(), workloads.ir_shapes(plan.ir))
    return runtime, workloads, wl, plan, w


def _timed(model, step, steps, warmup, timed_regions):
    """warmup untimed calls, then `steps` timed calls synchronised on both
    sides, in which HIP events on the model's stream bracket only the
    launches of `timed_regions` (the roofline's: every event pair leaves a
    gap of a few microseconds between launches, ~0.24 ms per c5 step if every
    region were timed); then `steps` more calls with every region timed, for
    the per-region breakdown.  The timed regions' figures in the returned
    profile are the timed run's."""
    for _ in range(warmup):
        step()
    model.sync()
    model.profile_select(timed_regions)
    model.profile(True)
    model.profile_reset()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    model.sync()
    dt = time.perf_counter() - t0
    timed = model.profile_report()
    model.profile_select(None)
    model.profile_reset()
    for _ in range(steps):
        step()
    model.sync()
    prof = model.profile_report()
    model.profile(False)
    prof.update(timed)
    prof["_steps"] = steps
    return dt, prof


KERNELS_NOTE = ("per profile region, HIP events around each launch, from a second run of the same number of "
                "steps after the timed one; the roofline region's figures are the timed run's")


def _roof_regions(key):
    """Profile regions of config `key`'s dominant kernel (and its variants)."""
    region = DOMINANT[key][0]
    return list(REGION_VARIANTS.get(region, (region,)))


def bench_forward(key, steps, warmup, with_cpu, budget):
    """Device-resident forward (nsh_eval_infer_device) of config `key`."""
    runtime, workloads, wl, plan, w = _setup(key)
    x = workloads.inputs(key)
    model = runtime.Model(plan, w)
    dx = runtime.DeviceArray.from_host(x)
    dy = runtime.DeviceArray(wl.rows * plan.out_cols)
    dt, prof = _timed(model, lambda: model.eval_infer_device(dx, dy), steps, warmup, _roof_regions(key))
    out = dy.to_host()
    if not np.isfinite(out).all():
        raise SystemExit(f"bench.py: non-finite {key} output")
    # host-pointer ABI (ns_eval_infer: PCIe copies included), for reference;
    # the caller's output array exists already, as an application's would
    host_out = model.eval_infer(x)
    t0 = time.perf_counter()
    for _ in range(3):
        model.eval_infer(x, out=host_out)
    abi_dt = (time.perf_counter() - t0) / 3
    routing = None
    if key == "c4":
        E = workloads.ir_shapes(plan.ir)["moe_g_w"][1]
        best, _, lg = model.last_routing(wl.rows, E)
        routing = routing_report(best, lg, E)
    model.free()
    dx.free()
    dy.free()
    work = {"c2": c2_work, "c3": c3_work, "c3d": c3_work, "c4": c4_work}[key]()
    hbm = {k: v for k, v in work.items() if k in HBM_REGIONS}
    res = {"value": wl.rows * steps / dt, "unit": "tokens/s", "ms_per_step": dt * 1e3 / steps,
           "workload": f"{key}: {wl.desc}", "tokens": wl.rows, "entry": "nsh_eval_infer_device",
           "roofline": roofline_of(key, work, prof), "kernels_note": KERNELS_NOTE, "kernels": kernel_table(prof, steps, work, hbm),
           "host_abi": {"tokens_per_s": wl.rows / abi_dt, "ms": abi_dt * 1e3,
                        "note": "ns_eval_infer with host buffers (PCIe-inclusive)"}}
    if routing is not None:
        res["routing"] = routing
    if with_cpu and key != "c3d":  # c3d is no BASELINE config: no CPU leg
        res["cpu_baseline"] = {"c2": cpu_c2, "c3": cpu_c3, "c4": cpu_c4}[key](w, budget)
    return res


def routing_report(best, logits, E):
    """Realised expert histogram and top-2 gate-logit ties (exact, and within
    1e-6 relative) of the last routed batch."""
    hist = np.bincount(best[best >= 0], minlength=E)
    lg = logits.reshape(-1, E).astype(np.float64)
    top2 = np.sort(lg, axis=1)[:, -2:]
    gap = top2[:, 1] - top2[:, 0]
    return {"histogram": hist.tolist(), "max_share": float(hist.max() / max(1, hist.sum())),
            "exact_ties": int((gap == 0).sum()),
            "near_ties_1e-6": int(((gap > 0) & (gap <= 1e-6 * np.maximum(1.0, np.abs(top2[:, 1])))).sum())}


def adamw_bandwidth(n, launches=20):
    """The AdamW kernel (nsh_op_adamw_step) over n parameters, as if every
    weight of the step took AdamW: 4 arrays read, 3 written (28 bytes per
    parameter), timed over `launches` back-to-back launches."""
    from neuralscript_amd import runtime
    bufs = [runtime.DeviceArray(n) for _ in range(4)]
    for b in bufs:
        b.fill_zero()
    w, g, m, v = (b.ptr for b in bufs)
    lib = runtime.lib()
    lr = ctypes.c_float(3e-4)
    lib.nsh_op_adamw_step(w, g, m, v, n, 1, lr)
    runtime.check(lib.nsh_device_synchronize(), "synchronize")
    t0 = time.perf_counter()
    for t in range(launches):
        lib.nsh_op_adamw_step(w, g, m, v, n, t + 2, lr)
    runtime.check(lib.nsh_device_synchronize(), "synchronize")
    us = (time.perf_counter() - t0) / launches * 1e6
    for b in bufs:
        b.free()
    gbs = 28.0 * n / (us * 1e-6) / 1e9
    return {"params": n, "us_per_launch": us, "GB/s": gbs, "hbm_frac": gbs / HBM_PEAK_GBS,
            "note": "the whole parameter count of the step through the AdamW kernel (28 B per parameter)"}


def rowop_bandwidth(dx, dy, M=16384, D=512, V=8192, C=8192, reps=50):
    """The step's row kernels at c5's shapes (its own ids and labels), each
    timed over `reps` back-to-back launches (nsh_bench_rowops): for kernels of
    10-50 us the per-launch HIP events of the profile regions add a large
    share of their time."""
    from neuralscript_amd import runtime
    us = (ctypes.c_double * 5)()
    runtime.check(runtime.lib().nsh_bench_rowops(dx.ptr, dy.ptr, M, D, V, C, reps, us), "bench_rowops")
    nbytes = {"embedding": 2.0 * M * D * 4, "layernorm": 2.0 * M * D * 4, "layernorm_grad": 3.0 * M * D * 4,
              "embedding_grad": emb_grad_bytes(M, V, D), "softmax_xent": 3.0 * M * C * 4}
    out = {"note": f"each kernel over {reps} back-to-back launches at c5's shapes, one event pair"}
    for k, (name, b) in enumerate(nbytes.items()):
        gbs = b / (us[k] * 1e-6) / 1e9
        out[name] = {"us_per_launch": us[k], "bytes": b, "GB/s": gbs, "hbm_frac": gbs / HBM_PEAK_GBS}
    return out


def bench_train(key, steps, warmup, with_cpu, budget):
    """Device-resident training steps (nsh_train_step_device); lr = 3e-4
    times the cosine-warmup multiplier, as the host applies it."""
    runtime, workloads, wl, plan, w = _setup(key)
    dx = runtime.DeviceArray.from_host(workloads.inputs(key))
    dy = runtime.DeviceArray.from_host(workloads.labels(key))
    model = runtime.Model(plan, w)
    t = [0]

    def step():
        model.train_step_device(dx, dy, 3e-4 * min(1.0, t[0] / 100.0), want_loss=False)
        t[0] += 1

    dt, prof = _timed(model, step, steps, warmup, _roof_regions(key))
    loss = model.train_step_device(dx, dy, 3e-4 * min(1.0, t[0] / 100.0))
    t[0] += 1
    # host-pointer ABI (ns_runtime_train_step: the [M, C] one-hot labels cross
    # PCIe every call), for reference
    xh, yh = workloads.inputs(key), workloads.labels(key)
    t0 = time.perf_counter()
    for _ in range(2):
        model.train_step(xh, yh, 3e-4 * min(1.0, t[0] / 100.0))
        t[0] += 1
    abi_dt = (time.perf_counter() - t0) / 2
    model.free()
    row_kernels = rowop_bandwidth(dx, dy) if key == "c5" else None
    dx.free()
    dy.free()
    work = c5_work()
    shapes = workloads.ir_shapes(plan.ir)
    # Muon matrices (codegen.cpp:3097): every 2-D weight with min(r, c) >= 8
    n_muon = sum(int(np.prod(v)) for v in shapes.values() if len(v) == 2 and min(v) >= 8)
    res = {"value": steps / dt, "unit": "steps/s", "ms_per_step": dt * 1e3 / steps,
           "workload": f"{key}: {wl.desc}", "tokens": wl.rows, "entry": "nsh_train_step_device",
           "achieved_TFLOP/s": work["total"] / (dt / steps) / 1e12, "last_loss": float(loss),
           "roofline": roofline_of(key, work, prof), "kernels_note": KERNELS_NOTE,
           "kernels": kernel_table(prof, steps, work, c5_hbm_bytes(n_muon)),
           "adamw": adamw_bandwidth(n_muon), "row_kernels": row_kernels,
           "host_abi": {"steps_per_s": 1.0 / abi_dt, "ms": abi_dt * 1e3,
                        "note": "ns_runtime_train_step with host buffers (labels uploaded every call)"}}
    if with_cpu:
        res["cpu_baseline"] = cpu_c5(w, budget)
    return res


def bench_moe_backward(steps, warmup):
    """The MoE backward at config 4's expert shape (d_model 1024, 64 experts,
    FFN 1024) over 4096 Zipf-routed tokens: training steps of the `moep`
    network (embedding -> MoE -> fc -> CE; not a BASELINE config), lr 0, with
    the backward's phases timed as profile regions: the expert-grouped
    products (dpre2 = dout We2[e]^T, dx += dH We1[e]^T: 4 M D H FLOP) and the
    K-grouped weight gradients (dWe1, dWe2: 4 M D H FLOP)."""
    from neuralscript_amd import runtime, workloads
    M, D, H = 4096, 1024, 1024
    plan = runtime.Plan.load("moep")
    w, x, y = workloads.moe_training_workload(M)
    model = runtime.Model(plan, w)
    dx, dy = runtime.DeviceArray.from_host(x), runtime.DeviceArray.from_host(y)
    dt, prof = _timed(model, lambda: model.train_step_device(dx, dy, 0.0, want_loss=False), steps, warmup,
                      ["moe_bwd_grouped", "moe_bwd_kgrouped"])
    model.free()
    dx.free()
    dy.free()
    work = {"moe_bwd_grouped": 4.0 * M * D * H, "moe_bwd_kgrouped": 4.0 * M * D * H}
    out = {"workload": "MoE backward at config 4's expert shape: moep (emb 8192x1024 -> MoE D 1024, E 64, "
                       "FFN 1024 -> fc 16), 4096 Zipf-routed tokens, train step at lr 0",
           "kernels_note": KERNELS_NOTE, "kernels": kernel_table(prof, steps, work, {})}
    for region, flop in work.items():
        ms = prof[region]["ms"] / prof[region]["calls"]
        tf = flop / (ms * 1e-3) / 1e12
        out[region] = {"bound": "mfma", "achieved": tf, "peak": MFMA_F32_PEAK_TFLOPS, "unit": "TFLOP/s",
                       "frac": tf / MFMA_F32_PEAK_TFLOPS, "flop_per_launch": flop, "avg_launch_ms": ms}
    return out


# ---------------------------------------------------------------------------
# CPU baselines: the reference's loop nests on a bounded sample
# ---------------------------------------------------------------------------

class _RefOrder:
    """The oracle's kernel wrappers routed to the reference-order library for
    the duration of a `with` block."""

    def __enter__(self):
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import oracle
        self.oracle = oracle
        self.prev = oracle.use_reference_order(True)
        return oracle

    def __exit__(self, *exc):
        self.oracle.use_reference_order(self.prev)


def _oracle_net(key):
    from neuralscript_amd import workloads
    with _RefOrder() as oracle:
        with open(os.path.join(ROOT, "neuralscript_amd", "nets", workloads.CONFIGS[key].net + ".mlir")) as f:
            return oracle.Net(f.read())


def _baseline(value, unit, sample, seconds, extrapolated, **extra):
    d = {"value": value, "unit": unit, "cores": 1, "kind": "port", "order": CPU_ORDER, "sample": sample,
         "cpu_seconds": seconds, "extrapolated": extrapolated}
    d.update(extra)
    return d


def cpu_c2(w, budget=10.0):
    """The whole forward (3 GEMMs + GELU epilogues, i-j-k) on the first rows
    of the batch; rows are independent, so tokens/s carries over."""
    from neuralscript_amd import workloads
    net = _oracle_net("c2")
    x = workloads.inputs("c2", rows=256)
    with _RefOrder() as oracle:
        m = oracle.Model(net, w)
        t0 = time.perf_counter()
        m.eval_infer(x[:1024])
        t1 = time.perf_counter() - t0
        rows = int(max(1, min(256, budget / t1)))
        t0 = time.perf_counter()
        m.eval_infer(x[: rows * 1024])
        dt = time.perf_counter() - t0
    return _baseline(rows / dt, "tokens/s", f"c2 forward of {rows} of the 8192 rows", dt, False)


def cpu_c3(w, budget=10.0, p_rows=64, q_rows=16):
    """Embedding and LayerNorm over all 16384 tokens; the four D x D
    projections on p_rows rows and the per-head S x S loops on q_rows query
    rows against all 16384 keys, each scaled to 16384 rows (rows are
    independent given K and V; K, V here are the sample's projections tiled
    over the sequence, which changes values, not work)."""
    from neuralscript_amd import workloads
    M, D, H, V = 16384, 1024, 16, 32000
    net = _oracle_net("c3")
    ids = workloads.inputs("c3")
    W = {n: w[net.offsets[n]: net.offsets[n] + r * c] for n, r, c in net.weights}
    names = [n for n, _, _ in net.weights]
    t = {}
    with _RefOrder() as oracle:
        t0 = time.perf_counter()
        x = oracle.embedding(W[names[0]], ids, V, D)
        t["embedding"] = time.perf_counter() - t0
        xs = x[: p_rows * D]
        t0 = time.perf_counter()
        proj = [oracle.matmul(xs, W[n], p_rows, D, D) for n in names[1:5]]
        t["projections"] = time.perf_counter() - t0
        Q, K, Vv = (np.ascontiguousarray(np.tile(p.reshape(p_rows, D), (M // p_rows, 1)).ravel()) for p in proj[:3])
        ctx = np.zeros(M * D, np.float32)
        t["core"] = oracle.lib().rl_attention_core_rows(oracle.fp(Q), oracle.fp(K), oracle.fp(Vv), oracle.fp(ctx),
                                                        M, D, H, 0, q_rows)
        t0 = time.perf_counter()
        oracle.layernorm(x, D)
        t["layernorm"] = time.perf_counter() - t0
    total = t["embedding"] + t["projections"] * M / p_rows + t["core"] * M / q_rows + t["layernorm"]
    return _baseline(M / total, "tokens/s",
                     f"c3 forward: embedding and LayerNorm of all {M} tokens, projections of {p_rows} rows and the "
                     f"attention's per-head loops for {q_rows} query rows against all {M} keys, scaled to {M} rows; "
                     f"extrapolated call time {total:.0f} s", sum(t.values()), True,
                     parts_s={k: round(v, 4) for k, v in t.items()})


def cpu_c4(w, budget=10.0):
    """The per-token MoE loop (router, top-1, expert FFN) on the first
    tokens of the batch; tokens are independent, so tokens/s carries over
    (the sample follows the same Zipf routing)."""
    from neuralscript_amd import workloads
    M, D, E, H = 65536, 1024, 64, 1024
    x = workloads.inputs("c4", rows=512)
    Wg, We1, We2 = w[: D * E], w[D * E: D * E + E * D * H], w[D * E + E * D * H:]
    with _RefOrder() as oracle:
        t0 = time.perf_counter()
        oracle.moe_fwd(x[:D], Wg, We1, We2, None, 1, D, H, E)
        t1 = time.perf_counter() - t0
        n = int(max(1, min(512, budget / t1)))
        t0 = time.perf_counter()
        oracle.moe_fwd(x[: n * D], Wg, We1, We2, None, n, D, H, E)
        dt = time.perf_counter() - t0
    return _baseline(n / dt, "tokens/s", f"c4 MoE forward of {n} of the {M} tokens", dt, False)


def cpu_c5(w, budget=20.0, m_small=64, nq=8, nk=8):
    """One training step, extrapolated per operation to c5's 16384 tokens:
      * a whole step of the train core at m_small tokens (full D, vocabulary,
        classes), every operation timed: GEMMs, their gradients, CE,
        LayerNorm, embedding and their gradients scale with the token count;
      * the attention's S x S loops timed at the full S = 16384 on a sample
        (forward: nq query rows of all heads; backward: one head, nq query
        rows and nk key rows, its S x S buffers filled), scaled to all rows
        and heads; the backward runs 5 times per step, once per output
        (codegen.cpp:3017-3051), so its recomputation counts 5 times;
      * Muon at full size (it does not depend on the token count), except the
        two 8192-long matrices, taken as 4x their 2048-long twins (MGS work
        R*C^2, same access pattern)."""
    from neuralscript_amd import synth, workloads
    M, D, H = 16384, 512, 8
    net = _oracle_net("c5")
    x = workloads.inputs("c5", rows=m_small)
    y = workloads.labels("c5", rows=m_small)
    r = M / m_small
    names = ["matmul", "matmul_grad_a", "matmul_grad_w", "act", "act_grad", "layernorm", "layernorm_grad",
             "embedding", "embedding_grad_w", "cross_entropy", "loss_grad", "attention_fwd", "attention_bwd"]
    t, split, opt = {}, (ctypes.c_double * 8)(), {}
    with _RefOrder() as oracle:
        orig = {n: getattr(oracle, n) for n in names}

        def wrap(n):
            f = orig[n]

            def g(*a, **k):
                t0 = time.perf_counter()
                out = f(*a, **k)
                dt = time.perf_counter() - t0
                if n.startswith("attention"):
                    oracle.lib().rl_last_attention_split(split)
                    t[n] = list(split)
                else:
                    t[n] = t.get(n, 0.0) + dt
                return out
            return g

        def opt_step(self, o, val, record, adamw_only=False):
            L = oracle.lib()
            done = {}
            for k in range(0, len(o) - 1, 2):
                name, g = o[k], o[k + 1]
                rr, cc = self.net.shape[name]
                if max(rr, cc) == 8192:
                    continue
                gr = oracle.f32(val(g)).copy()
                t0 = time.perf_counter()
                L.or_muon_step(oracle.fp(self.weight(name)), oracle.fp(gr), rr, cc, ctypes.c_float(self._lr))
                opt[name] = time.perf_counter() - t0
                done[(rr, cc)] = opt[name]
            for k in range(0, len(o) - 1, 2):
                rr, cc = self.net.shape[o[k]]
                if max(rr, cc) == 8192:
                    opt[o[k]] = 4.0 * done[(2048, cc) if rr == 8192 else (rr, 2048)]

        try:
            for n in names:
                setattr(oracle, n, wrap(n))
            model = oracle.Model(net, w)
            model._opt_step = opt_step.__get__(model)
            t0 = time.perf_counter()
            model.train_step(x, y, 3e-4)
            t_small = time.perf_counter() - t0
        finally:
            for n in names:
                setattr(oracle, n, orig[n])
        # the S x S loops at S = 16384 on a sample
        t0 = time.perf_counter()
        L = oracle.lib()
        Q, K, V, dP = (synth.normal(11 + i, M * D, 0.5) for i in range(4))
        ctx = np.zeros(M * D, np.float32)
        core_f = L.rl_attention_core_rows(oracle.fp(Q), oracle.fp(K), oracle.fp(V), oracle.fp(ctx), M, D, H, 0, nq)
        sc = np.full(M * M, 1.0 / M, np.float32)
        ds = np.full(M * M, 1e-6, np.float32)
        tb = (ctypes.c_double * 2)()
        L.rl_attention_bwd_core_sample(oracle.fp(Q), oracle.fp(K), oracle.fp(V), oracle.fp(dP), oracle.fp(sc),
                                       oracle.fp(ds), M, D, H, nq, nk, tb)
        del sc, ds
        t_attn_sample = time.perf_counter() - t0
    lin = sum(v for n, v in t.items() if not n.startswith("attention"))
    af, ab = t["attention_fwd"], t["attention_bwd"]
    attn_fwd = af[0] * r + core_f * M / nq
    attn_bwd_core = H * (tb[0] * M / nq + tb[1] * M / nk)
    attn_bwd = 5 * (ab[0] * r + attn_bwd_core) + sum(ab[2:7]) * r
    optim = sum(opt.values())
    total = lin * r + attn_fwd + attn_bwd + optim
    parts = {"token_linear_ops": lin * r, "attention_fwd": attn_fwd, "attention_bwd_x5": attn_bwd, "muon": optim}
    return _baseline(1.0 / total, "steps/s",
                     f"one c5 step extrapolated per operation: the train core at {m_small} tokens scaled to {M}, "
                     f"the attention's S x S loops at S = {M} on {nq} query / {nk} key rows, Muon at full size; "
                     f"extrapolated step time {total:.0f} s", t_small + t_attn_sample, True,
                     parts_s={k: round(v, 1) for k, v in parts.items()})


# ---------------------------------------------------------------------------
# peaks and calibration
# ---------------------------------------------------------------------------

def measured_peaks(reps=3):
    """Attainable peaks of this GPU, measured by libnship's microbenchmarks,
    best of `reps` runs each: a register-only fp32 MFMA loop (2048 workgroups
    x 4 waves, 4 independent 32x32x2 chains per wave) and a float4 copy of
    256 MiB each way.  The default run measures them first, on a cold GPU
    (the MFMA clock falls as the GPU heats)."""
    from neuralscript_amd import runtime
    lib = runtime.lib()
    tf = ctypes.c_double()
    tfs = []
    for _ in range(reps):
        runtime.check(lib.nsh_bench_mfma_peak(4000, 2048, ctypes.byref(tf)), "bench_mfma_peak")
        tfs.append(tf.value)
    n = 1 << 26
    src, dst = runtime.DeviceArray(n), runtime.DeviceArray(n)
    src.fill_zero()
    dst.fill_zero()
    gbs = ctypes.c_double()
    bws = []
    for _ in range(reps):
        runtime.check(lib.nsh_bench_copy(src.ptr, dst.ptr, n, 10, ctypes.byref(gbs)), "bench_copy")
        bws.append(gbs.value)
    src.free()
    dst.free()
    return {"mfma_f32_tflops": max(tfs), "mfma_frac_of_published": max(tfs) / MFMA_F32_PEAK_TFLOPS,
            "hbm_copy_gbs": max(bws), "hbm_frac_of_published": max(bws) / HBM_PEAK_GBS,
            "runs": {"mfma_f32_tflops": tfs, "hbm_copy_gbs": bws}}


def library_gemm(M=8192, N=4096, K=4096, reps=20):
    """The vendor library's fp32 GEMM (torch.mm -> hipBLASLt / rocBLAS, no
    reduced-precision modes) on c2's 4096x4096 layer, for comparison only."""
    import torch
    torch.backends.cuda.matmul.allow_tf32 = False
    a = torch.randn(M, K, device="cuda", dtype=torch.float32)
    b = torch.randn(K, N, device="cuda", dtype=torch.float32)
    for _ in range(3):
        c = torch.mm(a, b)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        c = torch.mm(a, b)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    del c
    return {"shape": [M, N, K], "ms": ms, "TFLOP/s": 2.0 * M * N * K / (ms * 1e-3) / 1e12,
            "torch": torch.__version__}


def bench_peak():
    """--config peak: the attainable peaks and the vendor library's fp32 GEMM
    next to libnship's on the same shape."""
    from neuralscript_amd import runtime
    res = {"measured_peak": measured_peaks()}
    M, N, K = 8192, 4096, 4096
    A, B, C = runtime.DeviceArray(M * K), runtime.DeviceArray(K * N), runtime.DeviceArray(M * N)
    for d in (A, B, C):
        d.fill_zero()
    for _ in range(3):
        runtime.op("gemm", A, B, C, M, N, K, K, N, N, 0, 0, 0)
    t0 = time.perf_counter()
    reps = 20
    for _ in range(reps):
        runtime.op("gemm", A, B, C, M, N, K, K, N, N, 0, 0, 0)
    ms = (time.perf_counter() - t0) / reps * 1e3
    res["libnship_gemm"] = {"shape": [M, N, K], "ms": ms, "TFLOP/s": 2.0 * M * N * K / (ms * 1e-3) / 1e12,
                            "note": "nsh_op_gemm, synchronous per call (host-timed)"}
    res["library_gemm"] = library_gemm(M, N, K)
    return res


def copy_calibration():
    """A plain copy of known size for calibrating rocprofv3's FETCH_SIZE /
    WRITE_SIZE counters: the embedding gather with identity ids copies a
    65536 x 1024 fp32 table (256 MiB read, 256 MiB written), three launches."""
    from neuralscript_amd import runtime
    V, D = 65536, 1024
    W = runtime.DeviceArray(V * D)
    out = runtime.DeviceArray(V * D)
    idx = runtime.DeviceArray.from_host(np.arange(V, dtype=np.float32))
    for _ in range(3):
        runtime.op("embedding", W, idx, out, V, V, D)
    runtime.check(runtime.lib().nsh_device_synchronize(), "synchronize")
    return {"calibration": "embedding identity copy", "bytes_read": V * D * 4, "bytes_written": V * D * 4,
            "launches": 3}


def headline(res, steps, warmup):
    """The driver's contract fields around config c5's result."""
    out = {"metric": METRIC, "value": res["value"], "unit": res["unit"], "n_gpus": 1, "steps": steps,
           "warmup": warmup, "ms_per_step": res["ms_per_step"], "higher_is_better": True, "scaling": "weak",
           "vs_baseline": None, "dtype": "f32", "data": "synthetic (seeded SplitMix64 weights and inputs)",
           "config": {"workload": res["workload"], "tokens": res["tokens"], "entry": res["entry"]}}
    for k in ("roofline", "cpu_baseline"):
        if k in res:
            out[k] = res[k]
    out.update({k: v for k, v in res.items() if k not in out and k not in ("workload", "tokens", "entry")})
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="all",
                    choices=["all", "c2", "c3", "c3d", "c4", "c5", "moe_bwd", "copy", "peak"],
                    help="all (default): c5 training steps/s as the headline, c2/c3/c4 forward (and c3d: c3 "
                         "with 8 heads of 128) nested under `configs`; c2..c5 alone (profiling runs); copy: "
                         "the rocprof counter calibration copy; peak: attainable MFMA / HBM peaks and the "
                         "vendor library's fp32 GEMM")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=8.0,
                    help="seconds of single-core CPU work per sampled baseline leg")
    a = ap.parse_args()
    if a.gpus != 1:
        raise SystemExit("bench.py: this build measures one GPU only (the path runs on one GPU; "
                         "--gpus must be 1)")
    cpu = not a.no_cpu_baseline
    if a.config == "copy":
        res = copy_calibration()
    elif a.config == "peak":
        res = bench_peak()
    elif a.config == "c5":
        res = headline(bench_train("c5", a.steps, a.warmup, cpu, a.cpu_budget), a.steps, a.warmup)
    elif a.config == "moe_bwd":
        res = bench_moe_backward(a.steps, a.warmup)
    elif a.config in ("c2", "c3", "c3d", "c4"):
        res = headline(bench_forward(a.config, a.steps, a.warmup, cpu, a.cpu_budget), a.steps, a.warmup)
    else:
        peaks = measured_peaks()
        res = headline(bench_train("c5", a.steps, a.warmup, cpu, a.cpu_budget), a.steps, a.warmup)
        res["configs"] = {}
        for key in ("c2", "c3", "c3d", "c4"):
            print(f"bench.py: {key}", file=sys.stderr, flush=True)
            res["configs"][key] = bench_forward(key, a.steps, a.warmup, cpu, a.cpu_budget)
        print("bench.py: MoE backward at production shape", file=sys.stderr, flush=True)
        res["moe_backward"] = bench_moe_backward(min(a.steps, 10), min(a.warmup, 2))
        res["measured_peak"] = peaks
        res["host"] = host_info()
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
