"""Benchmark of the NeuralScript HIP backend on one MI355X.

Default workload = BASELINE.json configs[1] (c2): ns_eval_infer forward of the
fp32 MLP 1024->4096 GELU->4096 GELU->1024 at batch 8192, inputs already in
HBM (nsh_eval_infer_device), synthetic data / seeded weights.  One "step" is
one forward pass over the 8192-row batch.

Prints ONE JSON line with the driver's contract plus
  roofline     -- the dominant kernel (fp32-MFMA GEMM): algorithmic FLOP per
                  launch / average launch time from HIP events recorded on the
                  model's stream around every launch in the timed region;
  cpu_baseline -- the reference CPU path (the driver the reference compiler
                  emits, built from its sources into oracle/_ref) on a bounded
                  sample of the same workload, 1 core; the oracle port when
                  that build is absent.
--config c3 | c4 (forward) and c5 (training step) time the other configs the
same way (device-resident inputs) and report a per-region breakdown and the
roofline of their dominant kernel; c4 adds the realised expert histogram and
the top-2 gate-logit ties.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "ns_eval_infer tokens/s + % of fp32-MFMA/HBM roofline; train steps/s"
MFMA_F32_PEAK_TFLOPS = 157.3   # MI355X dense fp32 MFMA
HBM_PEAK_GBS = 8000.0


def c2_flops(rows):
    return 2.0 * rows * (1024 * 4096 + 4096 * 4096 + 4096 * 1024)


def load_traffic(kernel):
    """HBM bytes per launch measured with rocprofv3 --pmc (profiles/), if any."""
    p = os.path.join(ROOT, "profiles", "traffic.json")
    if not os.path.exists(p):
        return None
    with open(p) as f:
        return json.load(f).get(kernel)


def cpu_baseline_c2(budget_s=15.0):
    """Reference CPU driver (nsc --cpp --runtime, g++ -O2) on a row sample."""
    from neuralscript_amd import runtime, workloads
    from neuralscript_amd.abi import NsLib
    ref = os.path.join(ROOT, "oracle", "_ref", "libc2.so")
    plan = runtime.Plan.load("c2")
    shapes = workloads.ir_shapes(plan.ir)
    w = workloads.weights("c2", plan.layout(), shapes)
    if os.path.exists(ref):
        kind = "reference"
        lib = NsLib(ref)
        m = lib.init(w)
        run = lambda x: lib.eval_infer(m, x)  # noqa: E731
        done = lambda: lib.free(m)  # noqa: E731
    else:
        kind = "port"
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import oracle
        os.environ.setdefault("OMP_NUM_THREADS", "1")
        om = oracle.Model(oracle.Net(plan.ir), w)
        run = om.eval_infer
        done = lambda: None  # noqa: E731
    x_all = workloads.inputs("c2", rows=160)
    t0 = time.perf_counter()
    run(x_all[:1024])                     # 1 row: calibrates the sample size
    t1 = time.perf_counter() - t0
    rows = int(max(1, min(160, budget_s / max(t1, 1e-3))))
    t0 = time.perf_counter()
    run(x_all[: rows * 1024])
    dt = time.perf_counter() - t0
    done()
    return {"value": rows / dt, "unit": "tokens/s", "cores": 1, "kind": kind,
            "sample": f"c2 forward on {rows} of the 8192 rows (same weights/inputs), "
                      f"{dt:.1f} s, single-threaded as the reference emits it"}


# Algorithmic work per forward of the other configs (FLOP, and bytes of the
# bandwidth-bound kernels), for the per-kernel breakdown of --config runs.
def c3_work(M=16384, D=1024, H=16, V=32000):
    # gemm: 4 projections; attention: QK^T + PV over all heads;
    # embedding / layernorm: bytes (one read + one write of [M, D] fp32)
    return {"gemm": 2.0 * M * D * D * 4, "attention_fwd": 4.0 * M * M * D,
            "embedding": 2.0 * M * D * 4, "layernorm": 2.0 * M * D * 4}


def c4_work(M=65536, D=1024, E=64, H=1024):
    return {"moe_route": 2.0 * M * D * E, "moe_experts": 4.0 * M * D * H}


# Dominant kernel of each --config run: (profile region, kernel, bound).
DOMINANT = {"c3": ("attention_fwd", "flash_fwd_kernel<64>", "mfma"),
            "c4": ("moe_experts", "gemm_f32_kernel (grouped by expert, gather/scatter rows)", "mfma"),
            "c5": ("attention_bwd", "flash_bwd_dkdv_kernel<64,true> + flash_bwd_dq_ds_kernel<64>", "mfma")}


def roofline_of(key, region, work, ms_per_call):
    """Roofline object of the dominant kernel: algorithmic FLOP of one call
    over the HIP-event time of that call (profile region on the model's
    stream); traffic = HBM bytes per call from rocprofv3 FETCH_SIZE /
    WRITE_SIZE (profiles/)."""
    _, kernel, bound = DOMINANT[key]
    achieved = work / (ms_per_call * 1e-3) / 1e12
    return {"bound": bound, "kernel": kernel, "region": region, "achieved": achieved, "peak": MFMA_F32_PEAK_TFLOPS,
            "unit": "TFLOP/s", "frac": achieved / MFMA_F32_PEAK_TFLOPS, "flop_per_launch": work,
            "avg_launch_ms": ms_per_call, "traffic": load_traffic(f"{key}:{region}")}


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


def bench_forward(key, steps, warmup):
    """Device-resident forward of config `key`; per-kernel HIP-event times."""
    from neuralscript_amd import runtime, workloads
    if not runtime.has_gpu():
        raise SystemExit("bench.py: no GPU visible to libnship")
    wl = workloads.CONFIGS[key]
    plan = runtime.Plan.load(wl.net)
    w = workloads.weights(key, plan.layout(), workloads.ir_shapes(plan.ir))
    x = workloads.inputs(key)
    model = runtime.Model(plan, w)
    dx = runtime.DeviceArray.from_host(x)
    dy = runtime.DeviceArray(wl.rows * plan.out_cols)
    for _ in range(warmup):
        model.eval_infer_device(dx, dy)
    model.sync()
    model.profile(True)
    model.profile_reset()
    t0 = time.perf_counter()
    for _ in range(steps):
        model.eval_infer_device(dx, dy)
    model.sync()
    dt = time.perf_counter() - t0
    prof = model.profile_report()
    model.profile(False)
    # host-pointer ABI (ns_eval_infer: PCIe copies included), for reference
    model.eval_infer(x)
    t0 = time.perf_counter()
    for _ in range(3):
        model.eval_infer(x)
    abi_dt = (time.perf_counter() - t0) / 3
    routing = None
    if key == "c4":
        E = workloads.ir_shapes(plan.ir)["moe_g_w"][1]
        best, _, lg = model.last_routing(wl.rows, E)
        routing = routing_report(best, lg, E)
    model.free()
    work = {"c3": c3_work, "c4": c4_work}.get(key, lambda: {})()
    kernels = {}
    for k, v in prof.items():
        ms = v["ms"] / steps
        e = {"ms_per_step": ms, "calls_per_step": v["calls"] / steps}
        if k in work:
            if k in ("embedding", "layernorm"):  # work = bytes read + written
                e["GB/s"] = work[k] / (ms * 1e-3) / 1e9
            else:
                e["TFLOP/s"] = work[k] / (ms * 1e-3) / 1e12
        kernels[k] = e
    region = DOMINANT[key][0]
    out = {"metric": METRIC, "value": wl.rows * steps / dt, "unit": "tokens/s", "n_gpus": 1, "steps": steps,
           "warmup": warmup, "ms_per_step": dt * 1e3 / steps, "higher_is_better": True, "scaling": "weak",
           "vs_baseline": None, "dtype": "f32", "data": "synthetic",
           "config": {"workload": f"{key}: {wl.desc}", "tokens": wl.rows, "entry": "nsh_eval_infer_device"},
           "roofline": roofline_of(key, region, work[region],
                                   prof[region]["ms"] / prof[region]["calls"]),
           "kernels": kernels}
    out["host_abi"] = {"tokens_per_s": wl.rows / abi_dt, "ms": abi_dt * 1e3,
                       "note": "ns_eval_infer with host buffers (PCIe-inclusive)"}
    if routing is not None:
        out["routing"] = routing
    return out


def c5_work(M=16384, D=512, H=8, V=8192, FF=2048, C=8192):
    """Algorithmic FLOP of one c5 training step (attention counted once)."""
    dense_fwd = 2.0 * M * (4 * D * D + D * FF + FF * D + D * C)
    return {"dense": 3 * dense_fwd, "attention": 4.0 * M * M * D * 3, "attention_bwd": 8.0 * M * M * D,
            "total": 3 * dense_fwd + 12.0 * M * M * D}


def c5_hbm_bytes(n_muon, M=16384, D=512, C=8192):
    """Algorithmic HBM bytes per step of c5's bandwidth-bound regions: CE reads
    the logits and the one-hot labels and writes the gradient ([M, C] each);
    the Muon gather reads g and writes its transpose, the update reads the q
    vectors and w and writes w (n_muon elements each); embedding and LayerNorm
    read and write [M, D] (LayerNorm's gradient also reads x)."""
    return {"softmax_xent": 3.0 * M * C * 4, "muon_gather": 2.0 * n_muon * 4, "muon_update": 3.0 * n_muon * 4,
            "embedding": 2.0 * M * D * 4, "layernorm": 2.0 * M * D * 4, "layernorm_grad": 3.0 * M * D * 4}


def adamw_bandwidth(n, launches=20):
    """The AdamW kernel (nsh_op_adamw_step) over n parameters, as if every
    weight of the step took AdamW: 4 arrays read, 3 written (28 bytes per
    parameter), timed over `launches` back-to-back launches."""
    import ctypes
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


def bench_train(key, steps, warmup):
    """Device-resident training steps of config `key` (nsh_train_step_device);
    lr = 3e-4 times the cosine-warmup multiplier, as the host applies it."""
    from neuralscript_amd import runtime, workloads
    if not runtime.has_gpu():
        raise SystemExit("bench.py: no GPU visible to libnship")
    wl = workloads.CONFIGS[key]
    plan = runtime.Plan.load(wl.net)
    w = workloads.weights(key, plan.layout(), workloads.ir_shapes(plan.ir))
    dx = runtime.DeviceArray.from_host(workloads.inputs(key))
    dy = runtime.DeviceArray.from_host(workloads.labels(key))
    model = runtime.Model(plan, w)
    scale = lambda t: min(1.0, t / 100.0)  # noqa: E731  (warmup ramp; t < 100 here)
    t = 0
    for _ in range(warmup):
        model.train_step_device(dx, dy, 3e-4 * scale(t), want_loss=False)
        t += 1
    model.sync()
    model.profile(True)
    model.profile_reset()
    t0 = time.perf_counter()
    for _ in range(steps):
        model.train_step_device(dx, dy, 3e-4 * scale(t), want_loss=False)
        t += 1
    model.sync()
    dt = time.perf_counter() - t0
    prof = model.profile_report()
    model.profile(False)
    loss = model.train_step_device(dx, dy, 3e-4 * scale(t))
    t += 1
    # host-pointer ABI (ns_runtime_train_step: the [M, C] one-hot labels cross
    # PCIe every call), for reference
    xh, yh = workloads.inputs(key), workloads.labels(key)
    t0 = time.perf_counter()
    for _ in range(2):
        model.train_step(xh, yh, 3e-4 * scale(t))
        t += 1
    abi_dt = (time.perf_counter() - t0) / 2
    model.free()
    work = c5_work()
    shapes = workloads.ir_shapes(plan.ir)
    # Muon matrices (codegen.cpp:3097): every 2-D weight with min(r, c) >= 8
    n_muon = sum(int(np.prod(v)) for v in shapes.values() if len(v) == 2 and min(v) >= 8)
    hbm = c5_hbm_bytes(n_muon)
    kernels = {}
    for k, v in prof.items():
        ms = v["ms"] / steps
        e = {"ms_per_step": ms, "calls_per_step": v["calls"] / steps}
        if k in hbm:
            e["GB/s"] = hbm[k] / (ms * 1e-3) / 1e9
            e["hbm_frac"] = e["GB/s"] / HBM_PEAK_GBS
        kernels[k] = e
    att = prof["attention_bwd"]
    return {"metric": METRIC, "value": steps / dt, "unit": "steps/s", "n_gpus": 1, "steps": steps, "warmup": warmup,
            "ms_per_step": dt * 1e3 / steps, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": "f32", "data": "synthetic",
            "config": {"workload": f"{key}: {wl.desc}", "tokens": wl.rows, "entry": "nsh_train_step_device"},
            "achieved_TFLOP/s": work["total"] / (dt / steps) / 1e12, "last_loss": float(loss),
            "roofline": roofline_of(key, "attention_bwd", work["attention_bwd"], att["ms"] / att["calls"]),
            "kernels": kernels, "adamw": adamw_bandwidth(n_muon),
            "host_abi": {"steps_per_s": 1.0 / abi_dt, "ms": abi_dt * 1e3,
                         "note": "ns_runtime_train_step with host buffers (labels uploaded every call)"}}


def bench_c2(steps, warmup, with_cpu):
    from neuralscript_amd import runtime, workloads
    if not runtime.has_gpu():
        raise SystemExit("bench.py: no GPU visible to libnship")
    rows = workloads.CONFIGS["c2"].rows
    plan = runtime.Plan.load("c2")
    shapes = workloads.ir_shapes(plan.ir)
    w = workloads.weights("c2", plan.layout(), shapes)
    x = workloads.inputs("c2")
    model = runtime.Model(plan, w)
    dx = runtime.DeviceArray.from_host(x)
    dy = runtime.DeviceArray(rows * 1024)
    for _ in range(warmup):
        model.eval_infer_device(dx, dy)
    model.sync()
    # timed region: K forward steps, per-launch HIP events on the model stream
    model.profile(True)
    model.profile_reset()
    model.sync()
    t0 = time.perf_counter()
    for _ in range(steps):
        model.eval_infer_device(dx, dy)
    model.sync()
    dt = time.perf_counter() - t0
    prof = model.profile_report()
    model.profile(False)
    out = dy.to_host()
    if not np.isfinite(out).all():
        raise SystemExit("bench.py: non-finite output")
    # host-pointer ABI rate (PCIe-inclusive), for reference only
    t0 = time.perf_counter()
    for _ in range(3):
        model.eval_infer(x)
    abi_dt = (time.perf_counter() - t0) / 3

    gemm_calls = sum(v["calls"] for k, v in prof.items() if k.startswith("gemm"))
    gemm_ms = sum(v["ms"] for k, v in prof.items() if k.startswith("gemm"))
    per_launch_ms = gemm_ms / max(gemm_calls, 1)
    flop_per_launch = c2_flops(rows) / 3.0
    achieved = flop_per_launch / (per_launch_ms * 1e-3) / 1e12
    res = {
        "metric": METRIC,
        "value": rows * steps / dt,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": dt * 1e3 / steps,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "c2: " + workloads.CONFIGS["c2"].desc, "batch": rows,
                   "layers": "1024->4096->4096->1024", "entry": "nsh_eval_infer_device"},
        "roofline": {"bound": "mfma", "kernel": "gemm_f32_kernel", "achieved": achieved,
                     "peak": MFMA_F32_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": achieved / MFMA_F32_PEAK_TFLOPS,
                     "flop_per_launch": flop_per_launch, "avg_launch_ms": per_launch_ms,
                     "launches": gemm_calls, "traffic": load_traffic("gemm_f32_kernel")},
        "host_abi": {"tokens_per_s": rows / abi_dt, "note": "ns_eval_infer with host buffers (PCIe-inclusive)"},
    }
    model.free()
    res["measured_peak"] = measured_peaks()
    res["roofline"]["frac_of_measured_peak"] = achieved / res["measured_peak"]["mfma_f32_tflops"]
    if with_cpu:
        res["cpu_baseline"] = cpu_baseline_c2()
    return res


def measured_peaks():
    """Attainable peaks of this GPU, measured by libnship's microbenchmarks:
    a register-only fp32 MFMA loop (2048 workgroups x 4 waves, 4 independent
    32x32x2 chains per wave) and a float4 copy of 256 MiB each way."""
    import ctypes
    from neuralscript_amd import runtime
    lib = runtime.lib()
    tf = ctypes.c_double()
    runtime.check(lib.nsh_bench_mfma_peak(4000, 2048, ctypes.byref(tf)), "bench_mfma_peak")
    n = 1 << 26
    src, dst = runtime.DeviceArray(n), runtime.DeviceArray(n)
    src.fill_zero()
    dst.fill_zero()
    gbs = ctypes.c_double()
    runtime.check(lib.nsh_bench_copy(src.ptr, dst.ptr, n, 10, ctypes.byref(gbs)), "bench_copy")
    src.free()
    dst.free()
    return {"mfma_f32_tflops": tf.value, "mfma_frac_of_published": tf.value / MFMA_F32_PEAK_TFLOPS,
            "hbm_copy_gbs": gbs.value, "hbm_frac_of_published": gbs.value / HBM_PEAK_GBS}


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


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="c2", choices=["c2", "c3", "c4", "c5", "copy", "peak"],
                    help="c2 (default) is the metric's workload; c3/c4 (forward) and c5 (training steps) "
                         "print per-kernel breakdowns; copy runs the rocprof counter calibration copy; peak "
                         "measures the attainable MFMA / HBM peaks and the vendor library's fp32 GEMM")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    a = ap.parse_args()
    if a.gpus != 1:
        raise SystemExit("bench.py: this build measures one GPU only (the path runs on one GPU; "
                         "--gpus must be 1)")
    if a.config == "copy":
        res = copy_calibration()
    elif a.config == "peak":
        res = bench_peak()
    elif a.config == "c2":
        res = bench_c2(a.steps, a.warmup, not a.no_cpu_baseline)
    elif a.config == "c5":
        res = bench_train(a.config, a.steps, a.warmup)
    else:
        res = bench_forward(a.config, a.steps, a.warmup)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
