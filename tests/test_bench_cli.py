"""bench.py's command-line contract on the CPU: more than one GPU is refused
with a message before anything touches a GPU."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_more_than_one_gpu_is_refused_with_a_message():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode != 0
    assert "one GPU" in (r.stderr + r.stdout)


def test_kernel_table_keeps_distinct_kernels_apart():
    """A region's rate covers its own variants only: `layernorm` does not
    absorb `layernorm_grad`, while `gemm` and `gemm_act` are summed."""
    sys.path.insert(0, ROOT)
    import bench
    prof = {"layernorm": {"ms": 1.0, "calls": 1}, "layernorm_grad": {"ms": 3.0, "calls": 1},
            "gemm": {"ms": 2.0, "calls": 2}, "gemm_act": {"ms": 2.0, "calls": 2}, "_steps": 1}
    assert bench._group(prof, "layernorm") == ["layernorm"]
    assert bench._group(prof, "gemm") == ["gemm", "gemm_act"]
    t = bench.kernel_table(prof, 1, {"gemm": 4e9}, {"layernorm": 8e6, "layernorm_grad": 12e6})
    assert abs(t["layernorm"]["GB/s"] - 8.0) < 1e-9
    assert abs(t["layernorm_grad"]["GB/s"] - 4.0) < 1e-9
    assert abs(t["gemm (all variants)"]["TFLOP/s"] - 1.0) < 1e-9
