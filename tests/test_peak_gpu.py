"""The attainable-peak microbenchmarks behind bench.py's `measured_peak`:
the copy copies, both report rates within physical bounds, and bad
arguments are rejected."""
import ctypes

import numpy as np
import pytest

from neuralscript_amd import runtime, synth
from neuralscript_amd.runtime import DeviceArray as DA

pytestmark = pytest.mark.gpu


def test_mfma_peak_reports_a_plausible_rate():
    tf = ctypes.c_double()
    runtime.check(runtime.lib().nsh_bench_mfma_peak(200, 1024, ctypes.byref(tf)), "bench_mfma_peak")
    print(f"fp32 MFMA: {tf.value:.1f} TFLOP/s")
    assert 10.0 < tf.value < 200.0  # published dense fp32 MFMA peak 157.3


def test_copy_copies_and_reports_a_plausible_rate():
    n = 1 << 22
    x = synth.normal(5, n)
    src, dst = DA.from_host(x), DA(n)
    gbs = ctypes.c_double()
    runtime.check(runtime.lib().nsh_bench_copy(src.ptr, dst.ptr, n, 3, ctypes.byref(gbs)), "bench_copy")
    print(f"copy: {gbs.value:.0f} GB/s")
    assert np.array_equal(dst.to_host(), x)
    assert 100.0 < gbs.value < 10000.0  # published HBM peak 8 TB/s


def test_bad_arguments_are_rejected():
    L = runtime.lib()
    d = ctypes.c_double()
    assert L.nsh_bench_mfma_peak(0, 1, ctypes.byref(d)) == -1
    a = DA(8)
    assert L.nsh_bench_copy(a.ptr, a.ptr + 4, 4, 1, ctypes.byref(d)) == -1  # misaligned
    assert L.nsh_bench_copy(a.ptr, a.ptr, 6, 1, ctypes.byref(d)) == -1      # n % 4
