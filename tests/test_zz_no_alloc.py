"""The allocation-free embedding-gradient entry point
(nsh_op_embedding_grad_noalloc: scratch in a static device array) against
the workspace entry point nsh_op_embedding_grad and the oracle, bit for bit,
on two calls in a row (the second smaller, so it runs over the first call's
leftover scratch) beyond 32768 tokens, where the counting sort uses the
array, and two up to 32768, where one launch needs no scratch; plus its size
limit."""
import numpy as np
import pytest

import oracle
from neuralscript_amd import runtime, synth

pytestmark = pytest.mark.gpu

MAX_INTS = 1048576  # NSH_EMBEDDING_GRAD_NOALLOC_MAX_INTS (include/nship.h)


def _ids(seed, n, V):
    """Uniform ids with a hot id repeated well past 32 times (the workgroup
    rank path of the segment sort), out-of-range ids (skipped) and
    fractional ids (truncated)."""
    ids = synth.token_ids(synth.stream_seed(seed, "ids"), n, V).astype(np.float32)
    rng = np.random.default_rng(seed)
    hot = rng.choice(n, size=min(n // 4, 400), replace=False)
    ids[hot] = np.float32(V // 3)
    special = np.array([-1.0, V, V + 5.0, -0.5, V - 0.5, 1.75], np.float32)
    pos = rng.choice(n, size=special.size, replace=False)
    ids[pos] = special
    return ids


def _both(n, V, D, seed):
    lib = runtime.lib()
    dout = synth.normal(seed, n * D)
    ids = _ids(seed, n, V)
    d_dout, d_ids = runtime.DeviceArray.from_host(dout), runtime.DeviceArray.from_host(ids)
    dW_ws, dW_na = runtime.DeviceArray(V * D), runtime.DeviceArray(V * D)
    ws = runtime.DeviceArray(lib.nsh_op_embedding_grad_workspace(n, V), np.uint8)
    print(f"embedding_grad n={n} V={V} D={D}: workspace entry", flush=True)
    runtime.check(lib.nsh_op_embedding_grad(d_dout.ptr, d_ids.ptr, dW_ws.ptr, n, V, D, ws.ptr), "embedding_grad")
    print("  no-alloc entry", flush=True)
    runtime.check(lib.nsh_op_embedding_grad_noalloc(d_dout.ptr, d_ids.ptr, dW_na.ptr, n, V, D, None),
                  "embedding_grad_noalloc")
    runtime.check(lib.nsh_device_synchronize(), "synchronize")
    a, b = dW_ws.to_host(), dW_na.to_host()
    ref = oracle.embedding_grad_w(dout, ids, V, D)
    for d in (d_dout, d_ids, dW_ws, dW_na, ws):
        d.free()
    return a, b, ref


def test_noalloc_matches_workspace_entry_on_two_calls():
    for n, V, D, seed in [(40000, 3000, 32, 13), (35000, 500, 32, 14), (6000, 3000, 96, 11), (700, 500, 32, 12)]:
        a, b, ref = _both(n, V, D, seed)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"n={n} V={V}: no-alloc differs"
        assert np.array_equal(b.view(np.uint32), ref.view(np.uint32)), f"n={n} V={V}: differs from the oracle"


def test_noalloc_rejects_sizes_beyond_its_scratch():
    lib = runtime.lib()
    dW = runtime.DeviceArray(16)
    V = 1000
    n = (MAX_INTS - (3 * V + 1)) // 2 + 1  # one int over
    assert lib.nsh_op_embedding_grad_noalloc(dW.ptr, dW.ptr, dW.ptr, n, V, 16, None) == -1
    assert "exceeds" in runtime.last_error()
    dW.free()
