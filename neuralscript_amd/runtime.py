"""Host-side binding of libnship (include/nship.h) via ctypes.

There is no fallback: if libnship.so is missing this module raises, so a
product path can never silently run on the CPU.
"""
from __future__ import annotations

import ctypes
import glob
import os

import numpy as np

from .abi import NsLib, WeightLayout

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG, "libnship.so")
NETS = os.path.join(PKG, "nets")

_f32p = ctypes.POINTER(ctypes.c_float)
_lib = None


class NshipError(RuntimeError):
    pass


def lib():
    """libnship, loaded once (RTLD_GLOBAL so per-network drivers bind to it)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise NshipError(f"libnship.so not built: {LIB_PATH} (run `python -m neuralscript_amd.build`)")
        L = ctypes.CDLL(LIB_PATH, mode=ctypes.RTLD_GLOBAL)
        vp, sz, ci, cf, i64 = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_float, ctypes.c_int64
        sigs = {
            "nsh_last_error": (ctypes.c_char_p, []),
            "nsh_device_count": (ci, []),
            "nsh_dev_alloc": (vp, [sz]),
            "nsh_dev_free": (ci, [vp]),
            "nsh_memcpy_h2d": (ci, [vp, vp, sz]),
            "nsh_memcpy_d2h": (ci, [vp, vp, sz]),
            "nsh_memset_d": (ci, [vp, ci, sz]),
            "nsh_device_synchronize": (ci, []),
            "nsh_plan_parse": (vp, [ctypes.c_char_p]),
            "nsh_plan_free": (None, [vp]),
            "nsh_plan_weight_count": (sz, [vp]),
            "nsh_plan_layout": (ctypes.POINTER(WeightLayout), [vp]),
            "nsh_plan_output_numel": (sz, [vp, sz]),
            "nsh_plan_has_train": (ci, [vp]),
            "nsh_plan_has_moe": (ci, [vp]),
            "nsh_plan_in_cols": (sz, [vp]),
            "nsh_plan_out_cols": (sz, [vp]),
            "nsh_model_init": (vp, [vp, _f32p, sz]),
            "nsh_model_free": (None, [vp]),
            "nsh_eval_infer": (ci, [vp, _f32p, _f32p, sz]),
            "nsh_eval_infer_device": (ci, [vp, vp, vp, sz]),
            "nsh_model_sync": (ci, [vp]),
            "nsh_model_weight_count": (sz, [vp]),
            "nsh_model_get_weights": (ci, [vp, _f32p, sz]),
            "nsh_save_checkpoint": (ci, [vp, ctypes.c_char_p]),
            "nsh_load_checkpoint": (ci, [vp, ctypes.c_char_p]),
            "nsh_expert_count": (sz, [vp]),
            "nsh_expert_birth": (sz, [vp, ci]),
            "nsh_expert_merge": (sz, [vp, ci, ci]),
            "nsh_expert_kill": (sz, [vp, ci]),
            "nsh_train_step": (ci, [vp, _f32p, _f32p, sz, _f32p, cf]),
            "nsh_objective_loss": (ci, [vp, _f32p, _f32p, sz, _f32p]),
            "nsh_profile_enable": (ci, [vp, ci]),
            "nsh_profile_reset": (ci, [vp]),
            "nsh_profile_select": (ci, [vp, ctypes.c_char_p]),
            "nsh_profile_report": (ci, [vp, ctypes.c_char_p, sz]),
            "nsh_op_gemm": (ci, [vp, vp, vp, i64, i64, i64, i64, i64, i64, ci, ci, ci]),
            "nsh_op_attention_bwd_workspace": (sz, [i64, i64, i64, ci]),
            "nsh_op_attention_bwd": (ci, [vp, vp, vp, vp, vp, vp, vp, vp, vp, i64, i64, i64, ci, vp]),
            "nsh_op_gemm_splitk_workspace": (sz, [i64, i64, i64, ci]),
            "nsh_op_gemm_splitk": (ci, [vp, vp, vp, i64, i64, i64, i64, i64, i64, ci, ci, ci, ci, vp]),
            "nsh_model_last_routing": (ci, [vp, vp, vp, vp, sz]),
            "nsh_train_step_device": (ci, [vp, vp, vp, sz, _f32p, cf]),
            "nsh_model_read_value": (ci, [vp, ctypes.c_char_p, vp, sz]),
            "nsh_op_muon_workspace": (sz, [i64, i64]),
            "nsh_op_orthonormalize": (ci, [vp, vp, i64, i64, vp]),
            "nsh_op_muon_step": (ci, [vp, vp, i64, i64, cf, vp]),
            "nsh_op_adamw_step": (ci, [vp, vp, vp, vp, i64, i64, cf]),
            "nsh_bench_mfma_peak": (ci, [ci, ci, ctypes.POINTER(ctypes.c_double)]),
            "nsh_bench_copy": (ci, [vp, vp, i64, ci, ctypes.POINTER(ctypes.c_double)]),
            "nsh_bench_rowops": (ci, [vp, vp, i64, i64, i64, i64, ci, ctypes.POINTER(ctypes.c_double)]),
            "nsh_op_muon_multi_workspace": (sz, [ci, vp, vp]),
            "nsh_op_muon_multi": (ci, [ci, vp, vp, vp, vp, cf, vp]),
            "nsh_op_embedding": (ci, [vp, vp, vp, i64, i64, i64]),
            "nsh_op_layernorm": (ci, [vp, vp, i64, i64]),
            "nsh_op_layernorm_grad": (ci, [vp, vp, vp, i64, i64]),
            "nsh_op_softmax_xent": (ci, [vp, vp, vp, vp, vp, i64, i64]),
            "nsh_op_act_grad": (ci, [vp, vp, vp, i64, ci]),
            "nsh_op_embedding_grad_workspace": (sz, [i64, i64]),
            "nsh_op_embedding_grad": (ci, [vp, vp, vp, i64, i64, i64, vp]),
            "nsh_op_embedding_grad_noalloc": (ci, [vp, vp, vp, i64, i64, i64, vp]),
            "nsh_op_attention_fwd": (ci, [vp, vp, vp, vp, vp, i64, i64, i64]),
        }
        for name, (res, args) in sigs.items():
            fn = getattr(L, name)
            fn.restype, fn.argtypes = res, args
        _lib = L
    return _lib


def last_error():
    return lib().nsh_last_error().decode(errors="replace")


def check(rc, what):
    if rc != 0:
        raise NshipError(f"{what} failed: {last_error()}")


def has_gpu():
    return lib().nsh_device_count() > 0


class DeviceArray:
    """A float32 (or raw byte) device buffer owned by libnship's allocator."""

    def __init__(self, n, dtype=np.float32):
        self.dtype = np.dtype(dtype)
        self.n = int(n)
        self.nbytes = self.n * self.dtype.itemsize
        self.ptr = lib().nsh_dev_alloc(self.nbytes)
        if not self.ptr:
            raise NshipError(f"device alloc of {self.nbytes} bytes failed: {last_error()}")

    @classmethod
    def from_host(cls, a, dtype=np.float32):
        a = np.ascontiguousarray(a, dtype=dtype).ravel()
        d = cls(a.size, dtype)
        check(lib().nsh_memcpy_h2d(d.ptr, a.ctypes.data, d.nbytes), "h2d")
        return d

    def to_host(self, n=None):
        n = self.n if n is None else int(n)
        out = np.empty(n, dtype=self.dtype)
        check(lib().nsh_memcpy_d2h(out.ctypes.data, self.ptr, n * self.dtype.itemsize), "d2h")
        return out

    def fill_zero(self):
        check(lib().nsh_memset_d(self.ptr, 0, self.nbytes), "memset")

    def free(self):
        if self.ptr:
            lib().nsh_dev_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Plan:
    """A parsed network (IR text of `nsc --mlir`)."""

    def __init__(self, ir_text):
        self.ir = ir_text
        self.h = lib().nsh_plan_parse(ir_text.encode())
        if not self.h:
            raise NshipError(last_error())

    @classmethod
    def load(cls, name):
        with open(os.path.join(NETS, name + ".mlir")) as f:
            return cls(f.read())

    @property
    def weight_count(self):
        return lib().nsh_plan_weight_count(self.h)

    def layout(self):
        lay = lib().nsh_plan_layout(self.h).contents
        return [(lay.desc[i].name.decode(), lay.desc[i].offset, lay.desc[i].count)
                for i in range(lay.num_weights)]

    def output_numel(self, n):
        return lib().nsh_plan_output_numel(self.h, n)

    @property
    def in_cols(self):
        return lib().nsh_plan_in_cols(self.h)

    @property
    def out_cols(self):
        return lib().nsh_plan_out_cols(self.h)

    def __del__(self):
        try:
            if self.h:
                lib().nsh_plan_free(self.h)
        except Exception:
            pass


class Model:
    """A model on the GPU, driven through the nsh_* entry points."""

    def __init__(self, plan: Plan, weights):
        self.plan = plan
        w = np.ascontiguousarray(weights, dtype=np.float32).ravel()
        self.h = lib().nsh_model_init(plan.h, w.ctypes.data_as(_f32p), w.size)
        if not self.h:
            raise NshipError(last_error())

    def eval_infer(self, x, out=None):
        """ns_eval_infer on host arrays; `out` (float32, contiguous, at least
        output_numel floats) is written in place when given."""
        x = np.ascontiguousarray(x, dtype=np.float32).ravel()
        n = self.plan.output_numel(x.size)
        if out is None:
            out = np.empty(n, dtype=np.float32)
        elif out.dtype != np.float32 or not out.flags.c_contiguous or out.size < n:
            raise NshipError("eval_infer: out must be contiguous float32 with room for the output")
        check(lib().nsh_eval_infer(self.h, x.ctypes.data_as(_f32p), out.ctypes.data_as(_f32p), x.size),
              "eval_infer")
        return out

    def eval_infer_device(self, d_x: DeviceArray, d_out: DeviceArray, n=None):
        check(lib().nsh_eval_infer_device(self.h, d_x.ptr, d_out.ptr, d_x.n if n is None else n),
              "eval_infer_device")

    def sync(self):
        check(lib().nsh_model_sync(self.h), "sync")

    def get_weights(self):
        out = np.empty(self.plan.weight_count, dtype=np.float32)
        check(lib().nsh_model_get_weights(self.h, out.ctypes.data_as(_f32p), out.size), "get_weights")
        return out

    def train_step(self, x, labels, lr):
        x = np.ascontiguousarray(x, dtype=np.float32).ravel()
        y = np.ascontiguousarray(labels, dtype=np.float32).ravel()
        loss = np.zeros(1, dtype=np.float32)
        check(lib().nsh_train_step(self.h, x.ctypes.data_as(_f32p), y.ctypes.data_as(_f32p), x.size,
                                   loss.ctypes.data_as(_f32p), ctypes.c_float(lr)), "train_step")
        return loss[0]

    def train_step_device(self, d_x: DeviceArray, d_y: DeviceArray, lr, want_loss=True):
        loss = np.zeros(1, dtype=np.float32)
        check(lib().nsh_train_step_device(self.h, d_x.ptr, d_y.ptr, d_x.n,
                                          loss.ctypes.data_as(_f32p) if want_loss else None,
                                          ctypes.c_float(lr)), "train_step_device")
        return loss[0]

    def objective_loss(self, x, labels):
        x = np.ascontiguousarray(x, dtype=np.float32).ravel()
        y = np.ascontiguousarray(labels, dtype=np.float32).ravel()
        loss = np.zeros(1, dtype=np.float32)
        check(lib().nsh_objective_loss(self.h, x.ctypes.data_as(_f32p), y.ctypes.data_as(_f32p), x.size,
                                       loss.ctypes.data_as(_f32p)), "objective_loss")
        return loss[0]

    def read_value(self, name, n):
        out = np.empty(n, dtype=np.float32)
        check(lib().nsh_model_read_value(self.h, name.encode(), out.ctypes.data, n), "read_value " + name)
        return out

    def last_routing(self, n, E):
        best = np.empty(n, dtype=np.int32)
        prob = np.empty(n, dtype=np.float32)
        lg = np.empty(n * E, dtype=np.float32)
        check(lib().nsh_model_last_routing(self.h, best.ctypes.data, prob.ctypes.data, lg.ctypes.data, n),
              "last_routing")
        return best, prob, lg

    def profile(self, on=True):
        check(lib().nsh_profile_enable(self.h, 1 if on else 0), "profile_enable")

    def profile_reset(self):
        check(lib().nsh_profile_reset(self.h), "profile_reset")

    def profile_select(self, regions=None):
        """Time only the named profile regions (None: every region)."""
        arg = ",".join(regions).encode() if regions else None
        check(lib().nsh_profile_select(self.h, arg), "profile_select")

    def profile_report(self):
        import json
        buf = ctypes.create_string_buffer(1 << 16)
        check(lib().nsh_profile_report(self.h, buf, len(buf)), "profile_report")
        return json.loads(buf.value.decode())

    def free(self):
        if self.h:
            lib().nsh_model_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def net_lib(name) -> NsLib:
    """The per-network ns_* driver (built by neuralscript_amd.build)."""
    lib()  # libnship first, globally, so the driver resolves against it
    path = os.path.join(NETS, f"lib{name}.so")
    if not os.path.exists(path):
        raise NshipError(f"network driver not built: {path}")
    return NsLib(path)


def bundled_nets():
    return sorted(os.path.splitext(os.path.basename(p))[0] for p in glob.glob(os.path.join(NETS, "*.mlir")))


def gemm(dA, dB, dC, M, N, K, lda, ldb, ldc, transA=False, transB=False, act=0):
    check(lib().nsh_op_gemm(dA.ptr, dB.ptr, dC.ptr, M, N, K, lda, ldb, ldc, int(transA), int(transB), act),
          "gemm")


def gemm_splitk(dA, dB, dC, M, N, K, lda, ldb, ldc, transA=False, transB=False, act=0, splits=0):
    """nsh_op_gemm_splitk with a workspace of its own (splits 0: heuristic)."""
    nb = lib().nsh_op_gemm_splitk_workspace(M, N, K, splits)
    ws = DeviceArray(max(1, (nb + 3) // 4))
    check(lib().nsh_op_gemm_splitk(dA.ptr, dB.ptr, dC.ptr, M, N, K, lda, ldb, ldc, int(transA), int(transB), act,
                                   splits, ws.ptr), "gemm_splitk")


def _p(d):
    return d.ptr if d is not None else None


def op(name, *args):
    """Call nsh_op_<name> with DeviceArray / scalar arguments."""
    conv = [_p(a) if isinstance(a, DeviceArray) or a is None else a for a in args]
    check(getattr(lib(), "nsh_op_" + name)(*conv), name)
