"""ctypes binding of the NeuralScript runtime C-ABI.

Mirrors /root/reference/include/ns/runtime/ns_runtime.h:30-129 function for
function (same names, argument meaning and 0 / -1 / NULL error convention).
Any shared library exporting that ABI can be driven through ``NsLib``: the
per-network libraries built on libnship, and equally a driver emitted by the
reference compiler.
"""
from __future__ import annotations

import ctypes

import numpy as np

_f32p = ctypes.POINTER(ctypes.c_float)


class WeightDesc(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("offset", ctypes.c_size_t), ("count", ctypes.c_size_t)]


class WeightLayout(ctypes.Structure):
    _fields_ = [("num_weights", ctypes.c_size_t), ("desc", ctypes.POINTER(WeightDesc))]


def _fp(a):
    if a is None:
        return None
    if a.dtype != np.float32 or not a.flags.c_contiguous:
        raise TypeError("expected a C-contiguous float32 array")
    return a.ctypes.data_as(_f32p)


class NsLib:
    """One loaded model library (the ABI has one network per library)."""

    def __init__(self, path, mode=ctypes.RTLD_LOCAL):
        self.path = path
        L = ctypes.CDLL(path, mode=mode)
        vp, sz, ci, cf = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_float
        sigs = {
            "ns_runtime_init": (vp, [_f32p, sz]),
            "ns_eval_infer": (ci, [vp, _f32p, _f32p, sz]),
            "ns_model_output_numel": (sz, [vp, sz]),
            "ns_model_weight_count": (sz, [vp]),
            "ns_weight_count_static": (sz, []),
            "ns_model_get_weights": (ci, [vp, _f32p, sz]),
            "ns_model_layout": (ctypes.POINTER(WeightLayout), [vp]),
            "ns_free": (None, [vp]),
            "ns_save_checkpoint": (ci, [vp, ctypes.c_char_p]),
            "ns_load_checkpoint": (ci, [vp, ctypes.c_char_p]),
        }
        optional = {
            "ns_runtime_train_step": (ci, [vp, _f32p, _f32p, sz, _f32p, cf]),
            "ns_objective_loss": (ci, [vp, _f32p, _f32p, sz, _f32p]),
            "ns_expert_count": (sz, [vp]),
            "ns_expert_birth": (sz, [vp, ci]),
            "ns_expert_merge": (sz, [vp, ci, ci]),
            "ns_expert_kill": (sz, [vp, ci]),
            "ns_train_core": (None, [vp, _f32p, sz, _f32p, _f32p, _f32p, _f32p, cf, ci]),
        }
        for name, (res, args) in sigs.items():
            fn = getattr(L, name)
            fn.restype, fn.argtypes = res, args
        self.has = set()
        for name, (res, args) in optional.items():
            if hasattr(L, name):
                fn = getattr(L, name)
                fn.restype, fn.argtypes = res, args
                self.has.add(name)
        self.lib = L
        # the emitted TU's entry function (codegen.cpp:2263-2265); MoE
        # networks take the liveness mask as a fifth argument
        self.moe = "ns_expert_count" in self.has
        self.forward_fn = getattr(L, "forward", None)
        if self.forward_fn is not None:
            self.forward_fn.restype = None
            self.forward_fn.argtypes = [_f32p, _f32p, _f32p, sz] + ([ctypes.c_void_p] if self.moe else [])

    def weight_count_static(self):
        return self.lib.ns_weight_count_static()

    def layout(self, model=None):
        lay = self.lib.ns_model_layout(model)
        return [(lay.contents.desc[i].name.decode(), lay.contents.desc[i].offset,
                 lay.contents.desc[i].count) for i in range(lay.contents.num_weights)]

    def init(self, weights):
        w = np.ascontiguousarray(weights, dtype=np.float32)
        return self.lib.ns_runtime_init(_fp(w), w.size)

    def free(self, m):
        self.lib.ns_free(m)

    def output_numel(self, m, n):
        return self.lib.ns_model_output_numel(m, n)

    def eval_infer(self, m, x):
        x = np.ascontiguousarray(x, dtype=np.float32).ravel()
        out = np.empty(self.output_numel(m, x.size), dtype=np.float32)
        rc = self.lib.ns_eval_infer(m, _fp(x), _fp(out), x.size)
        if rc != 0:
            raise RuntimeError(f"ns_eval_infer returned {rc}")
        return out

    def get_weights(self, m, n=None):
        n = self.lib.ns_model_weight_count(m) if n is None else n
        out = np.empty(n, dtype=np.float32)
        rc = self.lib.ns_model_get_weights(m, _fp(out), n)
        if rc != 0:
            raise RuntimeError(f"ns_model_get_weights returned {rc}")
        return out

    def train_step(self, m, x, labels, lr):
        x = np.ascontiguousarray(x, dtype=np.float32).ravel()
        y = np.ascontiguousarray(labels, dtype=np.float32).ravel()
        loss = np.zeros(1, dtype=np.float32)
        rc = self.lib.ns_runtime_train_step(m, _fp(x), _fp(y), x.size, _fp(loss),
                                            ctypes.c_float(lr))
        if rc != 0:
            raise RuntimeError(f"ns_runtime_train_step returned {rc}")
        return loss[0]

    def objective_loss(self, m, x, labels):
        x = np.ascontiguousarray(x, dtype=np.float32).ravel()
        y = np.ascontiguousarray(labels, dtype=np.float32).ravel()
        loss = np.zeros(1, dtype=np.float32)
        rc = self.lib.ns_objective_loss(m, _fp(x), _fp(y), x.size, _fp(loss))
        if rc != 0:
            raise RuntimeError(f"ns_objective_loss returned {rc}")
        return loss[0]

    def save(self, m, path):
        return self.lib.ns_save_checkpoint(m, path.encode())

    def load(self, m, path):
        return self.lib.ns_load_checkpoint(m, path.encode())

    def forward(self, x, weights, out_numel, moe_active=None):
        """The entry function `forward(input, weights, output, n[,
        moe_active])`: weights passed with the call; out_numel floats of
        output (pre-filled with NaN, so unwritten elements show)."""
        x = np.ascontiguousarray(x, dtype=np.float32).ravel()
        w = np.ascontiguousarray(weights, dtype=np.float32).ravel()
        out = np.full(out_numel, np.nan, dtype=np.float32)
        args = [_fp(x), _fp(w), _fp(out), x.size]
        if self.moe:
            mask = None if moe_active is None else np.ascontiguousarray(moe_active, dtype=np.uint8)
            args.append(None if mask is None else mask.ctypes.data)
        self.forward_fn(*args)
        return out

    def train_core(self, ctx, x, labels, weights, lr, train_mode, write_back=True):
        """`ns_train_core(ctx, x, nx, y, w, wout, loss_out, lr, train_mode)`
        (codegen.cpp:2753-2755) with w = `weights`: (loss, wout or None)."""
        x = np.ascontiguousarray(x, dtype=np.float32).ravel()
        y = np.ascontiguousarray(labels, dtype=np.float32).ravel()
        w = np.ascontiguousarray(weights, dtype=np.float32).ravel()
        wout = np.full(w.size, np.nan, dtype=np.float32) if write_back else None
        loss = np.full(1, np.nan, dtype=np.float32)
        self.lib.ns_train_core(ctx, _fp(x), x.size, _fp(y), _fp(w), _fp(wout), _fp(loss), ctypes.c_float(lr),
                               int(train_mode))
        return loss[0], wout


class _RefModel(ctypes.Structure):
    """The reference CPU driver's model struct (codegen.cpp:2438)."""
    _fields_ = [("w", ctypes.c_void_p), ("n", ctypes.c_size_t), ("ctx", ctypes.c_void_p)]


def reference_ctx(model):
    """The ns_cpu_ctx of a model made by a reference-emitted CPU driver (its
    ns_train_core takes the context, not the model)."""
    return ctypes.cast(ctypes.c_void_p(model), ctypes.POINTER(_RefModel)).contents.ctx
