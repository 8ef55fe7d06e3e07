"""CPU oracle for the NeuralScript emitted runtime (TEST INFRASTRUCTURE ONLY).

Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg
import this module, and only as the checker; the product (libnship) never
does.  It drives ``libns_oracle.so`` (ns_oracle.c, the bit-faithful kernel
restatement) in the order the reference's emitted C++ runs them:

* inference: ``gen_cpu`` forward body, /root/reference/src/codegen/codegen.cpp:1961-2288
* training:  ``emit_train_core``, codegen.cpp:2659-3158 (forward body, then
  reverse body, then the optimizer body, then the loss), wrapped as
  ``ns_runtime_train_step`` at codegen.cpp:2636-2644.

The network comes in as the text of ``nsc <net> --mlir``
(mlir_compiler.cpp:949-1025); this module parses it independently of the
product's C++ parser.
"""
from __future__ import annotations

import ctypes
import os
import re
from dataclasses import dataclass, field

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libns_oracle.so")
# The same kernels in the reference's own loop nests, single-threaded, -O2
# (ns_refloop.c): the CPU baseline, selected with use_reference_order().
REF_LIB_PATH = os.path.join(_HERE, "libns_refloop.so")

ACT_CODES = {"identity": 0, "relu": 1, "leaky_relu": 2, "sigmoid": 3, "tanh": 4,
             "swish": 5, "silu": 5, "gelu": 6}

_f32p = ctypes.POINTER(ctypes.c_float)
_i64p = ctypes.POINTER(ctypes.c_int64)
_u8p = ctypes.POINTER(ctypes.c_uint8)
_libs = {}
_order = "oracle"


def build_command():
    src = os.path.join(_HERE, "ns_oracle.c")
    # -ffp-contract=off: the reference's emitted code never fuses a multiply
    # and an add (g++ -O2 -std=c++11 on x86-64 has no FMA), so neither may we.
    return ["gcc", "-O3", "-march=x86-64-v3", "-ffp-contract=off", "-fno-fast-math",
            "-fopenmp", "-fPIC", "-shared", src, "-o", LIB_PATH, "-lm"]


def build_ref_command():
    """The reference-order library, built as the reference's tests build the
    emitted driver: -O2, baseline x86-64 (no FMA), no threads."""
    src = os.path.join(_HERE, "ns_refloop.c")
    return ["gcc", "-O2", "-ffp-contract=off", "-fno-fast-math", "-fPIC", "-shared", src,
            "-o", REF_LIB_PATH, "-lm"]


def use_reference_order(on=True):
    """Route every kernel wrapper below (and so Model) to the reference-order
    library (True) or back to the checker (False); returns the previous
    setting.  Functions the reference-order library does not restate (the
    MoE backward and routing helpers, the test-only MGS reordering) raise
    while it is selected; the LR multiplier is host arithmetic and always
    comes from the checker."""
    global _order
    prev = _order == "reference"
    _order = "reference" if on else "oracle"
    return prev


def set_mgs_partials(p):
    """Test-only: sum each MGS dot product as p interleaved partial sums
    (p > 1) or as -p contiguous blocks (p < -1); 1 = the reference's order."""
    lib().or_set_mgs_partials(int(p))


def lib():
    return _load(_order)


def _load(which):
    if which not in _libs:
        path = LIB_PATH if which == "oracle" else REF_LIB_PATH
        if not os.path.exists(path):
            raise RuntimeError(f"oracle library missing: {path} (run __graft_entry__.build())")
        L = ctypes.CDLL(path)
        i64, sz, ci, cf = ctypes.c_int64, ctypes.c_size_t, ctypes.c_int, ctypes.c_float
        sig = {
            "or_act": (None, [_f32p, _f32p, sz, ci]),
            "or_act_grad": (None, [_f32p, _f32p, _f32p, sz, ci]),
            "or_matmul": (None, [_f32p, _f32p, _f32p, i64, i64, i64, ci]),
            "or_matmul_rows": (None, [_f32p, _i64p, i64, _f32p, _f32p, i64, i64, ci]),
            "or_matmul_grad_a": (None, [_f32p, _f32p, _f32p, i64, i64, i64]),
            "or_matmul_grad_w": (None, [_f32p, _f32p, _f32p, i64, i64, i64]),
            "or_layernorm": (None, [_f32p, _f32p, sz, i64]),
            "or_softmax": (None, [_f32p, _f32p, sz, i64]),
            "or_layernorm_grad": (None, [_f32p, _f32p, _f32p, sz, i64]),
            "or_embedding": (None, [_f32p, _f32p, _f32p, i64, i64, i64]),
            "or_embedding_rows": (None, [_f32p, _i64p, i64, i64]),
            "or_embedding_grad_w": (None, [_f32p, _f32p, _f32p, sz, i64, i64]),
            "or_cross_entropy": (cf, [_f32p, _f32p, sz, i64]),
            "or_loss_grad": (None, [_f32p, _f32p, _f32p, sz, i64]),
            "or_attention_fwd": (None, [_f32p] * 6 + [i64, i64, i64]),
            "or_attention_fwd_rows": (None, [_f32p] * 5 + [_i64p, i64, _f32p, i64, i64, i64]),
            "or_attention_bwd": (None, [_f32p] * 11 + [i64, i64, i64]),
            "or_moe_gate_logits": (None, [_f32p, _f32p, _f32p, i64, i64, i64]),
            "or_moe_fwd": (None, [_f32p] * 4 + [_u8p, _f32p, _i64p, _f32p, i64, i64, i64, i64]),
            "or_moe_route": (None, [_f32p, _f32p, _u8p, _i64p, _f32p, _f32p, i64, i64, i64]),
            "or_moe_bwd": (None, [_f32p] * 5 + [_u8p] + [_f32p] * 4 + [i64, i64, i64, i64]),
            "or_orthonom": (None, [_f32p, i64, i64]),
            "or_muon_step": (None, [_f32p, _f32p, i64, i64, cf]),
            "or_adamw_step": (None, [_f32p, _f32p, _f32p, _f32p, sz, i64, cf]),
            "or_use_muon": (ci, [i64, i64]),
            "or_lr_scale_cosine": (cf, [i64]),
            "or_lr_scale": (cf, [ci, i64, i64, cf, i64]),
            "or_set_mgs_partials": (None, [ci]),
        }
        if which == "reference":
            sig["rl_last_attention_split"] = (None, [ctypes.POINTER(ctypes.c_double)])
            sig["rl_attention_core_rows"] = (ctypes.c_double, [_f32p] * 4 + [i64] * 5)
            sig["rl_attention_bwd_core_sample"] = (None, [_f32p] * 6 + [i64] * 5 + [ctypes.POINTER(ctypes.c_double)])
        for name, (res, args) in sig.items():
            if not hasattr(L, name):
                continue  # not restated in reference order: calling it raises
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _libs[which] = L
    return _libs[which]


def fp(a):
    """float32 pointer of a C-contiguous float32 array (None -> NULL)."""
    if a is None:
        return None
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(_f32p)


def ip(a):
    if a is None:
        return None
    assert a.dtype == np.int64 and a.flags.c_contiguous
    return a.ctypes.data_as(_i64p)


def up(a):
    if a is None:
        return None
    assert a.dtype == np.uint8 and a.flags.c_contiguous
    return a.ctypes.data_as(_u8p)


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def empty(n):
    return np.empty(int(n), dtype=np.float32)


def zeros(n):
    return np.zeros(int(n), dtype=np.float32)


# ---------------------------------------------------------------------------
# kernel wrappers (flat float32 arrays in, flat arrays out)
# ---------------------------------------------------------------------------

def matmul(A, B, M, K, N, act=0):
    C = empty(M * N)
    lib().or_matmul(fp(A), fp(B), fp(C), M, K, N, act)
    return C


def matmul_rows(A, rows, B, K, N, act=0):
    rows = np.ascontiguousarray(rows, dtype=np.int64)
    C = empty(len(rows) * N)
    lib().or_matmul_rows(fp(A), ip(rows), len(rows), fp(B), fp(C), K, N, act)
    return C


def act(x, code):
    y = empty(x.size)
    lib().or_act(fp(x), fp(y), x.size, code)
    return y


def act_grad(din, pre, code):
    y = empty(din.size)
    lib().or_act_grad(fp(din), fp(pre), fp(y), din.size, code)
    return y


def matmul_grad_a(dC, B, M, K, N):
    dA = empty(M * K)
    lib().or_matmul_grad_a(fp(dC), fp(B), fp(dA), M, K, N)
    return dA


def matmul_grad_w(A, dC, M, K, N):
    dB = empty(K * N)
    lib().or_matmul_grad_w(fp(A), fp(dC), fp(dB), M, K, N)
    return dB


def layernorm(x, last):
    y = empty(x.size)
    lib().or_layernorm(fp(x), fp(y), x.size, last)
    return y


def softmax(x, last):
    out = empty(x.size)
    lib().or_softmax(fp(x), fp(out), x.size, last)
    return out


def layernorm_grad(dout, x, last):
    y = empty(dout.size)
    lib().or_layernorm_grad(fp(dout), fp(x), fp(y), dout.size, last)
    return y


def embedding(W, idx, V, D):
    out = empty(idx.size * D)
    lib().or_embedding(fp(W), fp(idx), fp(out), idx.size, V, D)
    return out


def embedding_rows(idx, V):
    rows = np.empty(idx.size, dtype=np.int64)
    lib().or_embedding_rows(fp(idx), ip(rows), idx.size, V)
    return rows


def embedding_grad_w(dout, idx, V, D):
    dW = empty(V * D)
    lib().or_embedding_grad_w(fp(dout), fp(idx), fp(dW), dout.size // D, D, V)
    return dW


def cross_entropy(preds, labels, C):
    return float(lib().or_cross_entropy(fp(preds), fp(labels), preds.size, C))


def loss_grad(preds, labels, C):
    # elements past the last whole row of C are never written by ns_loss_grad
    # (codegen.cpp:1582-1595); its freshly resized buffer holds zeros there
    d = np.zeros(preds.size, dtype=np.float32)
    lib().or_loss_grad(fp(preds), fp(labels), fp(d), preds.size, C)
    return d


def attention_fwd(x, Wq, Wk, Wv, Wo, BS, D, H):
    out = empty(BS * D)
    lib().or_attention_fwd(fp(x), fp(Wq), fp(Wk), fp(Wv), fp(Wo), fp(out), BS, D, H)
    return out


def attention_fwd_rows(x, Wq, Wk, Wv, Wo, rows, BS, D, H):
    rows = np.ascontiguousarray(rows, dtype=np.int64)
    out = empty(len(rows) * D)
    lib().or_attention_fwd_rows(fp(x), fp(Wq), fp(Wk), fp(Wv), fp(Wo), ip(rows), len(rows),
                                fp(out), BS, D, H)
    return out


def attention_bwd(dout, x, Wq, Wk, Wv, Wo, BS, D, H):
    # zeros: with no tokens ns_attention_bwd returns before writing
    # (codegen.cpp:1789), leaving the train core's buffers as resized, which
    # is zero on a fresh context
    dX, dWq, dWk, dWv, dWo = empty(BS * D), zeros(D * D), zeros(D * D), zeros(D * D), zeros(D * D)
    lib().or_attention_bwd(fp(dout), fp(x), fp(Wq), fp(Wk), fp(Wv), fp(Wo), fp(dX), fp(dWq),
                           fp(dWk), fp(dWv), fp(dWo), BS, D, H)
    return dX, dWq, dWk, dWv, dWo


def moe_gate_logits(x, Wg, M, D, E):
    lg = empty(M * E)
    lib().or_moe_gate_logits(fp(x), fp(Wg), fp(lg), M, D, E)
    return lg


def moe_fwd(x, Wg, We1, We2, active, M, D, H, E):
    out = empty(M * D)
    best = np.empty(M, dtype=np.int64)
    prob = empty(M)
    lib().or_moe_fwd(fp(x), fp(Wg), fp(We1), fp(We2), up(active), fp(out), ip(best), fp(prob),
                     M, D, H, E)
    return out, best, prob


def moe_route(x, Wg, active, M, D, E, want_logits=False):
    best = np.empty(M, dtype=np.int64)
    prob = empty(M)
    lg = empty(M * E) if want_logits else None
    lib().or_moe_route(fp(x), fp(Wg), up(active), ip(best), fp(prob), fp(lg), M, D, E)
    return best, prob, lg


def moe_bwd(dout, x, Wg, We1, We2, active, M, D, H, E):
    dx, dWg, dWe1, dWe2 = empty(M * D), empty(D * E), empty(E * D * H), empty(E * H * D)
    lib().or_moe_bwd(fp(dout), fp(x), fp(Wg), fp(We1), fp(We2), up(active), fp(dx), fp(dWg),
                     fp(dWe1), fp(dWe2), M, D, H, E)
    return dx, dWg, dWe1, dWe2


def orthonom(G, M, N):
    G = f32(G).copy()
    lib().or_orthonom(fp(G), M, N)
    return G


def use_muon(r, c):
    return bool(lib().or_use_muon(r, c))


def lr_scale_cosine(step):
    return float(_load("oracle").or_lr_scale_cosine(step))


def lr_scale(sched, step):
    """The multiplier of schedule `sched` (Net.lr_schedule) at wrapper step
    `step` (optim_params.hpp:54-62)."""
    return float(_load("oracle").or_lr_scale(sched["kind"], sched["warmup"], sched["total"],
                                             ctypes.c_float(sched["min"]), step))


def parse_lr_schedule(text):
    """The `// ns.lr_schedule <kind> warmup=W total=T min=F` line of the IR
    text (the reference's compiled-in optim::kLRSchedule and its constants,
    optim_params.hpp:36-52); absent: the constant schedule."""
    out = {"kind": 0, "warmup": 100, "total": 10000, "min": 0.05}
    for raw in text.splitlines():
        line = raw.strip()
        if not line.startswith("// ns.lr_schedule"):
            continue
        toks = line[len("// ns.lr_schedule"):].split()
        out["kind"] = {"constant": 0, "cosine_warmup": 1}[toks[0]]
        for t in toks[1:]:
            k, v = t.split("=", 1)
            out[k] = float(np.float32(v)) if k == "min" else int(v)
    return out


# ---------------------------------------------------------------------------
# IR text (nsc --mlir) parsing
# ---------------------------------------------------------------------------

_LINE = re.compile(r"^\s*(ns\.[\w.]+)((?:\s+%[\w.]+)*)\s*(?::\s*Tensor\[([^\]]*)\][^/]*)?(?://\s?(.*))?$")


@dataclass
class Instr:
    op: str
    result: str | None
    operands: list
    dims: list | None
    comment: str


@dataclass
class Func:
    name: str
    instrs: list = field(default_factory=list)
    ret: str | None = None

    @property
    def is_train(self):
        return any(i.op == "ns.grad" for i in self.instrs)


_NO_RESULT = {"ns.grad", "ns.opt.step", "ns.forward"}


def parse_ir(text):
    funcs, cur = [], None
    for raw in text.splitlines():
        line = raw.strip()
        if not line or line.startswith("//"):
            continue
        if line.startswith("ns.func @"):
            cur = Func(line[len("ns.func @"):].split()[0])
            funcs.append(cur)
            continue
        if line == "}":
            cur = None
            continue
        if line.startswith("ns.return"):
            cur.ret = line.split("%", 1)[1].strip()
            continue
        m = _LINE.match(line)
        if not m:
            raise ValueError(f"unparsed IR line: {raw!r}")
        op, ids, dims, comment = m.group(1), m.group(2), m.group(3), m.group(4) or ""
        names = [t[1:] for t in ids.split()]
        if op in _NO_RESULT:
            res, opnds = None, names
        else:
            res, opnds = (names[0] if names else None), names[1:]
        dl = None
        if dims is not None:
            dl = []
            for d in dims.split(","):
                d = d.strip()
                dl.append(int(d) if d.lstrip("-").isdigit() else -1)
        cur.instrs.append(Instr(op, res, opnds, dl, comment.strip()))
    return funcs


def comment_attr(comment, key):
    m = re.search(r"\b%s=(\d+)" % key, comment)
    return int(m.group(1)) if m else None


def comment_str(comment, key):
    """Raw value of key=VALUE in an instruction comment (oracle/irdump), or None."""
    m = re.search(r"(?:^|\s)%s=(\S*)" % re.escape(key), comment)
    return m.group(1) if m else None


# Ops the reference's fusion pass may append to a GEMM (fusion.cpp:23-40).
_FUSIBLE = {"ns.activation." + k for k in ("relu", "leaky_relu", "sigmoid", "tanh", "swish", "gelu", "silu",
                                           "identity", "softmax")} | {"ns.layernorm", "ns.subview_binop"}


def fusion_groups(f):
    """The reference fusion pass (fusion.cpp:52-94, 97-175) on one function:
    {index of an absorbed epilogue instruction: N of its GEMM}.  Inside a
    group the emitted code applies activations as usual, layernorm and
    softmax over rows of N, and -- the binop's operator symbol being empty
    (the lexer gives operator tokens no text) -- a binop as the identity
    activation (codegen.cpp:2052-2076)."""
    ins = f.instrs
    uses = {}
    for i in ins:
        for o in i.operands:
            uses[o] = uses.get(o, 0) + 1
    out = {}
    i = 0
    while i < len(ins):
        lead = ins[i]
        if lead.op != "ns.matmul" or uses.get(lead.result, 0) != 1:
            i += 1
            continue
        end, consumed = i + 1, lead.result
        while end < len(ins):
            c = ins[end]
            if c.op not in _FUSIBLE or not c.operands or c.operands[0] != consumed:
                break
            nxt = ins[end + 1] if end + 1 < len(ins) else None
            is_last = (nxt is None or nxt.op not in _FUSIBLE or not nxt.operands or
                       nxt.operands[0] != c.result)
            u = uses.get(c.result, 0)
            if u > 1 or (not is_last and u == 0):
                break
            consumed = c.result
            end += 1
        if end > i + 1:
            for j in range(i + 1, end):
                out[j] = lead.operands[1]  # the GEMM's weight; N = its columns
            i = end
        else:
            i += 1
    return out


class Net:
    """Static facts of a network: weights in TENSOR_ALLOC order, geometry."""

    def __init__(self, ir_text):
        self.funcs = parse_ir(ir_text)
        self.lr_schedule = parse_lr_schedule(ir_text)
        self.fwd = next((f for f in self.funcs if not f.is_train), None)
        self.train = next((f for f in self.funcs if f.is_train), None)
        if self.fwd is None:
            raise ValueError("IR has no forward function")
        self.weights = []  # (name, rows, cols)
        for i in self.fwd.instrs:
            if i.op == "ns.tensor.alloc":
                r = i.dims[0] if len(i.dims) > 0 else 1
                c = i.dims[1] if len(i.dims) > 1 else 1
                self.weights.append((i.result, r, c))
        self.shape = {n: (r, c) for n, r, c in self.weights}
        self.offsets, off = {}, 0
        for n, r, c in self.weights:
            self.offsets[n] = off
            off += r * c
        self.total = off
        # attention heads and MoE geometry, keyed by the first weight operand
        self.heads, self.moe = {}, None
        for f in self.funcs:
            for i in f.instrs:
                if i.op == "ns.layer.attention":
                    self.heads[i.operands[1]] = comment_attr(i.comment, "heads") or 1
                if i.op == "ns.layer.moe":
                    D, E = self.shape[i.operands[1]]
                    H = self.shape[i.operands[2]][1] // D
                    k0 = comment_attr(i.comment, "initial") or E
                    if k0 <= 0 or k0 > E:
                        k0 = E
                    self.moe = dict(D=D, E=E, H=H, K0=k0, g=i.operands[1], e1=i.operands[2], e2=i.operands[3])
        self.fused = {f.name: fusion_groups(f) for f in self.funcs}
        self.in_cols, self.out_cols = self._geometry()

    def ids_table(self, f):
        """The emitted code's static (rows, cols) per value id, -1 = dynamic
        (codegen.cpp:1170-1224): result types, weight shapes, and the input's
        width (first GEMM's K, 1 for embedding-first or anything else)."""
        t = {}
        for i in f.instrs:
            if i.result and i.op != "ns.tensor.alloc":
                d = i.dims or []
                t[i.result] = (d[0] if len(d) > 0 else -1, d[1] if len(d) > 1 else -1)
        for n, r, c in self.weights:
            t[n] = (r, c)
        in_w = 1
        for i in f.instrs:
            if i.op == "ns.matmul" and len(i.operands) >= 2:
                in_w = self._static_dims(f, i.operands[1])[0]
                break
            if i.op == "ns.layer.embedding":
                break
        xid = _input_id(f, set(self.shape))
        if xid is not None:  # codegen.cpp:1209-1224: the input's cols become in_w
            t[xid] = (t.get(xid, (-1, -1))[0], in_w)
        return t

    def _static_dims(self, f, vid):
        """(rows, cols) of a GEMM's B operand: a weight's shape, or the
        static result type of the instruction that produced it."""
        if vid in self.shape:
            return self.shape[vid]
        for i in f.instrs:
            if i.result == vid and i.dims:
                return (i.dims[0] if len(i.dims) > 0 else -1, i.dims[1] if len(i.dims) > 1 else -1)
        return (-1, -1)

    def _rt_cols(self, f, vid):
        for i in f.instrs:
            if i.result == vid and i.dims and len(i.dims) > 1:
                return i.dims[1]
        if vid in self.shape:
            return self.shape[vid][1]
        return -1

    def _geometry(self):
        """in_cols / out_cols as the emitted driver computes them
        (codegen.cpp:2295-2320)."""
        f = self.fwd
        absorbed = fusion_groups(f)
        in_cols = out_cols = -1
        for i in f.instrs:
            if i.op != "ns.tensor.alloc" and i.result and i.result == f.ret:
                out_cols = self._rt_cols(f, i.result)
        for k, i in enumerate(f.instrs):
            if k in absorbed:
                continue
            if i.op == "ns.matmul" and len(i.operands) >= 2:
                r, c = self._static_dims(f, i.operands[1])
                if in_cols < 0:
                    in_cols = r
                out_cols = c
            if i.op == "ns.layer.embedding" and in_cols < 0:
                in_cols = 1
            if (i.op in ("ns.layer.attention", "ns.layernorm", "ns.layer.moe", "ns.activation.softmax",
                         "ns.concat", "ns.slice", "ns.index", "ns.scatter", "ns.transpose", "ns.reshape")
                    and i.result):
                c = self._rt_cols(f, i.result)
                if c > 0:
                    out_cols = c
        return (in_cols if in_cols > 0 else 1), (out_cols if out_cols > 0 else 1)

    def output_numel(self, input_numel):
        return (input_numel // self.in_cols) * self.out_cols


class MT19937:
    """std::mt19937 (the reference context's RNG, codegen.cpp:2419-2421):
    Matsumoto-Nishimura MT19937 with the standard's init_genrand seeding;
    numpy's MT19937 core generates, its state is set from that seeding.
    Pinned by the standard's check value (the 10000th draw of a default-
    seeded engine is 4123659995, [rand.predef]) in tests/test_oracle.py."""

    def __init__(self, seed):
        key = np.zeros(624, dtype=np.uint64)
        key[0] = seed & 0xFFFFFFFF
        for i in range(1, 624):
            prev = int(key[i - 1])
            key[i] = (1812433253 * (prev ^ (prev >> 30)) + i) & 0xFFFFFFFF
        self.bg = np.random.MT19937()
        self.bg.state = {"bit_generator": "MT19937", "state": {"key": key.astype(np.uint32), "pos": 624}}

    def draws(self, n):
        return self.bg.random_raw(n).astype(np.uint64)


def bernoulli(rng, n, p):
    """n draws of libstdc++'s std::bernoulli_distribution(p)(rng): true iff
    generate_canonical<double, 53>(rng) < p, where generate_canonical takes
    two 32-bit draws d1, d2 and returns (d1 + d2 * 2^32) / 2^64 in double
    arithmetic, clamped below 1 (bits/random.h, bits/random.tcc of the
    libstdc++ the reference's driver is compiled against)."""
    d = rng.draws(2 * n)
    s = d[0::2].astype(np.float64) + d[1::2].astype(np.float64) * 4294967296.0
    r = s / 18446744073709551616.0
    r[r >= 1.0] = np.nextafter(1.0, 0.0)
    return r < p


def dropout_rate(rate):
    """The rate as the emitted code spells it: clamped to [0, 0.999999] and
    printed with std::to_string (codegen.cpp:2877-2880)."""
    rate = 0.0 if rate < 0.0 else (0.999999 if rate >= 1.0 else rate)
    return float("%f" % rate)


def _act_of(f, pre):
    for i in f.instrs:
        if i.op.startswith("ns.activation.") and i.operands and i.operands[0] == pre:
            kind = i.op.split(".")[-1]
            # softmax's ACTIVATION_GRAD carries "softmax", derivative code 0 = 1
            # (mlir_compiler.cpp:348-360, codegen.cpp:3074-3081, 1305-1315)
            return 0 if kind == "softmax" else ACT_CODES[kind]
    raise ValueError(f"no activation consumes {pre}")


def _input_id(f, weights):
    for i in f.instrs:
        if i.op == "ns.layer.embedding" and len(i.operands) >= 2:
            return i.operands[1]
        if i.op == "ns.matmul" and i.operands and i.operands[0] not in weights:
            return i.operands[0]
        if i.op in ("ns.layer.attention", "ns.layernorm", "ns.layer.moe", "ns.dropout", "ns.transpose",
                    "ns.concat", "ns.reshape", "ns.slice", "ns.index", "ns.scatter") or \
                i.op.startswith("ns.activation."):
            if i.operands and i.operands[0] not in weights:
                return i.operands[0]
    return None


class Model:
    """One model instance: blob, MoE liveness, optimizer state, LR step."""

    def __init__(self, net: Net, weights):
        w = f32(weights).ravel()
        if w.size != net.total:
            raise ValueError("weight count mismatch")
        self.net = net
        self.w = w.copy()
        self.lr_step = 0
        self.rng = MT19937(0x9E3779B9)  # the context's engine, codegen.cpp:2421
        self.adam = {}  # name -> (m, v, t)
        self.active = None
        if net.moe:
            self.active = np.zeros(net.moe["E"], dtype=np.uint8)
            self.active[: net.moe["K0"]] = 1

    def weight(self, name):
        r, c = self.net.shape[name]
        o = self.net.offsets[name]
        return self.w[o:o + r * c]

    # -- shared op semantics ------------------------------------------------
    def _run(self, f, x, y, train_mode, record=None):
        net = self.net
        wset = set(net.shape)
        buf = {}
        masks = {}  # dropout result id -> its scaled mask (train_mode forward)
        static = net.ids_table(f) if f.is_train else {}

        def ce_cols(preds):
            # the class count of CROSS_ENTROPY / LOSS_GRAD: the logits' static
            # cols (result type or weight shape), else the input width
            # (codegen.cpp:2896, :2904), not the propagated width
            c = static.get(preds, (-1, -1))[1]
            return c if c > 0 else net.in_cols
        xid = _input_id(f, wset)
        yid = None
        for i in f.instrs:
            if i.op == "ns.cross_entropy":
                yid = i.operands[1]

        def val(v):
            if v == xid:
                return x
            if v == yid:
                return y
            if v in wset:
                return self.weight(v)
            return buf[v]

        width = {}

        def cols(v):
            if v in width:
                return width[v]
            if v in wset:
                return net.shape[v][1]
            if v == xid:
                return net.in_cols
            return -1

        grads = {}
        loss = None
        fused = net.fused[f.name]
        if fused and f.is_train:
            raise NotImplementedError("fused epilogue groups in a train function")
        ids = net.ids_table(f)

        def idr(v):
            return ids.get(v, (-1, -1))[0]

        def idc(v):
            return ids.get(v, (-1, -1))[1]

        for k, i in enumerate(f.instrs):
            op, o = i.op, i.operands
            if op in ("ns.tensor.alloc", "ns.grad", "ns.forward"):
                continue
            if k in fused and op in ("ns.subview_binop", "ns.layernorm", "ns.activation.softmax"):
                N = net.shape[fused[k]][1]
                src = val(o[0])
                if op == "ns.subview_binop":  # operator-less binop = identity activation
                    buf[i.result] = src.copy()
                elif op == "ns.layernorm":
                    buf[i.result] = layernorm(src, N)
                else:
                    buf[i.result] = softmax(src, N)
                width[i.result] = N
                continue
            if op in ("ns.subview_binop", "ns.constant", "ns.transpose", "ns.concat", "ns.reshape", "ns.slice",
                      "ns.index", "ns.scatter") and f.is_train:
                raise NotImplementedError(op + " in a train function (the reference's train core skips it)")
            if op == "ns.activation.softmax":
                src = val(o[0])
                if f.is_train:  # train core: rows of the input's width (codegen.cpp:2860-2873)
                    last = cols(o[0]) if cols(o[0]) > 0 else 1
                else:  # codegen.cpp:2027-2033
                    last = idc(i.result) if idc(i.result) > 0 else (idc(o[0]) if idc(o[0]) > 0 else 1)
                buf[i.result] = softmax(src, last)
                width[i.result] = last
                continue
            if op == "ns.subview_binop":  # ns_binop, codegen.cpp:1267-1278 / 2007-2018
                a = val(o[0])
                b = np.zeros(0, np.float32) if o[1] == xid else val(o[1])
                code = {"-": 1, "*": 2, "/": 3}.get(comment_str(i.comment, "op") or "", 0)
                bb = np.resize(b, a.size) if b.size else np.zeros(a.size, np.float32)
                with np.errstate(all="ignore"):
                    buf[i.result] = [a + bb, a - bb, a * bb, a / bb][code].astype(np.float32)
                width[i.result] = cols(o[0])
                continue
            if op == "ns.constant":
                v = comment_str(i.comment, "value")
                if v is None:
                    v = i.comment.split()[-1]
                buf[i.result] = np.array([np.float32(float(v))], np.float32)
                continue
            if op == "ns.reshape":
                buf[i.result] = val(o[0]).copy()
                width[i.result] = idc(i.result)
                continue
            if op == "ns.transpose":  # ns_transpose2d, codegen.cpp:1638-1644 / 2082-2100
                a = val(o[0])
                C = idc(o[0]) if idc(o[0]) > 0 else 1
                R = idr(o[0]) if idr(o[0]) > 0 else a.size // C
                buf[i.result] = np.ascontiguousarray(a[:R * C].reshape(R, C).T).ravel()
                width[i.result] = R
                continue
            if op == "ns.concat":  # ns_concat2 / ns_concat0, codegen.cpp:1646-1661 / 2102-2123
                a, b = val(o[0]), val(o[1])
                if comment_str(i.comment, "axis") == "0":
                    D = idc(o[0]) if idc(o[0]) > 0 else 1
                    Ba, Bb = a.size // D, b.size // D
                    buf[i.result] = np.concatenate([a[:Ba * D], b[:Bb * D]])
                else:
                    Ca = idc(o[0]) if idc(o[0]) > 0 else 1
                    Cb = idc(o[1]) if idc(o[1]) > 0 else 1
                    R = a.size // Ca
                    buf[i.result] = np.concatenate([a[:R * Ca].reshape(R, Ca), b[:R * Cb].reshape(R, Cb)],
                                                   axis=1).ravel()
                    width[i.result] = Ca + Cb
                continue
            if op == "ns.slice":  # ns_slice2 / ns_slicerows, codegen.cpp:1663-1676 / 2129-2150
                a = val(o[0])
                ax, s0, e0 = (int(comment_str(i.comment, kk)) for kk in ("axis", "start", "stop"))
                C = idc(o[0]) if idc(o[0]) > 0 else 1
                if ax == 0:
                    buf[i.result] = a[s0 * C:e0 * C].copy()
                else:
                    M = a.size // C
                    buf[i.result] = np.ascontiguousarray(a[:M * C].reshape(M, C)[:, s0:e0]).ravel()
                    width[i.result] = e0 - s0
                continue
            if op in ("ns.index", "ns.scatter"):  # codegen.cpp:1678-1709 / 2151-2203
                a = val(o[0])
                ax = int(comment_str(i.comment, "axis"))
                idx = [int(t) for t in (comment_str(i.comment, "idx") or "").split(",") if t]
                C = idc(o[0]) if idc(o[0]) > 0 else 1
                L = len(idx)
                if op == "ns.index":
                    if ax == 0:
                        buf[i.result] = np.concatenate([a[j * C:(j + 1) * C] for j in idx]) if L else empty(0)
                    else:
                        M = a.size // C
                        buf[i.result] = np.ascontiguousarray(a[:M * C].reshape(M, C)[:, idx]).ravel()
                        width[i.result] = L
                else:
                    u = val(o[1])
                    if ax == 0:
                        R = idr(o[0]) if idr(o[0]) > 0 else 0
                        out = a[:R * C].copy()
                        for kk, j in enumerate(idx):
                            out[j * C:(j + 1) * C] = u[kk * C:(kk + 1) * C]
                    else:
                        M = a.size // C
                        out = a[:M * C].copy().reshape(M, C)
                        for kk, j in enumerate(idx):
                            out[:, j] = u[kk::L][:M] if L else out[:, j]
                        out = out.ravel()
                    buf[i.result] = out
                    width[i.result] = C
                continue
            if op == "ns.matmul":
                A = val(o[0])
                K, N = net._static_dims(f, o[1])
                if K <= 0 or N <= 0:
                    raise ValueError(f"matmul {i.result}: operand {o[1]} has no static shape")
                M = A.size // K
                buf[i.result] = matmul(A, val(o[1]), M, K, N)
                width[i.result] = N
            elif op.startswith("ns.activation."):
                kind = op.split(".")[-1]
                if kind not in ACT_CODES:
                    raise NotImplementedError(op)
                buf[i.result] = act(val(o[0]), ACT_CODES[kind])
                width[i.result] = cols(o[0])
            elif op == "ns.dropout":
                src = val(o[0])
                if f.is_train and train_mode:
                    # codegen.cpp:2874-2893: m = keep ? 1/(1-r) : 0 per element, in order
                    r = dropout_rate(float(comment_str(i.comment, "rate") or 0.0))
                    scale = np.float32(1.0) / np.float32(1.0 - r)
                    keep = bernoulli(self.rng, src.size, 1.0 - r)
                    m = np.where(keep, scale, np.float32(0.0)).astype(np.float32)
                    masks[i.result] = m
                    buf[i.result] = (src * m).astype(np.float32)
                else:
                    buf[i.result] = src.copy()
                width[i.result] = cols(o[0])
            elif op == "ns.layernorm":
                src = val(o[0])
                last = i.dims[1] if (i.dims and len(i.dims) > 1 and i.dims[1] > 0) else cols(o[0])
                if f.is_train:
                    last = cols(o[0]) if cols(o[0]) > 0 else last
                buf[i.result] = layernorm(src, max(last, 1))
                width[i.result] = last
            elif op == "ns.layer.embedding":
                V, D = net.shape[o[0]]
                buf[i.result] = embedding(val(o[0]), val(o[1]), V, D)
                width[i.result] = D
            elif op == "ns.layer.attention":
                D = net.shape[o[1]][0]
                H = net.heads[o[1]]
                xa = val(o[0])
                BS = xa.size // D
                buf[i.result] = attention_fwd(xa, *(val(w) for w in o[1:5]), BS, D, H)
                width[i.result] = D
            elif op == "ns.layer.moe":
                m = net.moe
                xa = val(o[0])
                M = xa.size // m["D"]
                out, best, prob = moe_fwd(xa, *(val(w) for w in o[1:4]), self.active,
                                          M, m["D"], m["H"], m["E"])
                buf[i.result] = out
                width[i.result] = m["D"]
                if record is not None:
                    record["moe_best"] = best
                    record["moe_prob"] = prob
            elif op == "ns.cross_entropy":
                loss = cross_entropy(val(o[0]), y, ce_cols(o[0]))
            elif not train_mode:
                continue
            elif op == "ns.grad.loss":
                C = ce_cols(o[0])
                buf[i.result] = loss_grad(val(o[0]), y, C)
                width[i.result] = C
            elif op == "ns.grad.matmul.a":
                dC = val(o[0])
                K, N = net.shape[o[1]]
                M = dC.size // N
                buf[i.result] = matmul_grad_a(dC, val(o[1]), M, K, N)
                width[i.result] = K
            elif op == "ns.grad.matmul.w":
                dC = val(o[1])
                K, N = net.shape[o[2]]
                M = dC.size // N
                buf[i.result] = matmul_grad_w(val(o[0]), dC, M, K, N)
                grads[o[2]] = i.result
            elif op == "ns.grad.activation" and o[1] in masks:
                # dropout's gradient: dOut * the saved mask (codegen.cpp:3066-3073)
                buf[i.result] = (val(o[0]) * masks[o[1]]).astype(np.float32)
                width[i.result] = cols(o[0])
            elif op == "ns.grad.activation":
                code = _act_of(f, o[1])
                buf[i.result] = act_grad(val(o[0]), val(o[1]), code)
                width[i.result] = cols(o[0])
            elif op == "ns.grad.layernorm":
                last = cols(o[1])
                buf[i.result] = layernorm_grad(val(o[0]), val(o[1]), max(last, 1))
                width[i.result] = last
            elif op == "ns.grad.embedding.w":
                V, D = net.shape[o[2]]
                buf[i.result] = embedding_grad_w(val(o[0]), val(o[1]), V, D)
            elif op.startswith("ns.grad.attention."):
                which = op.split(".")[-1]
                key = ("attn", o[0], o[1], o[2])
                if key not in buf:
                    D = net.shape[o[2]][0]
                    H = net.heads[o[2]]
                    dout = val(o[0])
                    BS = dout.size // D
                    buf[key] = attention_bwd(dout, val(o[1]), *(val(w) for w in o[2:6]), BS, D, H)
                idx = {"x": 0, "wq": 1, "wk": 2, "wv": 3, "wo": 4}[which]
                buf[i.result] = buf[key][idx]
                if which == "x":
                    width[i.result] = net.shape[o[2]][0]
            elif op.startswith("ns.grad.moe."):
                which = op.split(".")[-1]
                key = ("moe", o[0], o[1])
                m = net.moe
                if key not in buf:
                    dout = val(o[0])
                    M = dout.size // m["D"]
                    buf[key] = moe_bwd(dout, val(o[1]), *(val(w) for w in o[2:5]), self.active,
                                       M, m["D"], m["H"], m["E"])
                idx = {"x": 0, "wg": 1, "we1": 2, "we2": 3}[which]
                buf[i.result] = buf[key][idx]
                if which == "x":
                    width[i.result] = m["D"]
            elif op == "ns.opt.step":
                self._opt_step(o, val, record, comment_str(i.comment, "optimizer") == "adamw")
            else:
                raise NotImplementedError(op)
        if record is not None:
            record["buf"] = buf
        return buf, loss

    def _opt_step(self, o, val, record, adamw_only=False):
        """codegen.cpp:3088-3124, pairs in TENSOR_ALLOC order.  adamw_only:
        every weight takes AdamW (the `optimizer=adamw` build knob of this
        backend; the reference chooses by shape)."""
        lr = self._lr
        L = lib()
        for k in range(0, len(o) - 1, 2):
            name, g = o[k], o[k + 1]
            r, c = self.net.shape[name]
            w = self.weight(name)  # view into the blob: updated in place
            gr = f32(val(g)).copy()
            if use_muon(r, c) and not adamw_only:
                L.or_muon_step(fp(w), fp(gr), r, c, ctypes.c_float(lr))
            else:
                m, v, t = self.adam.get(name, (np.zeros(r * c, np.float32),
                                               np.zeros(r * c, np.float32), 0))
                t += 1
                L.or_adamw_step(fp(w), fp(gr), fp(m), fp(v), r * c, t, ctypes.c_float(lr))
                self.adam[name] = (m, v, t)

    # -- C-ABI mirror -------------------------------------------------------
    def eval_infer(self, x, record=None):
        x = f32(x).ravel()
        buf, _ = self._run(self.net.fwd, x, None, False, record)
        return buf[self.net.fwd.ret].copy()

    def train_step(self, x, labels, lr, record=None):
        """ns_runtime_train_step: the compiled-in schedule's multiplier at the
        model's step counter, which then advances (codegen.cpp:2636-2644;
        the reference compiles the constant schedule, multiplier 1)."""
        step = self.lr_step
        self.lr_step += 1
        self._lr = np.float32(lr) * np.float32(lr_scale(self.net.lr_schedule, step))
        _, loss = self._run(self.net.train, f32(x).ravel(), f32(labels).ravel(), True, record)
        return np.float32(loss)

    def objective_loss(self, x, labels):
        self._lr = np.float32(0.0)
        _, loss = self._run(self.net.train, f32(x).ravel(), f32(labels).ravel(), False)
        return np.float32(loss)

    # -- MoE expert lifecycle: host-side blob edits (codegen.cpp:2562-2626) --
    def _moe_views(self):
        m = self.net.moe
        return m, self.weight(m["g"]), self.weight(m["e1"]), self.weight(m["e2"])

    def _noise(self, n):
        # ((float)(rng() % 1001) / 1000.f - 0.5f) * 1e-2f, one draw per element
        r = (self.rng.draws(n) % np.uint64(1001)).astype(np.float32)
        return (r / np.float32(1000.0) - np.float32(0.5)) * np.float32(1e-2)

    def expert_count(self):
        return int(self.active.sum()) if self.active is not None else 0

    def expert_birth(self, n):
        """ns_expert_birth (codegen.cpp:2567-2595): a random live source
        expert (rng() % cap, redrawn while dead, at most cap redraws) is copied
        with per-element noise into the first n dead slots, gate column first,
        then FFN-1, then FFN-2."""
        m, g, e1, e2 = self._moe_views()
        cap, D, H = m["E"], m["D"], m["H"]
        if n <= 0 or self.expert_count() >= cap:
            return self.expert_count()
        src = int(self.rng.draws(1)[0] % np.uint64(cap))
        tries = 0
        while tries < cap and not self.active[src]:
            tries += 1
            src = int(self.rng.draws(1)[0] % np.uint64(cap))
        gm = g.reshape(D, cap)
        for e in range(cap):
            if n <= 0:
                break
            if self.active[e]:
                continue
            gm[:, e] = gm[:, src] + self._noise(D)
            e1[e * D * H:(e + 1) * D * H] = e1[src * D * H:(src + 1) * D * H] + self._noise(D * H)
            e2[e * H * D:(e + 1) * H * D] = e2[src * H * D:(src + 1) * H * D] + self._noise(H * D)
            self.active[e] = 1
            n -= 1
        return self.expert_count()

    def expert_merge(self, a, b):
        """ns_expert_merge (codegen.cpp:2597-2617): expert a becomes the
        fp32 average 0.5f * (a + b) of both, b dies."""
        m, g, e1, e2 = self._moe_views()
        cap, D, H = m["E"], m["D"], m["H"]
        if a < 0 or b < 0 or a == b or a >= cap or b >= cap or not self.active[a] or not self.active[b]:
            return self.expert_count()
        gm = g.reshape(D, cap)
        half = np.float32(0.5)
        gm[:, a] = half * (gm[:, a] + gm[:, b])
        sa, sb = slice(a * D * H, (a + 1) * D * H), slice(b * D * H, (b + 1) * D * H)
        e1[sa] = half * (e1[sa] + e1[sb])
        e2[sa] = half * (e2[sa] + e2[sb])
        self.active[b] = 0
        return self.expert_count()

    def expert_kill(self, k):
        """ns_expert_kill (codegen.cpp:2619-2626): only the mask changes."""
        if k < 0 or k >= self.net.moe["E"] or not self.active[k]:
            return self.expert_count()
        self.active[k] = 0
        return self.expert_count()
