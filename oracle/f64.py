"""Float64 evaluation of a training step's forward and reverse bodies
(TEST INFRASTRUCTURE ONLY: tests/ and the fixture scripts under
tests/golden/ use it as an accuracy yardstick; the product never does).

The oracle (oracle.py + ns_oracle.c) reproduces the reference's float32
arithmetic bit for bit.  This module evaluates the SAME formulas -- the
reference's, quirks included -- in float64, so that the rounding error of
any float32 implementation (the reference's own sequential sums, or the
GPU's blocked ones) can be measured against a common yardstick:

* matmul and its gradients: codegen.cpp:1257-1265, :1318-1337;
* activations and their derivatives: :1244-1255, :1305-1315 (the float
  constants 1.41421356f and 2.50662827f of GELU are kept as the float32
  values the emitted code uses);
* LayerNorm forward (:1280-1291) and the reference's gradient formula,
  which omits the 1/(var+eps) factor on the projection term (:1346-1371);
* embedding forward (:1711-1718, out-of-range ids read row 0) and its
  gradient (:1374-1383, out-of-range ids skipped);
* attention over ONE sequence of all tokens (S = BS), forward :1724-1777,
  backward :1785-1907 (dPre = dout Wo^T, per head P, oh = P V, dp = dPre V^T,
  dS = P (dp - rowsum(P dp)), dQ = dS K scale, dV = P^T dPre, dK = dS^T Q
  scale; dW* = x^T d*, dWo = oh^T dout, dX = dQ Wq^T + dK Wk^T + dV Wv^T);
* cross-entropy mean over rows of -sum_{y>0} log p (:1598-1613) and its
  gradient (p - y) / rows (:1582-1595);
* the top-1 mixture of experts, forward (:1915-1945: p = softmax of the
  live experts' gate logits, out = p_best GELU(x We1[best]) We2[best], GELU
  with erf and the float32 constant 0.70710678f) and its four gradients
  (:1388-1579), with each token's expert taken from the float32 oracle's
  routing (`moe_best`): float64 logits could break a near tie the other
  way, and the choice is a discrete decision, not a rounding error.

The instruction walk follows oracle.Model._run (the reference's train core,
codegen.cpp:2755-3157) for the subset of operations above; anything else
raises NotImplementedError.  Pinned in tests/test_oracle.py: on small
networks every value agrees with the bit-exact float32 oracle to within the
float32 rounding of the oracle's own sums.
"""
from __future__ import annotations

import numpy as np

import oracle

F64 = np.float64
_SQ2 = F64(np.float32(1.41421356))
_SQ2PI = F64(np.float32(2.50662827))


def _erf(x):
    from scipy.special import erf
    return erf(x)


def act(x, code):
    if code == 1:
        return np.where(x > 0, x, 0.0)
    if code == 2:
        return np.where(x > 0, x, F64(np.float32(0.01)) * x)
    if code == 3:
        return 1.0 / (1.0 + np.exp(-x))
    if code == 4:
        return np.tanh(x)
    if code == 5:
        return x / (1.0 + np.exp(-x))
    if code == 6:
        return 0.5 * x * (1.0 + _erf(x / _SQ2))
    return x.copy()


def act_deriv(x, code):
    if code == 1:
        return np.where(x > 0, 1.0, 0.0)
    if code == 2:
        return np.where(x > 0, 1.0, F64(np.float32(0.01)))
    if code == 3:
        s = 1.0 / (1.0 + np.exp(-x))
        return s * (1.0 - s)
    if code == 4:
        t = np.tanh(x)
        return 1.0 - t * t
    if code == 5:
        s = x / (1.0 + np.exp(-x))
        return s + x * (1.0 - s)
    if code == 6:
        u = x / _SQ2
        return 0.5 * (1.0 + _erf(u)) + x * np.exp(-u * u) / _SQ2PI
    return np.ones_like(x)


def layernorm(x, last):
    r = x.reshape(-1, last)
    mu = r.mean(axis=1, keepdims=True)
    var = ((r - mu) ** 2).mean(axis=1, keepdims=True)
    return ((r - mu) / np.sqrt(var + F64(np.float32(1e-5)))).ravel()


def layernorm_grad(dout, x, last):
    xr, dr = x.reshape(-1, last), dout.reshape(-1, last)
    xc = xr - xr.mean(axis=1, keepdims=True)
    var = (xc * xc).mean(axis=1, keepdims=True)
    gamma = (xc * dr).mean(axis=1, keepdims=True)
    inv = 1.0 / np.sqrt(var + F64(np.float32(1e-5)))
    return ((dr - dr.mean(axis=1, keepdims=True) - xc * gamma) * inv).ravel()


def _rows(idx, V):
    """Resolved embedding row per id, -1 when out of range (truncation)."""
    f = np.asarray(idx, np.float32)
    ok = (f > -1.0) & (f < np.float32(V))
    k = np.where(ok, np.trunc(np.where(ok, f, 0)).astype(np.int64), -1)
    return np.where((k >= 0) & (k < V), k, -1)


def embedding(W, idx, V, D):
    rows = _rows(idx, V)
    return W.reshape(V, D)[np.maximum(rows, 0)].ravel()


def embedding_grad(dout, idx, V, D):
    rows = _rows(idx, V)
    dW = np.zeros((V, D))
    ok = rows >= 0
    np.add.at(dW, rows[ok], dout.reshape(-1, D)[ok])
    return dW.ravel()


def _softmax_rows(s):
    s -= s.max(axis=1, keepdims=True)
    np.exp(s, out=s)
    s /= s.sum(axis=1, keepdims=True)
    return s


def attention_fwd(x, Wq, Wk, Wv, Wo, D, H):
    X = x.reshape(-1, D)
    Q, K, V = X @ Wq.reshape(D, D), X @ Wk.reshape(D, D), X @ Wv.reshape(D, D)
    Dk = D // H
    scale = F64(np.float32(1.0) / np.sqrt(np.float32(Dk)))
    ctx = np.empty_like(Q)
    for h in range(H):
        c = slice(h * Dk, (h + 1) * Dk)
        P = Q[:, c] @ K[:, c].T
        P *= scale
        ctx[:, c] = _softmax_rows(P) @ V[:, c]
        del P
    return (ctx @ Wo.reshape(D, D)).ravel()


def attention_bwd(dout, x, Wq, Wk, Wv, Wo, D, H):
    X, G = x.reshape(-1, D), dout.reshape(-1, D)
    Wq, Wk, Wv, Wo = (w.reshape(D, D) for w in (Wq, Wk, Wv, Wo))
    Q, K, V = X @ Wq, X @ Wk, X @ Wv
    dPre = G @ Wo.T
    Dk = D // H
    scale = F64(np.float32(1.0) / np.sqrt(np.float32(Dk)))
    oh, dQ, dK, dV = (np.zeros_like(Q) for _ in range(4))
    for h in range(H):
        c = slice(h * Dk, (h + 1) * Dk)
        P = Q[:, c] @ K[:, c].T
        P *= scale
        _softmax_rows(P)
        oh[:, c] = P @ V[:, c]
        dV[:, c] = P.T @ dPre[:, c]
        dS = dPre[:, c] @ V[:, c].T
        dS -= np.einsum("ij,ij->i", P, dS)[:, None]
        dS *= P
        del P
        dQ[:, c] = (dS @ K[:, c]) * scale
        dK[:, c] = (dS.T @ Q[:, c]) * scale
        del dS
    dX = dQ @ Wq.T + dK @ Wk.T + dV @ Wv.T
    return (dX.ravel(), (X.T @ dQ).ravel(), (X.T @ dK).ravel(), (X.T @ dV).ravel(), (oh.T @ G).ravel())


def cross_entropy(preds, labels, C):
    p = _softmax_rows(preds.reshape(-1, C).copy())
    y = labels.reshape(-1, C)
    with np.errstate(divide="ignore"):
        return float(-np.sum(np.where(y > 0, np.log(np.where(y > 0, p, 1.0)), 0.0)) / p.shape[0])


def loss_grad(preds, labels, C):
    p = _softmax_rows(preds.reshape(-1, C).copy())
    return ((p - labels.reshape(-1, C)) / p.shape[0]).ravel()


_MOE_C = F64(np.float32(0.7071067811865476))   # the emitted GELU's 1/sqrt(2)
_MOE_C2 = F64(np.float32(0.3989422804014327))  # and its 1/sqrt(2 pi)


def _moe_probs(X, Wg, live):
    lg = X @ Wg
    mx = np.where(live, lg, -np.inf).max(axis=1, keepdims=True)
    ex = np.where(live, np.exp(lg - mx), 0.0)
    return ex / ex.sum(axis=1, keepdims=True)


def moe_fwd(x, Wg, We1, We2, live, best, D, H, E):
    """or_moe_fwd's formula in float64 with the given expert per token
    (best < 0: no live expert, zero output)."""
    X = x.reshape(-1, D)
    Wg, We1, We2 = Wg.reshape(D, E), We1.reshape(E, D, H), We2.reshape(E, H, D)
    p = _moe_probs(X, Wg, live)
    out = np.zeros_like(X)
    for e in np.unique(best[best >= 0]):
        t = best == e
        u = X[t] @ We1[e]
        out[t] = p[t, e][:, None] * ((0.5 * u * (1.0 + _erf(u * _MOE_C))) @ We2[e])
    return out.ravel()


def moe_bwd(dout, x, Wg, We1, We2, live, best, D, H, E):
    """or_moe_bwd's formulas in float64: (dx, dWg, dWe1, dWe2).  Per token
    with expert b: u = x We1[b], dp = We2[b] dout, g = GELU(u), g' = GELU'(u),
    dpb = g . dp, dH = dp p_b g', dG_e = p_e ([e = b] dpb - dpb p_b);
    dx = dG Wg^T + dH We1[b]^T, dWg = x^T dG, dWe1[b] = x^T dH,
    dWe2[b] = (p_b g)^T dout over the tokens of b."""
    X, G = x.reshape(-1, D), dout.reshape(-1, D)
    M = X.shape[0]
    Wg, We1, We2 = Wg.reshape(D, E), We1.reshape(E, D, H), We2.reshape(E, H, D)
    p = _moe_probs(X, Wg, live)
    DG = np.zeros((M, E))
    dx = np.zeros((M, D))
    dWe1, dWe2 = np.zeros((E, D, H)), np.zeros((E, H, D))
    for e in np.unique(best[best >= 0]):
        t = np.nonzero(best == e)[0]
        u = X[t] @ We1[e]
        dp = G[t] @ We2[e].T
        er = _erf(u * _MOE_C)
        g = 0.5 * u * (1.0 + er)
        gd = 0.5 * (1.0 + er) + u * np.exp(-u * u * 0.5) * _MOE_C2
        pb = p[t, e]
        dpb = np.sum(g * dp, axis=1)
        dH = dp * pb[:, None] * gd
        DG[t] = p[t] * (-(dpb * pb)[:, None])
        DG[t, e] += p[t, e] * dpb
        dx[t] = dH @ We1[e].T
        dWe1[e] = X[t].T @ dH
        dWe2[e] = (g * pb[:, None]).T @ G[t]
    dx += DG @ Wg.T
    return dx.ravel(), (X.T @ DG).ravel(), dWe1.ravel(), dWe2.ravel()


def train_values(net, w, x, y, moe_best=None):
    """Every value of one training step's forward and reverse bodies of
    `net` (an oracle.Net) at weights `w`, ids/inputs `x` and one-hot labels
    `y`, in float64: (values by IR id, loss).  The optimizer is not run.
    A MoE network needs `moe_best`, the float32 oracle's expert per token
    (record["moe_best"] of oracle.Model.train_step); its initial K0 experts
    are the live ones."""
    f = net.train
    wset = set(net.shape)
    w = np.asarray(w, np.float32).astype(F64)
    xs, ys = np.asarray(x, np.float32), np.asarray(y, np.float32).astype(F64)
    xid = oracle._input_id(f, wset)
    yid = next((i.operands[1] for i in f.instrs if i.op == "ns.cross_entropy"), None)
    ids = net.ids_table(f)
    buf, width, loss = {}, {}, None

    def weight(n):
        r, c = net.shape[n]
        o = net.offsets[n]
        return w[o:o + r * c]

    def val(v):
        if v == xid:
            return xs.astype(F64)
        if v == yid:
            return ys
        if v in wset:
            return weight(v)
        return buf[v]

    def cols(v):
        if v in width:
            return width[v]
        if v in wset:
            return net.shape[v][1]
        return net.in_cols if v == xid else -1

    def ce_cols(v):
        c = ids.get(v, (-1, -1))[1]
        return c if c > 0 else net.in_cols

    for i in f.instrs:
        op, o = i.op, i.operands
        if op in ("ns.tensor.alloc", "ns.grad", "ns.forward", "ns.opt.step"):
            continue
        if op == "ns.matmul":
            K, N = net._static_dims(f, o[1])
            buf[i.result] = (val(o[0]).reshape(-1, K) @ val(o[1]).reshape(K, N)).ravel()
            width[i.result] = N
        elif op.startswith("ns.activation.") and op.split(".")[-1] in oracle.ACT_CODES:
            buf[i.result] = act(val(o[0]), oracle.ACT_CODES[op.split(".")[-1]])
            width[i.result] = cols(o[0])
        elif op == "ns.layernorm":
            last = cols(o[0])
            buf[i.result] = layernorm(val(o[0]), last)
            width[i.result] = last
        elif op == "ns.layer.embedding":
            V, D = net.shape[o[0]]
            buf[i.result] = embedding(weight(o[0]), xs if o[1] == xid else val(o[1]), V, D)
            width[i.result] = D
        elif op == "ns.layer.attention":
            D = net.shape[o[1]][0]
            buf[i.result] = attention_fwd(val(o[0]), *(weight(n) for n in o[1:5]), D, net.heads[o[1]])
            width[i.result] = D
        elif op == "ns.cross_entropy":
            loss = cross_entropy(val(o[0]), ys, ce_cols(o[0]))
        elif op == "ns.grad.loss":
            C = ce_cols(o[0])
            buf[i.result] = loss_grad(val(o[0]), ys, C)
            width[i.result] = C
        elif op == "ns.grad.matmul.a":
            K, N = net.shape[o[1]]
            buf[i.result] = (val(o[0]).reshape(-1, N) @ val(o[1]).reshape(K, N).T).ravel()
            width[i.result] = K
        elif op == "ns.grad.matmul.w":
            K, N = net.shape[o[2]]
            buf[i.result] = (val(o[0]).reshape(-1, K).T @ val(o[1]).reshape(-1, N)).ravel()
        elif op == "ns.grad.activation" and "dropout_mask" not in i.comment:
            code = oracle._act_of(f, o[1])
            buf[i.result] = val(o[0]) * act_deriv(val(o[1]), code)
            width[i.result] = cols(o[0])
        elif op == "ns.grad.layernorm":
            last = cols(o[1])
            buf[i.result] = layernorm_grad(val(o[0]), val(o[1]), last)
            width[i.result] = last
        elif op == "ns.grad.embedding.w":
            V, D = net.shape[o[2]]
            buf[i.result] = embedding_grad(val(o[0]), xs if o[1] == xid else val(o[1]), V, D)
        elif op == "ns.layer.moe":
            m = net.moe
            if moe_best is None:
                raise NotImplementedError("float64 MoE needs the oracle's routing (moe_best)")
            live = np.zeros(m["E"], bool)
            live[:m["K0"]] = True
            best = np.asarray(moe_best)
            buf[i.result] = moe_fwd(val(o[0]), *(weight(n) for n in o[1:4]), live, best, m["D"], m["H"], m["E"])
            width[i.result] = m["D"]
        elif op.startswith("ns.grad.moe."):
            m = net.moe
            key = ("moe", o[0], o[1])
            if key not in buf:
                live = np.zeros(m["E"], bool)
                live[:m["K0"]] = True
                buf[key] = moe_bwd(val(o[0]), val(o[1]), *(weight(n) for n in o[2:5]), live,
                                   np.asarray(moe_best), m["D"], m["H"], m["E"])
            which = {"x": 0, "wg": 1, "we1": 2, "we2": 3}[op.split(".")[-1]]
            buf[i.result] = buf[key][which]
            if which == 0:
                width[i.result] = m["D"]
        elif op.startswith("ns.grad.attention."):
            key = ("attn", o[0], o[1], o[2])
            if key not in buf:
                D = net.shape[o[2]][0]
                buf[key] = attention_bwd(val(o[0]), val(o[1]), *(weight(n) for n in o[2:6]), D,
                                         net.heads[o[2]])
            which = {"x": 0, "wq": 1, "wk": 2, "wv": 3, "wo": 4}[op.split(".")[-1]]
            buf[i.result] = buf[key][which]
            if which == 0:
                width[i.result] = net.shape[o[2]][0]
        else:
            raise NotImplementedError(f"float64 evaluation of {op}")
    return {k: v for k, v in buf.items() if isinstance(k, str)}, loss


def adamw_step(w, g, m, v, t, lr):
    """One AdamW update in float64 (codegen.cpp:3108-3119, constants the
    float32 literals of optim_params.hpp:20-32), in place on w, m, v."""
    f = lambda c: F64(np.float32(c))  # noqa: E731
    lr = f(lr)
    b1t = 1.0 - f(0.9) ** t
    b2t = 1.0 - f(0.999) ** t
    m *= f(0.9)
    m += f(0.1) * g
    v *= f(0.999)
    v += f(0.001) * g * g
    w -= lr * (m / b1t) / (np.sqrt(v / b2t) + f(1e-8)) + (f(0.01) * lr) * w
