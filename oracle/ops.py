"""numpy restatement of the hot-path ops (test oracle; see oracle/__init__).

All inputs are numpy arrays; computation is float64 so the oracle is at
least as accurate as the f32 CPU reference it stands in for.  Citations are
to files under the reference repository.
"""

from __future__ import annotations

import math

import numpy as np

_SQRT1_2 = 1.0 / math.sqrt(2.0)


def _f64(x):
    return np.asarray(x, dtype=np.float64)


# ---------------------------------------------------------------------------
# layer norm — fast_aten_native_layer_norm (eager_kernels/aten_fast.py:5248-5371),
# backward fast_aten_native_layer_norm_backward (aten_fast.py:5374-5517)
# ---------------------------------------------------------------------------
def layer_norm(x, gamma=None, beta=None, eps=1e-5):
    """y over the last dim; returns (y, mean, rstd) with biased variance."""
    x = _f64(x)
    mean = x.mean(-1, keepdims=True)
    var = ((x - mean) ** 2).mean(-1, keepdims=True)
    rstd = 1.0 / np.sqrt(var + eps)
    y = (x - mean) * rstd
    if gamma is not None:
        y = y * _f64(gamma)
    if beta is not None:
        y = y + _f64(beta)
    return y, mean, rstd


def layer_norm_backward(dy, x, mean, rstd, gamma=None):
    """(dx, dgamma, dbeta) for y = (x-mean)*rstd*gamma + beta."""
    dy, x = _f64(dy), _f64(x)
    xh = (x - mean) * rstd
    g = dy * (_f64(gamma) if gamma is not None else 1.0)
    n = x.shape[-1]
    dx = rstd * (g - g.sum(-1, keepdims=True) / n - xh * (g * xh).sum(-1, keepdims=True) / n)
    red = tuple(range(x.ndim - 1))
    return dx, (dy * xh).sum(red), dy.sum(red)


# ---------------------------------------------------------------------------
# GELU — fast_aten_gelu / gelu_backward (aten_fast.py:2940-3009;
# activation_forward_kernels.mojo:1-60, activation_backward_ops.mojo:80-233)
# ---------------------------------------------------------------------------
def _erf(x):
    return np.vectorize(math.erf, otypes=[np.float64])(x)


def gelu(x, approximate="none"):
    x = _f64(x)
    if approximate == "tanh":
        k = math.sqrt(2.0 / math.pi)
        return 0.5 * x * (1.0 + np.tanh(k * (x + 0.044715 * x**3)))
    return 0.5 * x * (1.0 + _erf(x * _SQRT1_2))


def gelu_backward(dy, x, approximate="none"):
    dy, x = _f64(dy), _f64(x)
    if approximate == "tanh":
        k = math.sqrt(2.0 / math.pi)
        inner = k * (x + 0.044715 * x**3)
        t = np.tanh(inner)
        return dy * (0.5 * (1 + t) + 0.5 * x * (1 - t * t) * k * (1 + 3 * 0.044715 * x * x))
    cdf = 0.5 * (1.0 + _erf(x * _SQRT1_2))
    pdf = np.exp(-0.5 * x * x) / math.sqrt(2 * math.pi)
    return dy * (cdf + x * pdf)


# ---------------------------------------------------------------------------
# softmax / log_softmax — fast_aten__softmax (aten_fast.py:9220-9254),
# fast_aten__log_softmax (aten_fast.py:5792-5825) and backward
# (aten_fast.py:5828-5971; softmax_backward_kernels.mojo:76-231)
# ---------------------------------------------------------------------------
def softmax(x, axis=-1):
    x = _f64(x)
    m = np.max(x, axis=axis, keepdims=True)
    e = np.exp(x - m)
    return e / e.sum(axis=axis, keepdims=True)


def log_softmax(x, axis=-1):
    x = _f64(x)
    m = np.max(x, axis=axis, keepdims=True)
    return x - m - np.log(np.exp(x - m).sum(axis=axis, keepdims=True))


def log_softmax_backward(dy, y, axis=-1):
    dy, y = _f64(dy), _f64(y)
    return dy - np.exp(y) * dy.sum(axis=axis, keepdims=True)


def softmax_backward(dy, y, axis=-1):
    dy, y = _f64(dy), _f64(y)
    return y * (dy - (dy * y).sum(axis=axis, keepdims=True))


# ---------------------------------------------------------------------------
# NLL — fast_aten_nll_loss_forward_output / _backward_grad_input
# (aten_fast.py:5974-6130; loss_ops.mojo:73-306)
# ---------------------------------------------------------------------------
def nll_loss(logp, target, weight=None, reduction="mean", ignore_index=-100):
    """(output, total_weight)."""
    logp = _f64(logp)
    target = np.asarray(target, dtype=np.int64)
    n = target.shape[0]
    valid = target != ignore_index
    t = np.where(valid, target, 0)
    w = (_f64(weight)[t] if weight is not None else np.ones(n)) * valid
    losses = -logp[np.arange(n), t] * w
    total = w.sum()
    if reduction == "none":
        return losses, total
    if reduction == "sum":
        return losses.sum(), total
    return losses.sum() / total, total


def nll_loss_backward(grad, logp_shape, target, weight=None, reduction="mean",
                      ignore_index=-100, total_weight=None):
    n, c = logp_shape
    target = np.asarray(target, dtype=np.int64)
    valid = target != ignore_index
    t = np.where(valid, target, 0)
    w = (_f64(weight)[t] if weight is not None else np.ones(n)) * valid
    g = _f64(grad)
    vals = -w * (g if reduction == "none" else g.reshape(()))
    if reduction == "mean":
        vals = vals / total_weight
    out = np.zeros((n, c))
    out[np.arange(n), t] = np.where(valid, vals, 0.0)
    return out


# ---------------------------------------------------------------------------
# embedding — fast_aten_embedding (aten_fast.py:9262-9304, Gather0
# nn_ops.mojo:1774-1796) and embedding_dense_backward (aten_fast.py:9307-9368)
# ---------------------------------------------------------------------------
def embedding(weight, idx):
    return np.asarray(weight)[np.asarray(idx, dtype=np.int64)]


def embedding_backward_f32(grad_out, idx, num_weights, padding_idx=-1):
    """Sequential f32 accumulation in index order (ATen CPU's index_add
    order), so the result is the bit pattern a sequential f32 sum gives."""
    g = np.asarray(grad_out, dtype=np.float32).reshape(-1, np.asarray(grad_out).shape[-1])
    ids = np.asarray(idx, dtype=np.int64).reshape(-1)
    out = np.zeros((num_weights, g.shape[1]), dtype=np.float32)
    for n, r in enumerate(ids):
        if r != padding_idx:
            out[r] += g[n]
    return out


# ---------------------------------------------------------------------------
# attention — fused flash attention forward/backward
# (flash_attention_fwd_kernels.mojo:885-963, flash_attention_bwd_kernels.mojo:
# 13-26 math, 63-66 top-left causal, 1403-1404 natural-log LSE)
# ---------------------------------------------------------------------------
def _kv_heads(q, x):
    """Grouped-query attention: K/V with H_kv heads serve H_q = g*H_kv query
    heads, query head h reading K/V head h // g (torch SDPA enable_gqa)."""
    x = _f64(x)
    hq, hk = np.asarray(q).shape[-3], x.shape[-3]
    if hk == hq:
        return x
    assert hq % hk == 0, (hq, hk)
    return np.repeat(x, hq // hk, axis=-3)


def _scores(q, k, scale, causal, window=0):
    s = np.einsum("...id,...jd->...ij", _f64(q), _kv_heads(q, k)) * scale
    if causal:
        sq, skv = s.shape[-2], s.shape[-1]
        i, j = np.arange(sq)[:, None], np.arange(skv)[None, :]
        mask = j > i  # top-left
        if window:
            mask = mask | (i - j >= window)  # sliding window: keys i-window+1 .. i
        s = np.where(mask, -np.inf, s)
    return s


def sdpa_forward(q, k, v, scale=None, causal=False, window=0):
    """(O, LSE) with LSE the natural-log row log-sum-exp.  K/V may have fewer
    heads than Q (grouped-query attention); `window` > 0 (causal only) keeps
    keys i-window+1 .. i for query i, the sliding-window mask of the Gemma-3
    shaped workload (which the reference runs through its masked-math
    decomposition, aten_fast.py:9112-9123, :6869)."""
    d = q.shape[-1]
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    s = _scores(q, k, scale, causal, window)
    m = s.max(-1, keepdims=True)
    e = np.exp(s - m)
    lse = (m + np.log(e.sum(-1, keepdims=True)))[..., 0]
    p = np.exp(s - lse[..., None])
    return np.einsum("...ij,...jd->...id", p, _kv_heads(q, v)), lse


def sdpa_backward(do, q, k, v, o, lse, scale=None, causal=False, window=0):
    """(dQ, dK, dV) recomputing P from LSE and D_i = sum(dO*O).  With grouped
    K/V heads (K/V with H/g heads), dK and dV of K/V head h sum the
    contributions of query heads h*g .. h*g+g-1; `window` as in
    sdpa_forward."""
    d = q.shape[-1]
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    s = _scores(q, k, scale, causal, window)
    p = np.exp(s - _f64(lse)[..., None])
    do, o = _f64(do), _f64(o)
    kk, vv = _kv_heads(q, k), _kv_heads(q, v)
    dv = np.einsum("...ij,...id->...jd", p, do)
    dp = np.einsum("...id,...jd->...ij", do, vv)
    delta = (do * o).sum(-1, keepdims=True)
    ds = p * (dp - delta)
    dq = scale * np.einsum("...ij,...jd->...id", ds, kk)
    dk = scale * np.einsum("...ij,...id->...jd", ds, _f64(q))
    hk = np.asarray(k).shape[-3]
    if hk != q.shape[-3]:  # fold the query heads of each group onto their K/V head
        g = q.shape[-3] // hk
        dk = dk.reshape(dk.shape[:-3] + (hk, g) + dk.shape[-2:]).sum(-3)
        dv = dv.reshape(dv.shape[:-3] + (hk, g) + dv.shape[-2:]).sum(-3)
    return dq, dk, dv


# ---------------------------------------------------------------------------
# RMSNorm — the Gemma-3-shaped workload's norm.  The reference has no eager
# RMSNorm kernel; this follows torch.nn.functional.rms_norm:
# y = x / sqrt(mean(x^2 over the last dim) + eps) * weight.
# ---------------------------------------------------------------------------
def rms_norm(x, weight=None, eps=1e-6):
    """y over the last dim; returns (y, rstd)."""
    x = _f64(x)
    rstd = 1.0 / np.sqrt((x * x).mean(-1, keepdims=True) + eps)
    y = x * rstd
    if weight is not None:
        y = y * _f64(weight)
    return y, rstd[..., 0]


def rms_norm_backward(dy, x, weight=None, eps=1e-6, weight_offset=0.0):
    """(dx, dweight) of rms_norm with scale (weight + weight_offset): the
    chain rule through y = x r s, r = (mean(x^2) + eps)^-1/2."""
    dy, x = _f64(dy), _f64(x)
    n = x.shape[-1]
    r = 1.0 / np.sqrt((x * x).mean(-1, keepdims=True) + eps)
    s = (_f64(weight) + weight_offset) if weight is not None else np.ones(n)
    gs = dy * s
    dx = r * gs - x * r**3 * (gs * x).sum(-1, keepdims=True) / n
    dw = (dy * x * r).reshape(-1, n).sum(0) if weight is not None else None
    return dx, dw


# ---------------------------------------------------------------------------
# GEMM — fast_aten_mm / addmm / bmm (aten_fast.py:8713-8935)
# ---------------------------------------------------------------------------
def addmm(a, b, bias=None):
    c = _f64(a) @ _f64(b)
    if bias is not None:
        c = c + _f64(bias)
    return c


# ---------------------------------------------------------------------------
# AdamW — _fused_adamw_f32 update rule (optimizer_kernels.mojo:59-74,100-132)
# ---------------------------------------------------------------------------
def adamw_step(p, g, m, v, step, lr, beta1, beta2, weight_decay, eps, maximize=False,
               amsgrad=False, vmax=None, grad_scale=None):
    """One AdamW update of (p, m, v[, vmax]) at the already-incremented step."""
    p, g, m, v = _f64(p).copy(), _f64(g).copy(), _f64(m).copy(), _f64(v).copy()
    if grad_scale is not None:
        g = g / grad_scale
    if maximize:
        g = -g
    if weight_decay != 0.0:  # IEEE guard: no 0*inf when decay is off
        p = p - lr * weight_decay * p
    m = beta1 * m + (1 - beta1) * g
    v = beta2 * v + (1 - beta2) * g * g
    bc1 = 1 - beta1**step
    bc2 = 1 - beta2**step
    vv = v
    if amsgrad:
        vmax = np.maximum(_f64(vmax), v)
        vv = vmax
    denom = np.sqrt(vv) / math.sqrt(bc2) + eps
    p = p - (lr / bc1) * m / denom
    return (p, m, v, vmax) if amsgrad else (p, m, v)


def l2_norm(x):
    return float(np.sqrt((_f64(x) ** 2).sum()))
