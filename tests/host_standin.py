"""Host stand-in for the kernel library, for CPU-only tests of the host layer.

It implements the C ABI of include/mi355x_kernels.h over host memory with
stock PyTorch CPU ops, so the Python device layer (dispatch, views, autograd
and autocast wiring, argument packing) can be exercised without a GPU.  It
checks the ABI contract (pointer/stride/shape meaning, workspace sizes) but
says nothing about the gfx950 kernels themselves: those are covered by the
`gpu`-marked parity tests.  Never used outside tests.
"""

from __future__ import annotations

import ctypes
import math

import torch

DT = {
    0: torch.float32, 1: torch.bfloat16, 2: torch.float16, 3: torch.float64, 4: torch.int64,
    5: torch.int32, 6: torch.int16, 7: torch.int8, 8: torch.uint8, 9: torch.bool,
}


def _val(x):
    if x is None:
        return None
    if isinstance(x, ctypes.c_void_p):
        return x.value
    return int(x) if not isinstance(x, float) else x


def _arr(a, n):
    return [int(a[i]) for i in range(n)]


def view(ptr, dtype, shape, strides):
    shape = tuple(int(s) for s in shape)
    strides = tuple(int(s) for s in strides)
    if math.prod(shape) == 0:
        return torch.empty(shape, dtype=dtype)
    extent = 1 + sum((s - 1) * st for s, st in zip(shape, strides))
    nbytes = extent * dtype.itemsize
    buf = (ctypes.c_uint8 * nbytes).from_address(int(ptr))
    base = torch.frombuffer(buf, dtype=torch.uint8).view(dtype)
    return base.as_strided(shape, strides)


def dense(ptr, dtype, shape):
    strides = []
    acc = 1
    for s in reversed(shape):
        strides.append(acc)
        acc *= max(s, 1)
    return view(ptr, dtype, shape, tuple(reversed(strides)))


def _compute(dts, out_dt):
    if out_dt == torch.float64 or torch.float64 in dts:
        return torch.float64
    if out_dt.is_floating_point or any(d.is_floating_point for d in dts):
        return torch.float32
    return torch.int64


class HostStandIn:
    """Attribute access mirrors ctypes.CDLL of libmi355x_kernels.so."""

    def __init__(self):
        self.error = b""
        self.calls: dict[str, int] = {}

    def __getattribute__(self, name):
        if name.startswith("mi355x_"):
            calls = object.__getattribute__(self, "calls")
            calls[name] = calls.get(name, 0) + 1
        return object.__getattribute__(self, name)

    def mi355x_abi_version(self):
        return 1

    def mi355x_last_error(self):
        return self.error

    def mi355x_target(self):
        return b"host"

    def mi355x_source_hash(self):
        return b"host"

    # ---- data movement ----
    def mi355x_copy(self, dst, ddt, dst_st, src, sdt, src_st, shape, ndim, stream):
        shp = _arr(shape, ndim)
        d = view(_val(dst), DT[ddt], shp, _arr(dst_st, ndim))
        s = view(_val(src), DT[sdt], shp, _arr(src_st, ndim))
        d.copy_(s.to(d.dtype))
        return 0

    def mi355x_fill(self, dst, dt, strides, shape, ndim, value, stream):
        view(_val(dst), DT[dt], _arr(shape, ndim), _arr(strides, ndim)).fill_(value)
        return 0

    def mi355x_arange(self, dst, dt, n, start, step, stream):
        out = dense(_val(dst), DT[dt], (n,))
        out.copy_((start + step * torch.arange(n, dtype=torch.float64)).to(DT[dt]))
        return 0

    _BIN = {
        0: lambda a, b, s0, s1: a + s0 * b, 1: lambda a, b, s0, s1: a - s0 * b,
        2: lambda a, b, s0, s1: a * b, 3: lambda a, b, s0, s1: a / b,
        4: lambda a, b, s0, s1: torch.maximum(a, b), 5: lambda a, b, s0, s1: torch.minimum(a, b),
        6: lambda a, b, s0, s1: torch.pow(a, b), 7: lambda a, b, s0, s1: a == b,
        8: lambda a, b, s0, s1: a != b, 9: lambda a, b, s0, s1: a < b, 10: lambda a, b, s0, s1: a <= b,
        11: lambda a, b, s0, s1: a > b, 12: lambda a, b, s0, s1: a >= b,
        13: lambda a, b, s0, s1: torch.logical_and(a, b), 14: lambda a, b, s0, s1: torch.logical_or(a, b),
        15: lambda a, b, s0, s1: torch.logical_xor(a, b), 16: lambda a, b, s0, s1: a & b,
        17: lambda a, b, s0, s1: a | b, 18: lambda a, b, s0, s1: a ^ b,
        19: lambda a, b, s0, s1: torch.remainder(a, b), 20: lambda a, b, s0, s1: torch.floor_divide(a, b),
        21: lambda a, b, s0, s1: torch.div(a, b, rounding_mode="trunc"),
        22: lambda a, b, s0, s1: torch.div(a, b, rounding_mode="floor"),
    }
    _UN = {
        60: lambda a, s0, s1: a, 61: torch.neg, 62: torch.abs, 63: torch.exp, 64: torch.log,
        65: torch.sqrt, 66: torch.rsqrt, 67: torch.reciprocal, 68: torch.sin, 69: torch.cos,
        70: torch.tanh, 71: torch.sigmoid, 72: torch.erf, 73: torch.relu,
        74: torch.nn.functional.silu, 75: torch.log1p, 76: torch.expm1, 77: torch.floor,
        78: torch.ceil, 79: torch.round, 80: torch.trunc, 81: torch.sign,
        82: lambda a, s0, s1: torch.pow(a, s0), 83: lambda a, s0, s1: torch.clamp(a, s0, s1),
        84: torch.logical_not, 85: torch.bitwise_not, 86: torch.isnan, 87: torch.isinf,
        88: torch.isfinite, 89: torch.tan, 90: torch.atan, 91: torch.asin, 92: torch.acos,
        93: torch.sinh, 94: torch.cosh, 95: torch.asinh, 96: torch.acosh, 97: torch.atanh,
        98: torch.log2, 99: torch.exp2, 100: torch.log10, 101: torch.square,
        102: lambda a, s0, s1: torch.clamp(a, min=s0), 103: lambda a, s0, s1: torch.clamp(a, max=s0),
        104: lambda a, s0, s1: s0 - a * s1,
    }

    def mi355x_map(self, op, out, out_dt, nin, ins, in_dts, strides, shape, ndim, s0, s1, stream):
        shp = _arr(shape, ndim)
        st = _arr(strides, (nin + 1) * ndim)
        o = view(_val(out), DT[out_dt], shp, st[:ndim])
        dts = [DT[in_dts[j]] for j in range(nin)]
        cdt = _compute(dts, DT[out_dt])
        xs = []
        for j in range(nin):
            p = ins[j]
            if p is None or p == 0:
                xs.append(torch.full(shp, s1, dtype=cdt))
            else:
                xs.append(view(p, dts[j], shp, st[(j + 1) * ndim : (j + 2) * ndim]).to(cdt))
        if cdt != torch.int64:
            s0c, s1c = float(s0), float(s1)
        else:
            s0c, s1c = int(s0), int(s1)
        if op in self._BIN:
            r = self._BIN[op](xs[0], xs[1], s0c, s1c)
        elif op == 40:
            r = torch.where(xs[0] != 0, xs[1], xs[2])
        elif op == 41:
            r = xs[0] + s0c * xs[1] * xs[2]
        elif op == 42:
            r = xs[0] + s0c * (xs[1] / xs[2])
        elif op == 43:
            r = torch.lerp(xs[0], xs[1], s0c)
        else:
            fn = self._UN[op]
            try:
                r = fn(xs[0], s0c, s1c)
            except TypeError:
                r = fn(xs[0])
        o.copy_(r.to(o.dtype) if isinstance(r, torch.Tensor) else torch.tensor(r))
        return 0

    # ---- reductions ----
    def mi355x_reduce_workspace_bytes(self, o, r, i):
        return 0

    def mi355x_reduce(self, op, out, out_dt, inp, in_dt, outer, r, inner, so, sr, si, ws, wsb, stream):
        x = view(_val(inp), DT[in_dt], (outer, r, inner), (so, sr, si))
        acc = torch.float64 if DT[in_dt] == torch.float64 else (torch.float32 if DT[in_dt].is_floating_point else torch.int64)
        xa = x.to(acc)
        if op == 0:
            res = xa.sum(1)
        elif op == 1:
            res = xa.mean(1)
        elif op == 2:
            res = xa.amax(1)
        elif op == 3:
            res = xa.amin(1)
        elif op == 4:
            res = xa.float().pow(2).sum(1).sqrt()
        elif op == 5:
            res = xa.pow(2).sum(1)
        elif op == 6:
            res = xa.abs().amax(1)
        elif op == 7:
            res = xa.prod(1)
        elif op == 8:
            res = (xa != 0).any(1)
        elif op == 9:
            res = (xa != 0).all(1)
        else:
            res = xa.abs().sum(1)
        dense(_val(out), DT[out_dt], (outer, inner)).copy_(res.to(DT[out_dt]))
        return 0

    def mi355x_argreduce(self, is_min, out_idx, out_val, inp, dt, outer, r, inner, so, sr, si, stream):
        x = view(_val(inp), DT[dt], (outer, r, inner), (so, sr, si))
        vals, idx = (x.min(1) if is_min else x.max(1))
        dense(_val(out_idx), torch.int64, (outer, inner)).copy_(idx)
        if out_val:
            dense(_val(out_val), DT[dt], (outer, inner)).copy_(vals)
        return 0

    def mi355x_index_select(self, out, inp, dt, idx, outer, n_idx, rows, inner, so, sj, err, stream):
        ids = dense(_val(idx), torch.int64, (n_idx,))
        if ((ids < 0) | (ids >= rows)).any():
            if err:
                dense(_val(err), torch.int32, (1,)).fill_(1)
            ids = ids.clamp(0, max(rows - 1, 0))
        x = view(_val(inp), DT[dt], (outer, rows, inner), (so, sj, 1))
        dense(_val(out), DT[dt], (outer, n_idx, inner)).copy_(x[:, ids, :])
        return 0

    def mi355x_embedding_fwd(self, out, w, dt, idx, n, num, dim, wrs, err, stream):
        ids = dense(_val(idx), torch.int64, (n,))
        if ((ids < 0) | (ids >= num)).any():
            if err:
                dense(_val(err), torch.int32, (1,)).fill_(1)
            ids = ids.clamp(0, num - 1)
        W = view(_val(w), DT[dt], (num, dim), (wrs, 1))
        dense(_val(out), DT[dt], (n, dim)).copy_(W[ids])
        return 0

    def mi355x_embedding_bwd_workspace_bytes(self, n, num):
        return 16

    def mi355x_embedding_bwd(self, gw, go, dt, idx, n, num, dim, pad, ws, wsb, stream):
        ids = dense(_val(idx), torch.int64, (n,))
        g = dense(_val(go), DT[dt], (n, dim)).float()
        acc = torch.zeros(num, dim).index_add_(0, ids, g)
        if pad >= 0:
            acc[pad] = 0
        dense(_val(gw), DT[dt], (num, dim)).copy_(acc)
        return 0

    def mi355x_embedding_bwd_accumulate(self, gw, base, go, dt, idx, n, num, dim, pad, ws, wsb, stream):
        ids = dense(_val(idx), torch.int64, (n,))
        g = dense(_val(go), DT[dt], (n, dim)).float()
        acc = torch.zeros(num, dim).index_add_(0, ids, g).to(DT[dt]).float()
        rows = torch.unique(ids)
        rows = rows[rows != pad]
        B = dense(_val(base), DT[dt], (num, dim)).clone()
        B[rows] = (B[rows].float() + acc[rows]).to(DT[dt])
        dense(_val(gw), DT[dt], (num, dim)).copy_(B)
        return 0

    # ---- norms / activations ----
    def mi355x_layer_norm_fwd_ex(self, y, y_low, low_dt, mean, rstd, x, g, b, rows, cols, eps, dt, stream):
        self.mi355x_layer_norm_fwd(y, mean, rstd, x, g, b, rows, cols, eps, dt, stream)
        if y_low:
            dense(_val(y_low), DT[low_dt], (rows, cols)).copy_(self.last_ln_y)
        return 0

    def mi355x_add_cast(self, out, low, low_dt, a, r, r_dt, n, stream):
        self.add_cast_calls = getattr(self, "add_cast_calls", 0) + 1
        A = dense(_val(a), torch.float32, (n,))
        R = dense(_val(r), DT[r_dt], (n,)).float()
        O = A + R
        dense(_val(out), torch.float32, (n,)).copy_(O)
        dense(_val(low), DT[low_dt], (n,)).copy_(O.to(DT[low_dt]))
        return 0

    def mi355x_layer_norm_fwd_add(self, y, y_low, low_dt, mean, rstd, x_out, a, r, r_dt, g, b, rows, cols, eps,
                                  dt, stream):
        self.fused_add_calls = getattr(self, "fused_add_calls", 0) + 1
        A = dense(_val(a), DT[dt], (rows, cols))
        R = dense(_val(r), DT[r_dt], (rows, cols)).float()
        dense(_val(x_out), DT[dt], (rows, cols)).copy_(A.float() + R)
        return self.mi355x_layer_norm_fwd_ex(y, y_low, low_dt, mean, rstd, x_out, g, b, rows, cols, eps, dt, stream)

    def mi355x_layer_norm_apply(self, y, x, mean, rstd, g, b, rows, cols, dt, stream):
        X = dense(_val(x), DT[dt], (rows, cols)).float()
        mu = dense(_val(mean), torch.float32, (rows, 1))
        r = dense(_val(rstd), torch.float32, (rows, 1))
        Y = (X - mu) * r
        if g:
            Y = Y * dense(_val(g), DT[dt], (cols,)).float()
        if b:
            Y = Y + dense(_val(b), DT[dt], (cols,)).float()
        dense(_val(y), DT[dt], (rows, cols)).copy_(Y)
        return 0

    def mi355x_layer_norm_fwd(self, y, mean, rstd, x, g, b, rows, cols, eps, dt, stream):
        X = dense(_val(x), DT[dt], (rows, cols)).float()
        mu = X.mean(1, keepdim=True)
        var = ((X - mu) ** 2).mean(1, keepdim=True)
        r = 1.0 / torch.sqrt(var + eps)
        Y = (X - mu) * r
        if g:
            Y = Y * dense(_val(g), DT[dt], (cols,)).float()
        if b:
            Y = Y + dense(_val(b), DT[dt], (cols,)).float()
        self.last_ln_y = Y.to(DT[dt])
        if y:
            dense(_val(y), DT[dt], (rows, cols)).copy_(Y)
        if mean:
            dense(_val(mean), torch.float32, (rows,)).copy_(mu[:, 0])
        if rstd:
            dense(_val(rstd), torch.float32, (rows,)).copy_(r[:, 0])
        return 0

    def mi355x_layer_norm_bwd_workspace_bytes(self, rows, cols):
        return 8 * cols

    def mi355x_layer_norm_bwd(self, dx, dg, db, dy, x, mean, rstd, g, rows, cols, dt, ws, wsb, stream):
        X = dense(_val(x), DT[dt], (rows, cols)).float()
        DY = dense(_val(dy), DT[dt], (rows, cols)).float()
        mu = dense(_val(mean), torch.float32, (rows, 1))
        rs = dense(_val(rstd), torch.float32, (rows, 1))
        xh = (X - mu) * rs
        G = dense(_val(g), DT[dt], (cols,)).float() if g else torch.ones(cols)
        gy = DY * G
        if dx:
            DX = rs * (gy - gy.mean(1, keepdim=True) - xh * (gy * xh).mean(1, keepdim=True))
            dense(_val(dx), DT[dt], (rows, cols)).copy_(DX)
        if dg:
            dense(_val(dg), DT[dt], (cols,)).copy_((DY * xh).sum(0))
        if db:
            dense(_val(db), DT[dt], (cols,)).copy_(DY.sum(0))
        return 0

    def mi355x_gelu_fwd(self, y, x, n, approx, dt, stream):
        X = dense(_val(x), DT[dt], (n,)).float()
        Y = torch.nn.functional.gelu(X, approximate="tanh" if approx else "none")
        dense(_val(y), DT[dt], (n,)).copy_(Y)
        return 0

    def mi355x_gelu_bwd(self, dx, dy, x, n, approx, dt, stream):
        X = dense(_val(x), DT[dt], (n,)).float()
        DY = dense(_val(dy), DT[dt], (n,)).float()
        DX = torch.ops.aten.gelu_backward(DY, X, approximate="tanh" if approx else "none")
        dense(_val(dx), DT[dt], (n,)).copy_(DX)
        return 0

    def mi355x_softmax_fwd(self, y, ydt, x, xdt, rows, cols, log, stream):
        X = dense(_val(x), DT[xdt], (rows, cols)).float()
        Y = torch.log_softmax(X, 1) if log else torch.softmax(X, 1)
        dense(_val(y), DT[ydt], (rows, cols)).copy_(Y)
        return 0

    def mi355x_softmax_bwd(self, dx, dxdt, dy, dydt, y, ydt, rows, cols, log, stream):
        DY = dense(_val(dy), DT[dydt], (rows, cols)).float()
        Y = dense(_val(y), DT[ydt], (rows, cols)).float()
        if log:
            DX = DY - torch.exp(Y) * DY.sum(1, keepdim=True)
        else:
            DX = Y * (DY - (DY * Y).sum(1, keepdim=True))
        dense(_val(dx), DT[dxdt], (rows, cols)).copy_(DX)
        return 0

    def mi355x_nll_workspace_bytes(self, n):
        return 16

    def mi355x_nll_fwd(self, out, tw, lp, dt, tgt, w, n, c, red, ign, err, ws, wsb, stream):
        LP = dense(_val(lp), DT[dt], (n, c)).float()
        T = dense(_val(tgt), torch.int64, (n,))
        W = dense(_val(w), DT[dt], (c,)).float() if w else None
        valid = T != ign
        if ((T[valid] < 0) | (T[valid] >= c)).any() and err:
            dense(_val(err), torch.int32, (1,)).fill_(1)
        Tc = torch.where(valid, T, torch.zeros_like(T)).clamp(0, c - 1)
        wt = (W[Tc] if W is not None else torch.ones(n)) * valid.float()
        losses = -LP.gather(1, Tc[:, None])[:, 0] * wt
        if red == 0:
            dense(_val(out), DT[dt], (n,)).copy_(losses)
        elif red == 1:
            dense(_val(out), DT[dt], ()).copy_(losses.sum() / wt.sum())
        else:
            dense(_val(out), DT[dt], ()).copy_(losses.sum())
        dense(_val(tw), DT[dt], ()).copy_(wt.sum())
        return 0

    def mi355x_nll_bwd(self, gi, go, tgt, w, tw, n, c, red, ign, dt, stream):
        T = dense(_val(tgt), torch.int64, (n,))
        W = dense(_val(w), DT[dt], (c,)).float() if w else None
        valid = T != ign
        Tc = torch.where(valid, T, torch.zeros_like(T)).clamp(0, c - 1)
        wt = (W[Tc] if W is not None else torch.ones(n)) * valid.float()
        G = torch.zeros(n, c)
        if red == 0:
            g = dense(_val(go), DT[dt], (n,)).float()
            vals = -wt * g
        else:
            g = dense(_val(go), DT[dt], ()).float()
            vals = -wt * g
            if red == 1:
                vals = vals / dense(_val(tw), DT[dt], ()).float()
        G[torch.arange(n), Tc] = vals
        dense(_val(gi), DT[dt], (n, c)).copy_(G)
        return 0

    def mi355x_cross_entropy_workspace_bytes(self, n):
        return 8 * n + 256

    def mi355x_cross_entropy_fwd(self, out, tw, lse, x, dt, ld, tgt, n, c, red, ign, err, ws, wsb, stream):
        X = view(_val(x), DT[dt], (n, c), (ld, 1)).float()
        T = dense(_val(tgt), torch.int64, (n,))
        L = torch.logsumexp(X, 1)
        dense(_val(lse), torch.float32, (n,)).copy_(L)
        valid = T != ign
        if ((T[valid] < 0) | (T[valid] >= c)).any() and err:
            dense(_val(err), torch.int32, (1,)).fill_(1)
        Tc = torch.where(valid, T, torch.zeros_like(T)).clamp(0, c - 1)
        rows = (L - X.gather(1, Tc[:, None])[:, 0]) * valid.float()
        w = valid.float().sum()
        if red == 0:
            dense(_val(out), torch.float32, (n,)).copy_(rows)
        else:
            dense(_val(out), torch.float32, ()).copy_(rows.sum() / w if red == 1 else rows.sum())
        dense(_val(tw), torch.float32, ()).copy_(w)
        return 0

    def mi355x_cross_entropy_fwd_bwd(self, out, tw, lse, dx, lddx, x, dt, ld, tgt, g, n, c, red, ign, err, ws, wsb,
                                     stream):
        if max((c + 2 * (16 // DT[dt].itemsize) - 2) // (16 // DT[dt].itemsize), lddx // (16 // DT[dt].itemsize)) > 8192:
            return 3  # MI355X_EUNSUPPORTED
        self.mi355x_cross_entropy_fwd(out, tw, lse, x, dt, ld, tgt, n, c, red, ign, err, ws, wsb, stream)
        return self.mi355x_cross_entropy_bwd(dx, dt, lddx, x, dt, ld, lse, tgt, g, red, tw, n, c, ign, stream)

    def mi355x_cross_entropy_bwd(self, dx, dxdt, lddx, x, dt, ld, lse, tgt, g, red, tw, n, c, ign, stream):
        X = view(_val(x), DT[dt], (n, c), (ld, 1)).float()
        T = dense(_val(tgt), torch.int64, (n,))
        L = dense(_val(lse), torch.float32, (n,))
        G = dense(_val(g), torch.float32, (n,) if red == 0 else ()).expand(n).clone()
        if red == 1:
            G = G / dense(_val(tw), torch.float32, ()).item()
        valid = (T != ign) & (T >= 0) & (T < c)
        G = G * valid.float()
        P = torch.exp(X - L[:, None])
        Tc = torch.where(valid, T, torch.zeros_like(T))
        P[torch.arange(n), Tc] -= valid.float()
        D = view(_val(dx), DT[dxdt], (n, lddx), (lddx, 1))
        D.zero_()
        D[:, :c].copy_(P * G[:, None])
        return 0

    # ---- optimizer ----
    def mi355x_fused_adamw_ex(self, descs, lows, low_dt, n, lr, lr_ptr, b1, b2, wd, eps, flags, gs, fi, gm, stream):
        if fi and dense(_val(fi), torch.float32, ()).item() != 0:
            return 0
        self.grad_mul = gm
        try:
            self.mi355x_fused_adamw(descs, n, lr, lr_ptr, b1, b2, wd, eps, flags, gs, fi, stream)
        finally:
            self.grad_mul = None
        if lows:
            arr = ctypes.cast(lows, ctypes.POINTER(ctypes.c_void_p))
            for i in range(n):
                if arr[i]:
                    m = descs[i].numel
                    dense(arr[i], DT[low_dt], (m,)).copy_(dense(descs[i].param, torch.float32, (m,)))
        return 0

    def mi355x_fused_adamw(self, descs, n, lr, lr_ptr, b1, b2, wd, eps, flags, gs, fi, stream):
        if fi and dense(_val(fi), torch.float32, ()).item() != 0:
            return 0
        if lr_ptr:
            lr = dense(_val(lr_ptr), torch.float32, ()).item()
        for i in range(n):
            d = descs[i]
            m = d.numel
            p = dense(d.param, torch.float32, (m,))
            g = dense(d.grad, torch.float32, (m,)).clone()
            gm = getattr(self, "grad_mul", None)
            if gm:
                g = g * dense(_val(gm), torch.float32, ()).item()
            if gs:
                g = g / dense(_val(gs), torch.float32, ()).item()
            if flags & 2:
                g = -g
            ea = dense(d.exp_avg, torch.float32, (m,))
            eas = dense(d.exp_avg_sq, torch.float32, (m,))
            step = dense(d.step, torch.float32, ()).item()
            p.mul_(1 - lr * wd)
            ea.lerp_(g, 1 - b1)
            eas.mul_(b2).addcmul_(g, g, value=1 - b2)
            bc1 = 1 - b1**step
            bc2 = 1 - b2**step
            denom = (eas.sqrt() / math.sqrt(bc2)).add_(eps)
            p.addcdiv_(ea, denom, value=-lr / bc1)
        return 0

    def mi355x_foreach_norm_workspace_bytes(self, numels, n):
        return 16

    def mi355x_foreach_norm(self, outs, odt, ins, idt, numels, n, ord, ws, wsb, stream):
        for i in range(n):
            x = dense(ins[i], DT[idt], (int(numels[i]),)).float()
            v = torch.linalg.vector_norm(x, ord)
            dense(outs[i], DT[odt], ()).copy_(v)
        return 0

    def mi355x_foreach_apply(self, op, a, b, c, scalars, numels, n, dt, s0, ts, stream):
        tsv = dense(_val(ts), torch.float32, ()).item() if ts else None
        for i in range(n):
            m = int(numels[i])
            A = dense(a[i], DT[dt], (m,))
            B = dense(b[i], DT[dt], (m,)).float() if b else None
            C = dense(c[i], DT[dt], (m,)).float() if c else None
            sc = float(scalars[i]) if scalars else None
            x = A.float()
            if op == 0:
                r = x + s0 * (B if B is not None else 1.0)
            elif op in (2, 3):
                f = tsv if tsv is not None else (sc if sc is not None else (B if B is not None else s0))
                r = x * f if op == 2 else x / f
            elif op == 43:
                r = torch.lerp(x, B, s0)
            elif op == 41:
                r = x + (sc if sc is not None else s0) * B * C
            elif op == 42:
                r = x + (sc if sc is not None else s0) * B / C
            else:
                r = x.sqrt()
            A.copy_(r)
        return 0

    # ---- gemm / attention ----
    def mi355x_gemm_workspace_bytes(self, a, ars, acs, abs_, b, brs, bcs, bbs, dt, batch, m, n, k):
        return 0

    def mi355x_gemm(self, c, cdt, crs, cbs, a, ars, acs, abs_, b, brs, bcs, bbs, abdt, bias, bdt,
                    beta, batch, m, n, k, ws, wsb, stream):
        A = view(_val(a), DT[abdt], (batch, m, k), (abs_, ars, acs)).float()
        B = view(_val(b), DT[abdt], (batch, k, n), (bbs, brs, bcs)).float()
        C = view(_val(c), DT[cdt], (batch, m, n), (cbs, crs, 1))
        r = torch.bmm(A, B)
        if bias:
            r = r + dense(_val(bias), DT[bdt], (n,)).float()
        if beta:
            r = r + C.float()
        C.copy_(r)
        return 0

    def mi355x_gemm_ex(self, c, cdt, crs, cbs, a, ars, acs, abs_, b, brs, bcs, bbs, abdt, bias, bdt,
                       flags, rowsum, rsdt, batch, m, n, k, ws, wsb, stream):
        A = view(_val(a), DT[abdt], (batch, m, k), (abs_, ars, acs)).float()
        B = view(_val(b), DT[abdt], (batch, k, n), (bbs, brs, bcs)).float()
        C = view(_val(c), DT[cdt], (batch, m, n), (cbs, crs, 1))
        r = torch.bmm(A, B)
        if bias:
            r = r + dense(_val(bias), DT[bdt], (n,)).float()
        if flags & 1:
            r = r + C.float()
        if flags & 2:
            r = r.to(DT[abdt]).float()
        C.copy_(r)
        if rowsum:
            rs = A.sum(2)
            if flags & 2:
                rs = rs.to(DT[abdt]).float()
            dense(_val(rowsum), DT[rsdt], (batch, m)).copy_(rs)
        return 0

    def mi355x_attn_fwd(self, o, obhs, lse, q, qbhs, k, kbhs, v, vbhs, B, H, Sq, Skv, D, scale, causal, dt, stream):
        def t(p, st, s):
            return view(_val(p), DT[dt], (B, H, s, D), (st[0], st[1], st[2], 1))

        Q, K, V = t(q, qbhs, Sq).float(), t(k, kbhs, Skv).float(), t(v, vbhs, Skv).float()
        S = Q @ K.transpose(-1, -2) * scale
        if causal:
            mask = torch.ones(Sq, Skv, dtype=torch.bool).tril()
            S = S.masked_fill(~mask, float("-inf"))
        L = torch.logsumexp(S, -1)
        P = torch.exp(S - L[..., None])
        t(o, obhs, Sq).copy_(P @ V)
        dense(_val(lse), torch.float32, (B, H, Sq)).copy_(L)
        return 0

    def mi355x_rms_norm_fwd(self, y, rstd, x, w, wdt, woff, rows, cols, eps, dt, stream):
        X = dense(_val(x), DT[dt], (rows, cols)).double()
        r = torch.rsqrt((X * X).mean(-1) + eps)
        Y = X * r[:, None]
        if w:
            Y = Y * (dense(_val(w), DT[wdt], (cols,)).double() + woff)
        dense(_val(y), DT[dt], (rows, cols)).copy_(Y.to(DT[dt]))
        if rstd:
            dense(_val(rstd), torch.float32, (rows,)).copy_(r.float())
        return 0

    def mi355x_rms_norm_bwd(self, dx, dw, dy, x, rstd, w, woff, rows, cols, dt, ws, wsb, stream):
        if cols % 4 or cols > 2048:
            return 3
        X = dense(_val(x), DT[dt], (rows, cols)).double()
        G = dense(_val(dy), DT[dt], (rows, cols)).double()
        r = dense(_val(rstd), torch.float32, (rows,)).double()[:, None]
        s = (dense(_val(w), DT[dt], (cols,)).double() + woff) if w else torch.ones(cols, dtype=torch.float64)
        gw = G * s
        DX = r * gw - X * r ** 3 * (gw * X).mean(-1, keepdim=True)
        dense(_val(dx), DT[dt], (rows, cols)).copy_(DX.to(DT[dt]))
        if dw:
            dense(_val(dw), DT[dt], (cols,)).copy_((G * X * r).sum(0).to(DT[dt]))
        return 0

    def mi355x_rope(self, y, ybht, x, xbht, cos, sin, B, H, T, D, inverse, dt, stream):
        X = view(_val(x), DT[dt], (B, H, T, D), (xbht[0], xbht[1], xbht[2], 1)).float()
        C = dense(_val(cos), DT[dt], (T, D)).float()
        S = dense(_val(sin), DT[dt], (T, D)).float()
        h = D // 2
        x1, x2 = X[..., :h], X[..., h:]
        if inverse:
            out = torch.cat([x1 * C[:, :h] + x2 * S[:, h:], x2 * C[:, h:] - x1 * S[:, :h]], -1)
        else:
            out = torch.cat([x1 * C[:, :h] - x2 * S[:, :h], x2 * C[:, h:] + x1 * S[:, h:]], -1)
        view(_val(y), DT[dt], (B, H, T, D), (ybht[0], ybht[1], ybht[2], 1)).copy_(out)
        return 0

    def mi355x_geglu_fwd(self, y, gate, up, n, approximate, dt, stream):
        g = dense(_val(gate), DT[dt], (n,))
        u = dense(_val(up), DT[dt], (n,))
        a = torch.nn.functional.gelu(g.float(), approximate="tanh" if approximate else "none").to(DT[dt])
        dense(_val(y), DT[dt], (n,)).copy_((a.float() * u.float()).to(DT[dt]))
        return 0

    def mi355x_geglu_bwd(self, dg, du, grad, gate, up, n, approximate, dt, stream):
        mode = "tanh" if approximate else "none"
        gr, g, u = (dense(_val(t), DT[dt], (n,)).float() for t in (grad, gate, up))
        a = torch.nn.functional.gelu(g, approximate=mode).to(DT[dt]).float()
        dense(_val(du), DT[dt], (n,)).copy_((gr * a).to(DT[dt]))
        gu = (gr * u).to(DT[dt]).float()
        dense(_val(dg), DT[dt], (n,)).copy_(torch.ops.aten.gelu_backward(gu, g, approximate=mode).to(DT[dt]))
        return 0

    def mi355x_attn_fwd_ex(self, o, obhs, lse, q, qbhs, k, kbhs, v, vbhs, B, H, Hk, Sq, Skv, D, scale, causal,
                           window, dt, stream):
        def t(p, st, h, s):
            return view(_val(p), DT[dt], (B, h, s, D), (st[0], st[1], st[2], 1))

        Q = t(q, qbhs, H, Sq).float()
        K = t(k, kbhs, Hk, Skv).float().repeat_interleave(H // Hk, dim=1)
        V = t(v, vbhs, Hk, Skv).float().repeat_interleave(H // Hk, dim=1)
        S = Q @ K.transpose(-1, -2) * scale
        if causal:
            i = torch.arange(Sq)[:, None]
            j = torch.arange(Skv)[None, :]
            keep = j <= i
            if window:
                keep = keep & (i - j < window)
            S = S.masked_fill(~keep, float("-inf"))
        L = torch.logsumexp(S, -1)
        P = torch.exp(S - L[..., None])
        t(o, obhs, H, Sq).copy_(P @ V)
        dense(_val(lse), torch.float32, (B, H, Sq)).copy_(L)
        return 0

    def mi355x_attn_fwd_gen(self, o, obhs, lse, q, qbhs, k, kbhs, v, vbhs, B, H, Hk, Sq, Skv, D, scale, causal,
                            window, dt, stream):
        return self.mi355x_attn_fwd_ex(o, obhs, lse, q, qbhs, k, kbhs, v, vbhs, B, H, Hk, Sq, Skv, D, scale,
                                       causal, window, dt, stream)

    def mi355x_attn_bwd_gen_workspace_bytes(self, B, H, Hk, Sq, Skv, D):
        return 16

    def mi355x_attn_bwd_gen(self, dq, dqs, dk, dks, dv, dvs, do, dos, q, qs, k, ks, v, vs, o, os_, lse,
                            B, H, Hk, Sq, Skv, D, scale, causal, window, dt, ws, wsb, stream):
        def t(p, st, h, s):
            return view(_val(p), DT[dt], (B, h, s, D), (st[0], st[1], st[2], 1))

        g = H // Hk
        Q = t(q, qs, H, Sq).float()
        K = t(k, ks, Hk, Skv).float().repeat_interleave(g, dim=1)
        V = t(v, vs, Hk, Skv).float().repeat_interleave(g, dim=1)
        O, DO = t(o, os_, H, Sq).float(), t(do, dos, H, Sq).float()
        L = dense(_val(lse), torch.float32, (B, H, Sq))
        S = Q @ K.transpose(-1, -2) * scale
        if causal:
            i = torch.arange(Sq)[:, None]
            j = torch.arange(Skv)[None, :]
            keep = j <= i
            if window:
                keep = keep & (i - j < window)
            S = S.masked_fill(~keep, float("-inf"))
        P = torch.exp(S - L[..., None])
        Dr = (DO * O).sum(-1, keepdim=True)
        dS = P * (DO @ V.transpose(-1, -2) - Dr)
        t(dq, dqs, H, Sq).copy_(dS @ K * scale)
        dK = (dS.transpose(-1, -2) @ Q * scale).view(B, Hk, g, Skv, D).sum(2)
        dV = (P.transpose(-1, -2) @ DO).view(B, Hk, g, Skv, D).sum(2)
        t(dk, dks, Hk, Skv).copy_(dK)
        t(dv, dvs, Hk, Skv).copy_(dV)
        return 0

    def mi355x_attn_bwd_workspace_bytes(self, B, H, Sq, Skv, D):
        return 16

    def mi355x_attn_bwd(self, dq, dqs, dk, dks, dv, dvs, do, dos, q, qs, k, ks, v, vs, o, os_, lse,
                        B, H, Sq, Skv, D, scale, causal, dt, ws, wsb, stream):
        def t(p, st, s):
            return view(_val(p), DT[dt], (B, H, s, D), (st[0], st[1], st[2], 1))

        Q, K, V = t(q, qs, Sq).float(), t(k, ks, Skv).float(), t(v, vs, Skv).float()
        O, DO = t(o, os_, Sq).float(), t(do, dos, Sq).float()
        L = dense(_val(lse), torch.float32, (B, H, Sq))
        S = Q @ K.transpose(-1, -2) * scale
        if causal:
            mask = torch.ones(Sq, Skv, dtype=torch.bool).tril()
            S = S.masked_fill(~mask, float("-inf"))
        P = torch.exp(S - L[..., None])
        Dr = (DO * O).sum(-1, keepdim=True)
        dP = DO @ V.transpose(-1, -2)
        dS = P * (dP - Dr)
        t(dq, dqs, Sq).copy_(dS @ K * scale)
        t(dk, dks, Skv).copy_(dS.transpose(-1, -2) @ Q * scale)
        t(dv, dvs, Skv).copy_(P.transpose(-1, -2) @ DO)
        return 0
