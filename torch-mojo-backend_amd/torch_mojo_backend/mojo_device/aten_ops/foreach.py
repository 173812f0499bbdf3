"""``_foreach_*`` registrations (reference: aten_ops/foreach.py:14-77 and the
batched kernels behind aten_fast.py:515-971).

The common regimes (contiguous same-dtype f32/bf16/f16 lists) go to one
batched library call; anything else (mixed dtypes, strided tensors, aliasing
lists, overloads without a batched form) falls back to ATen's sequential
semantics, op by op on the device.
"""

from __future__ import annotations

from ...eager_kernels import aten_fast as F
from ...eager_kernels.aten_fast import NOT_HANDLED


def _seq_binary(name, a_list, other, alpha=1):
    for i, a in enumerate(a_list):
        o = other[i] if isinstance(other, (list, tuple)) else other
        F._binary(name, a, o, alpha, inplace=True)


def _try(fn, *args, **kwargs):
    return fn(*args, **kwargs) is not NOT_HANDLED


def _no_alias(*lists):
    ids = set()
    for lst in lists:
        for t in lst:
            key = getattr(t, "_ptr", None)
            if key in ids:
                return False
            ids.add(key)
    return True


def _inplace(op_name, self, *args, **kwargs):
    overload = op_name.split(".", 1)[1] if "." in op_name else "default"
    base = op_name.split("::")[1].split(".")[0]
    a = list(self)
    if not a:
        return None
    if base in ("_foreach_add_", "_foreach_sub_"):
        sign = 1.0 if base == "_foreach_add_" else -1.0
        if overload == "Scalar":
            if _try(F.foreach_apply, "add", a, s0=sign * float(F._scalar_value(args[0]))):
                return None
            return _seq_binary("add", a, args[0], sign)
        if overload == "List":
            alpha = kwargs.get("alpha", args[1] if len(args) > 1 else 1)
            other = list(args[0])
            if _no_alias(a) and _try(F.foreach_apply, "add", a, other, s0=sign * float(alpha)):
                return None
            return _seq_binary("add", a, other, sign * alpha)
        if overload == "Tensor":
            alpha = kwargs.get("alpha", args[1] if len(args) > 1 else 1)
            return _seq_binary("add", a, args[0], sign * alpha)
        if overload == "ScalarList":
            return _seq_binary("add", a, [sign * float(s) for s in args[0]])
    if base in ("_foreach_mul_", "_foreach_div_"):
        kind = "mul" if base == "_foreach_mul_" else "div"
        if overload == "Scalar":
            if _try(F.foreach_apply, kind, a, s0=float(F._scalar_value(args[0]))):
                return None
            return _seq_binary(kind, a, args[0])
        if overload == "List":
            other = list(args[0])
            if _no_alias(a) and _try(F.foreach_apply, kind, a, other):
                return None
            return _seq_binary(kind, a, other)
        if overload == "Tensor":
            if kind == "mul" and _try(F.foreach_mul_deferred, a, args[0]):
                return None
            if _try(F.foreach_apply, kind, a, tensor_scalar=args[0]):
                return None
            return _seq_binary(kind, a, args[0])
        if overload == "ScalarList":
            if _try(F.foreach_apply, kind, a, scalars=list(args[0])):
                return None
            return _seq_binary(kind, a, list(args[0]))
    if base == "_foreach_lerp_":
        ends = list(args[0])
        w = args[1]
        if overload == "Scalar":
            if _no_alias(a) and _try(F.foreach_apply, "lerp", a, ends, s0=float(w)):
                return None
            for x, e in zip(a, ends):
                F.fast_aten_lerp(x, e, w, inplace=True)
            return None
        for x, e, wi in zip(a, ends, list(w)):
            F.fast_aten_lerp(x, e, wi, inplace=True)
        return None
    if base in ("_foreach_addcmul_", "_foreach_addcdiv_"):
        kind = "addcmul" if base == "_foreach_addcmul_" else "addcdiv"
        t1, t2 = list(args[0]), list(args[1])
        value = args[2] if len(args) > 2 else kwargs.get("value", kwargs.get("scalars", 1))
        if overload == "Scalar":
            if _no_alias(a) and _try(F.foreach_apply, kind, a, t1, t2, s0=float(value)):
                return None
            for x, p, q in zip(a, t1, t2):
                F._ternary(kind, x, p, q, value, True)
            return None
        if overload == "ScalarList":
            scal = list(value)
            if _no_alias(a) and _try(F.foreach_apply, kind, a, t1, t2, scalars=scal):
                return None
            for x, p, q, s in zip(a, t1, t2, scal):
                F._ternary(kind, x, p, q, s, True)
            return None
    if base == "_foreach_sqrt_":
        if _try(F.foreach_apply, "sqrt", a):
            return None
        for x in a:
            F._unary("sqrt", x, inplace=True)
        return None
    if base == "_foreach_zero_":
        for x in a:
            F.fill_(F._require(x), 0)
        return None
    if base == "_foreach_copy_":
        for x, s in zip(a, list(args[0])):
            F.fast_aten_copy_(x, s)
        return None
    raise NotImplementedError(f"{op_name} is not supported by the mojo eager device")


def inplace_dispatcher(op_name: str):
    def dispatcher(self, *args, **kwargs):
        return _inplace(op_name, self, *args, **kwargs)

    dispatcher.__name__ = op_name.replace("::", "_").replace(".", "_")
    return dispatcher


def functional_dispatcher(op_name: str):
    """`_foreach_<op>.<ov>` = clone each input, then the in-place form."""
    base, _, overload = op_name.partition(".")
    name = base.split("::")[1]

    def dispatcher(self, *args, **kwargs):
        outs = [F.fast_aten_clone(x) for x in self]
        if name == "_foreach_neg":
            return [F._unary("neg", x, inplace=True) for x in outs]
        if name == "_foreach_abs":
            return [F._unary("abs", x, inplace=True) for x in outs]
        if name == "_foreach_maximum":
            return [F._binary("maximum", x, args[0], inplace=True) for x in outs]
        inplace = f"aten::{name}_" + (f".{overload}" if overload else "")
        _inplace(inplace, outs, *args, **kwargs)
        return outs

    dispatcher.__name__ = op_name.replace("::", "_").replace(".", "_")
    return dispatcher


def foreach_norm(self, ord=2, dtype=None):
    res = F.fast_aten__foreach_norm(list(self), ord, dtype)
    if res is NOT_HANDLED:
        return [F.fast_aten_linalg_vector_norm(x, ord, None, False, dtype=dtype) for x in self]
    return res
