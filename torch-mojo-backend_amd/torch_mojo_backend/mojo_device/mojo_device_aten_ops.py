"""ATen op registrations for the eager mojo device.

Same role as the reference's registration list (torch_mojo_backend/
mojo_device/mojo_device_aten_ops.py:153-410): one entry per ``aten::`` name,
bound to a ``fast_aten_*`` host wrapper in ``eager_kernels/aten_fast.py``
(which calls the gfx950 library) or to a small adapter in ``aten_ops/``.
An entry whose wrapper returns ``NOT_HANDLED`` raises a
``NotImplementedError`` naming the op (aten_ops/support.py:104-120).

Elementwise families (binary, comparison, unary, in-place and ``out=``
overloads) are generated from tables instead of being spelled out.
"""

from __future__ import annotations

import functools
from collections.abc import Callable

import torch

from ..eager_kernels import aten_fast as F
from .aten_ops import foreach as _foreach
from .aten_ops.support import eager_impl, out_variant, unsupported

# (qualified aten name, python impl), in registration order
_aten_ops_registry: list[tuple[str, Callable]] = []

# per-op call counters (tests assert that the device impl ran)
EAGER_CALL_COUNTERS: dict[str, int] = {}
COUNT_CALLS = False


def register_aten_op(op_name: str):
    def decorator(func: Callable) -> Callable:
        if COUNT_CALLS:
            inner = func

            @functools.wraps(inner)
            def counted(*args, **kwargs):
                EAGER_CALL_COUNTERS[op_name] = EAGER_CALL_COUNTERS.get(op_name, 0) + 1
                return inner(*args, **kwargs)

            func = counted
        _aten_ops_registry.append((op_name, func))
        return func

    return decorator


def _reg(op_name: str, impl: Callable) -> None:
    register_aten_op(op_name)(eager_impl(impl, op_name))


def _op_exists(qualname: str) -> bool:
    ns, rest = qualname.split("::")
    name, _, overload = rest.partition(".")
    packet = getattr(getattr(torch.ops, ns), name, None)
    if packet is None:
        return False
    return (overload or "default") in packet.overloads()


# ---------------------------------------------------------------------------
# transfers, factories, views
# ---------------------------------------------------------------------------
for _name, _impl in [
    ("aten::_copy_from", F.fast_aten__copy_from),
    ("aten::copy_", F.fast_aten_copy_),
    ("aten::_to_copy", F.fast_aten__to_copy),
    ("aten::clone", F.fast_aten_clone),
    ("aten::_local_scalar_dense", F.fast_aten__local_scalar_dense),
    ("aten::empty.memory_format", F.fast_aten_empty_memory_format),
    ("aten::empty_strided", F.fast_aten_empty_strided),
    ("aten::empty_like", F.fast_aten_empty_like),
    ("aten::full", F.fast_aten_full),
    ("aten::zeros", F.fast_aten_zeros),
    ("aten::ones", F.fast_aten_ones),
    ("aten::zeros_like", F.fast_aten_zeros_like),
    ("aten::ones_like", F.fast_aten_ones_like),
    ("aten::full_like", F.fast_aten_full_like),
    ("aten::new_empty", F.fast_aten_new_empty),
    ("aten::new_empty_strided", F.fast_aten_new_empty_strided),
    ("aten::new_zeros", F.fast_aten_new_zeros),
    ("aten::new_ones", F.fast_aten_new_ones),
    ("aten::new_full", F.fast_aten_new_full),
    ("aten::scalar_tensor", F.fast_aten_scalar_tensor),
    ("aten::arange", F.fast_aten_arange),
    ("aten::arange.start", F.fast_aten_arange_start),
    ("aten::arange.start_step", F.fast_aten_arange_start_step),
    ("aten::fill_.Scalar", F.fast_aten_fill__scalar),
    ("aten::fill_.Tensor", F.fast_aten_fill__tensor),
    ("aten::zero_", F.fast_aten_zero_),
    ("aten::view", F.fast_aten_view),
    ("aten::_unsafe_view", F.fast_aten__unsafe_view),
    ("aten::_reshape_alias", F.fast_aten__reshape_alias),
    ("aten::as_strided", F.fast_aten_as_strided),
    ("aten::alias", F.fast_aten_alias),
    ("aten::detach", F.fast_aten_detach),
    ("aten::t", F.fast_aten_t),
    ("aten::transpose.int", F.fast_aten_transpose),
    ("aten::permute", F.fast_aten_permute),
    ("aten::expand", F.fast_aten_expand),
    ("aten::slice.Tensor", F.fast_aten_slice),
    ("aten::select.int", F.fast_aten_select),
    ("aten::split.Tensor", F.fast_aten_split),
    ("aten::split_with_sizes", F.fast_aten_split_with_sizes),
    ("aten::unbind.int", F.fast_aten_unbind),
    ("aten::squeeze", F.fast_aten_squeeze),
    ("aten::squeeze.dim", F.fast_aten_squeeze_dims),
    ("aten::squeeze.dims", F.fast_aten_squeeze_dims),
    ("aten::unsqueeze", F.fast_aten_unsqueeze),
    # reductions / index
    ("aten::sum.dim_IntList", F.fast_aten_sum),
    ("aten::sum", F.fast_aten_sum_default),
    ("aten::mean.dim", F.fast_aten_mean),
    ("aten::mean", F.fast_aten_mean_default),
    ("aten::amax", F.fast_aten_amax),
    ("aten::amin", F.fast_aten_amin),
    ("aten::max", F.fast_aten_max_default),
    ("aten::min", F.fast_aten_min_default),
    ("aten::max.dim", F.fast_aten_max_dim),
    ("aten::min.dim", F.fast_aten_min_dim),
    ("aten::argmax", F.fast_aten_argmax),
    ("aten::argmin", F.fast_aten_argmin),
    ("aten::any", F.fast_aten_any),
    ("aten::any.dim", F.fast_aten_any),
    ("aten::any.dims", F.fast_aten_any),
    ("aten::all", F.fast_aten_all),
    ("aten::all.dim", F.fast_aten_all),
    ("aten::all.dims", F.fast_aten_all),
    ("aten::linalg_vector_norm", F.fast_aten_linalg_vector_norm),
    ("aten::cat", F.fast_aten_cat),
    ("aten::stack", F.fast_aten_stack),
    ("aten::index_select", F.fast_aten_index_select),
    ("aten::index.Tensor", F.fast_aten_index_tensor),
    ("aten::where.self", F.fast_aten_where),
    ("aten::masked_fill.Scalar", F.fast_aten_masked_fill),
    ("aten::masked_fill.Tensor", F.fast_aten_masked_fill),
    ("aten::masked_fill_.Scalar", functools.partial(F.fast_aten_masked_fill, inplace=True)),
    ("aten::masked_fill_.Tensor", functools.partial(F.fast_aten_masked_fill, inplace=True)),
    ("aten::clamp", F.fast_aten_clamp),
    ("aten::clamp.Tensor", F.fast_aten_clamp),
    ("aten::clamp_", functools.partial(F.fast_aten_clamp, inplace=True)),
    ("aten::clamp_min", lambda self, min: F.fast_aten_clamp(self, min, None)),
    ("aten::clamp_max", lambda self, max: F.fast_aten_clamp(self, None, max)),
    ("aten::clamp_min_", lambda self, min: F.fast_aten_clamp(self, min, None, inplace=True)),
    ("aten::clamp_max_", lambda self, max: F.fast_aten_clamp(self, None, max, inplace=True)),
    ("aten::lerp.Scalar", F.fast_aten_lerp),
    ("aten::lerp.Tensor", F.fast_aten_lerp),
    ("aten::lerp_.Scalar", functools.partial(F.fast_aten_lerp, inplace=True)),
    ("aten::lerp_.Tensor", functools.partial(F.fast_aten_lerp, inplace=True)),
    ("aten::addcmul", lambda self, t1, t2, *, value=1: F._ternary("addcmul", self, t1, t2, value)),
    ("aten::addcdiv", lambda self, t1, t2, *, value=1: F._ternary("addcdiv", self, t1, t2, value)),
    ("aten::addcmul_", lambda self, t1, t2, *, value=1: F._ternary("addcmul", self, t1, t2, value, True)),
    ("aten::addcdiv_", lambda self, t1, t2, *, value=1: F._ternary("addcdiv", self, t1, t2, value, True)),
    ("aten::pow.Tensor_Scalar", F.fast_aten_pow_tensor_scalar),
    ("aten::pow_.Scalar", functools.partial(F.fast_aten_pow_tensor_scalar, inplace=True)),
    ("aten::pow.Scalar", F.fast_aten_pow_scalar),
    ("aten::pow.Tensor_Tensor", lambda self, exponent: F._binary("pow", self, exponent)),
    ("aten::pow_.Tensor", lambda self, exponent: F._binary("pow", self, exponent, inplace=True)),
    ("aten::rsub.Tensor", F.fast_aten_rsub),
    ("aten::rsub.Scalar", F.fast_aten_rsub),
    # nn
    ("aten::mm", F.fast_aten_mm),
    ("aten::addmm", F.fast_aten_addmm),
    ("aten::bmm", F.fast_aten_bmm),
    ("aten::native_layer_norm", F.fast_aten_native_layer_norm),
    ("aten::native_layer_norm_backward", F.fast_aten_native_layer_norm_backward),
    ("aten::gelu", F.fast_aten_gelu),
    ("aten::gelu_", F.fast_aten_gelu_),
    ("aten::gelu_backward", F.fast_aten_gelu_backward),
    ("aten::_softmax", F.fast_aten__softmax),
    ("aten::_log_softmax", F.fast_aten__log_softmax),
    ("aten::_softmax_backward_data", F.fast_aten__softmax_backward_data),
    ("aten::_log_softmax_backward_data", F.fast_aten__log_softmax_backward_data),
    ("aten::nll_loss_forward", F.fast_aten_nll_loss_forward),
    ("aten::nll_loss_backward", F.fast_aten_nll_loss_backward),
    ("aten::embedding", F.fast_aten_embedding),
    ("aten::embedding_dense_backward", F.fast_aten_embedding_dense_backward),
    ("aten::_scaled_dot_product_flash_attention", F.fast_aten__scaled_dot_product_flash_attention),
    (
        "aten::_scaled_dot_product_flash_attention_backward",
        F.fast_aten__scaled_dot_product_flash_attention_backward,
    ),
    ("aten::scaled_dot_product_attention", F.fast_aten_scaled_dot_product_attention),
    ("aten::_fused_adamw_", F.fast_aten__fused_adamw_),
    ("aten::_fused_adamw_.tensor_lr", F.fast_aten__fused_adamw_),
]:
    _reg(_name, _impl)

register_aten_op("aten::_foreach_norm.Scalar")(_foreach.foreach_norm)
for _name in (
    "_foreach_add_.Scalar", "_foreach_add_.List", "_foreach_add_.Tensor",
    "_foreach_add_.ScalarList", "_foreach_sub_.Scalar", "_foreach_sub_.List",
    "_foreach_mul_.Scalar", "_foreach_mul_.List", "_foreach_mul_.Tensor",
    "_foreach_mul_.ScalarList", "_foreach_div_.Scalar", "_foreach_div_.List",
    "_foreach_div_.ScalarList", "_foreach_div_.Tensor", "_foreach_lerp_.Scalar",
    "_foreach_lerp_.List", "_foreach_addcmul_.Scalar", "_foreach_addcmul_.ScalarList",
    "_foreach_addcdiv_.Scalar", "_foreach_addcdiv_.ScalarList", "_foreach_sqrt_",
    "_foreach_zero_", "_foreach_copy_",
):
    if _op_exists("aten::" + _name):
        register_aten_op("aten::" + _name)(_foreach.inplace_dispatcher("aten::" + _name))
for _name in (
    "_foreach_add.Scalar", "_foreach_add.List", "_foreach_mul.Scalar", "_foreach_mul.List",
    "_foreach_mul.Tensor", "_foreach_div.Scalar", "_foreach_div.List", "_foreach_div.ScalarList",
    "_foreach_sqrt", "_foreach_addcdiv.ScalarList", "_foreach_addcdiv.Scalar", "_foreach_sub.Scalar",
    "_foreach_sub.List", "_foreach_neg", "_foreach_abs", "_foreach_maximum.Scalar",
):
    if _op_exists("aten::" + _name):
        register_aten_op("aten::" + _name)(_foreach.functional_dispatcher("aten::" + _name))

# ---------------------------------------------------------------------------
# elementwise families
# ---------------------------------------------------------------------------
_BINARY_WITH_ALPHA = ("add", "sub")
_BINARY = (
    "mul", "div", "eq", "ne", "lt", "le", "gt", "ge", "bitwise_and", "bitwise_or",
    "bitwise_xor", "remainder",
)
_BINARY_DEFAULT = ("maximum", "minimum", "logical_and", "logical_or", "logical_xor", "floor_divide")


def _bin(name, inplace=False):
    def impl(self, other, *, alpha=1, out=None):
        return F._binary(name, self, other, alpha, inplace=inplace, out=out)

    return impl


def _bin_mode(inplace=False):
    def impl(self, other, *, rounding_mode=None, out=None):
        return F._binary("div", self, other, inplace=inplace, mode=rounding_mode, out=out)

    return impl


def _bin_scalar_alpha(name, inplace=False):
    def impl(self, other, alpha=1):
        return F._binary(name, self, other, alpha, inplace=inplace)

    return impl


for _n in _BINARY_WITH_ALPHA:
    _reg(f"aten::{_n}.Tensor", _bin(_n))
    _reg(f"aten::{_n}.Scalar", _bin_scalar_alpha(_n))
    _reg(f"aten::{_n}_.Tensor", _bin(_n, True))
    _reg(f"aten::{_n}_.Scalar", _bin_scalar_alpha(_n, True))
    _reg(f"aten::{_n}.out", _bin(_n))
for _n in _BINARY:
    for _ov, _ip in (("Tensor", False), ("Scalar", False)):
        if _op_exists(f"aten::{_n}.{_ov}"):
            _reg(f"aten::{_n}.{_ov}", _bin(_n, _ip))
        if _op_exists(f"aten::{_n}_.{_ov}"):
            _reg(f"aten::{_n}_.{_ov}", _bin(_n, True))
    if _op_exists(f"aten::{_n}.out"):
        _reg(f"aten::{_n}.out", _bin(_n))
_reg("aten::div.Tensor_mode", _bin_mode())
_reg("aten::div_.Tensor_mode", _bin_mode(True))
_reg("aten::div.Scalar_mode", _bin_mode())
for _n in _BINARY_DEFAULT:
    _reg(f"aten::{_n}", _bin(_n))
    if _op_exists(f"aten::{_n}_"):
        _reg(f"aten::{_n}_", _bin(_n, True))
    if _op_exists(f"aten::{_n}.Scalar"):
        _reg(f"aten::{_n}.Scalar", _bin(_n))

_UNARY_FLOAT = (
    "exp", "log", "sqrt", "rsqrt", "reciprocal", "sin", "cos", "tan", "tanh", "sigmoid",
    "erf", "log1p", "expm1", "log2", "exp2", "log10", "atan", "asin", "acos", "sinh",
    "cosh", "asinh", "acosh", "atanh", "silu",
)
_UNARY_SAME = ("neg", "abs", "relu", "floor", "ceil", "round", "trunc", "sign", "bitwise_not")
_UNARY_BOOL = ("logical_not", "isnan")


def _un(name, inplace=False, float_result=True):
    def impl(self, *, out=None):
        return F._unary(name, self, inplace=inplace, out=out, float_result=float_result)

    return impl


for _n in _UNARY_FLOAT + _UNARY_SAME + _UNARY_BOOL:
    fr = _n in _UNARY_FLOAT
    if _op_exists(f"aten::{_n}"):
        _reg(f"aten::{_n}", _un(_n, False, fr))
    if _op_exists(f"aten::{_n}_"):
        _reg(f"aten::{_n}_", _un(_n, True, fr))
    if _op_exists(f"aten::{_n}.out"):
        _reg(f"aten::{_n}.out", _un(_n, False, fr))


__all__ = ["_aten_ops_registry", "register_aten_op", "EAGER_CALL_COUNTERS", "unsupported", "out_variant"]
