"""AutocastPrivateUse1 policies for eager mojo tensors.

Same policy table as the reference (torch_mojo_backend/mojo_device/
mojo_device_autocast.py:537-567): matmul and attention run in the active
lower precision; layer_norm and NLL run in f32; everything else falls
through.  Casts are ordinary ``_to_copy`` ops on the device, except for
``linear``, whose casts and GEMMs run inside one fused autograd Function
(mojo_device_autograd._FusedLinear) with the same numerics.
"""

from __future__ import annotations

import functools
from collections.abc import Mapping

import torch

_registered = False
_fallback_library = None
_aten_library = None

_AUTOCAST_KEYSET = torch._C.DispatchKeySet(torch._C.DispatchKey.AutocastPrivateUse1)


def _cast_mojo_floating(value, dtype):
    if isinstance(value, torch.Tensor):
        if (
            value.device.type == "mojo"
            and value.is_floating_point()
            and value.dtype != torch.float64
            and value.dtype != dtype
        ):
            return value.to(dtype=dtype)
        return value
    if isinstance(value, tuple):
        return tuple(_cast_mojo_floating(v, dtype) for v in value)
    if isinstance(value, list):
        return [_cast_mojo_floating(v, dtype) for v in value]
    if isinstance(value, Mapping):
        return {k: _cast_mojo_floating(v, dtype) for k, v in value.items()}
    return value


def _policy_wrapper(op, dtype_getter, mark_low=False):
    """Run op with its floating mojo arguments cast to dtype_getter().  With
    mark_low (the f32 layer norms) the op also learns the autocast dtype, so
    its kernel can write the lower-precision copy of its output that the
    next autocast matmul casts to."""
    @functools.wraps(op)
    def wrapper(*args, **kwargs):
        with torch._C._ExcludeDispatchKeyGuard(_AUTOCAST_KEYSET):
            dtype = dtype_getter()
            cargs, ckwargs = _cast_mojo_floating(args, dtype), _cast_mojo_floating(kwargs, dtype)
            if mark_low:
                from ..eager_kernels import aten_fast

                with aten_fast.autocast_low_scope(torch.get_autocast_dtype("mojo")):
                    return op(*cargs, **ckwargs)
            return op(*cargs, **ckwargs)

    return wrapper


def register_autocast_ops() -> None:
    global _registered, _fallback_library, _aten_library
    if _registered:
        return
    _fallback_library = torch.library.Library("_", "IMPL", "AutocastPrivateUse1")
    _fallback_library.fallback(torch.library.fallthrough_kernel)
    _aten_library = torch.library.Library("aten", "IMPL", "AutocastPrivateUse1")
    lower = (
        torch.ops.aten.addmm.default,
        torch.ops.aten.bmm.default,
        torch.ops.aten.matmul.default,
        torch.ops.aten.mm.default,
        torch.ops.aten.scaled_dot_product_attention.default,
        torch.ops.aten._scaled_dot_product_flash_attention.default,
    )
    fp32 = (
        torch.ops.aten.layer_norm.default,
        torch.ops.aten.native_layer_norm.default,
        torch.ops.aten.nll_loss.default,
        torch.ops.aten.nll_loss_forward.default,
    )
    for op in lower:
        _aten_library.impl(
            op._schema.name, _policy_wrapper(op, lambda: torch.get_autocast_dtype("mojo"))
        )
    for op in fp32:
        norm = "layer_norm" in op._schema.name
        _aten_library.impl(op._schema.name, _policy_wrapper(op, lambda: torch.float32, mark_low=norm))
    _aten_library.impl("linear", _linear_autocast)
    _registered = True


def _linear_autocast(input, weight, bias=None):
    from .mojo_device_autograd import fused_linear, fused_linear_inputs

    with torch._C._ExcludeDispatchKeyGuard(_AUTOCAST_KEYSET):
        dt = torch.get_autocast_dtype("mojo")
        if fused_linear_inputs(input, weight, bias, dt):
            return fused_linear(input, weight, bias, dt)
        args = _cast_mojo_floating((input, weight, bias), dt)
        return torch.ops.aten.linear.default(*args)
