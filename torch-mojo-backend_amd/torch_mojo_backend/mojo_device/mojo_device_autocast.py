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

import torch

_EXCLUDE_AUTOCAST = torch._C.DispatchKeySet(torch._C.DispatchKey.AutocastPrivateUse1)

# Policy table (the drop-in contract): "low" runs the op in the active
# autocast dtype, "f32" in float32; unlisted ops fall through unchanged.
_POLICY = {
    "low": ("addmm", "bmm", "matmul", "mm", "scaled_dot_product_attention",
            "_scaled_dot_product_flash_attention"),
    "f32": ("layer_norm", "native_layer_norm", "nll_loss", "nll_loss_forward"),
}
# f32 ops whose kernels also write the autocast-dtype copy of their output
_WRITES_LOW_COPY = frozenset({"layer_norm", "native_layer_norm"})


def _autocast_dtype():
    return torch.get_autocast_dtype("mojo")


_RETYPED = (torch.float32, torch.float16, torch.bfloat16)


def _retype(x, dtype):
    """A floating mojo tensor below float64 that is not already `dtype`
    becomes a `dtype` copy, also inside a list or tuple argument (a tensor
    list); everything else passes unchanged.  (Aten arguments nest no
    deeper, so no general tree walk is needed.)"""
    if isinstance(x, torch.Tensor):
        if x.dtype != dtype and x.dtype in _RETYPED and x.device.type == "mojo":
            return x.to(dtype)
        return x
    if isinstance(x, (list, tuple)) and any(isinstance(e, torch.Tensor) for e in x):
        return type(x)(_retype(e, dtype) for e in x)
    return x


def _retype_call(args, kwargs, dtype):
    args = tuple(_retype(a, dtype) for a in args)
    if kwargs:
        kwargs = {k: _retype(v, dtype) for k, v in kwargs.items()}
    return args, kwargs


def _under_policy(op, target, low_copy=False):
    """op's AutocastPrivateUse1 kernel: retype the floating mojo arguments to
    target() and call op below the autocast key.  low_copy (the f32 layer
    norms) also tells the kernel the autocast dtype, so it writes the
    lower-precision copy of its output that the next autocast matmul would
    otherwise cast."""
    @functools.wraps(op)
    def kernel(*args, **kwargs):
        with torch._C._ExcludeDispatchKeyGuard(_EXCLUDE_AUTOCAST):
            args, kwargs = _retype_call(args, kwargs, target())
            if not low_copy:
                return op(*args, **kwargs)
            from ..eager_kernels import aten_fast

            with aten_fast.autocast_low_scope(_autocast_dtype()):
                return op(*args, **kwargs)

    return kernel


class _AutocastRegistry:
    """Owns the torch.library handles (they unregister when collected)."""

    def __init__(self) -> None:
        self.libs: list = []

    def install(self) -> None:
        fall = torch.library.Library("_", "IMPL", "AutocastPrivateUse1")
        fall.fallback(torch.library.fallthrough_kernel)
        aten = torch.library.Library("aten", "IMPL", "AutocastPrivateUse1")
        targets = {"low": _autocast_dtype, "f32": lambda: torch.float32}
        for kind, names in _POLICY.items():
            for name in names:
                op = getattr(torch.ops.aten, name).default
                aten.impl(name, _under_policy(op, targets[kind], low_copy=name in _WRITES_LOW_COPY))
        aten.impl("linear", _linear_autocast)
        self.libs = [fall, aten]


_registry: _AutocastRegistry | None = None


def register_autocast_ops() -> None:
    global _registry
    if _registry is None:
        reg = _AutocastRegistry()
        reg.install()
        _registry = reg


def _linear_autocast(input, weight, bias=None):
    from .mojo_device_autograd import fused_linear, fused_linear_inputs

    with torch._C._ExcludeDispatchKeyGuard(_EXCLUDE_AUTOCAST):
        dt = _autocast_dtype()
        if fused_linear_inputs(input, weight, bias, dt):
            return fused_linear(input, weight, bias, dt)
        input, weight, bias = (_retype(t, dt) for t in (input, weight, bias))
        return torch.ops.aten.linear.default(input, weight, bias)
