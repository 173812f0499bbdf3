"""Shared plumbing for the op registrations (aten_ops/support.py:28-120 in
the reference): binding a host wrapper to an op name, turning ``NOT_HANDLED``
into an actionable ``NotImplementedError``."""

from __future__ import annotations

from collections.abc import Callable

import torch

from ...eager_kernels.aten_fast import NOT_HANDLED, copy_into, _require


def _describe_args(args, kwargs) -> str:
    descs = []
    for a in list(args) + list(kwargs.values()):
        if isinstance(a, torch.Tensor):
            descs.append(f"{tuple(a.shape)}:{a.dtype}:{a.device}")
        elif isinstance(a, (list, tuple)) and a and isinstance(a[0], torch.Tensor):
            descs.append(f"[{len(a)} tensors]")
    return ", ".join(descs) or "none"


def unsupported(op_name: str, args=(), kwargs=None) -> NotImplementedError:
    return NotImplementedError(
        f"{op_name} is not supported by the mojo eager device for these inputs "
        f"(tensor args: {_describe_args(args, kwargs or {})})."
    )


def eager_impl(fast_fn: Callable, op_name: str) -> Callable:
    """Bind an op to a fast_aten_* function; raise on NOT_HANDLED."""

    def dispatcher(*args, **kwargs):
        result = fast_fn(*args, **kwargs)
        if result is NOT_HANDLED:
            raise unsupported(op_name, args, kwargs)
        return result

    dispatcher.__name__ = getattr(fast_fn, "__name__", op_name)
    return dispatcher


def out_variant(op_name: str, fast_fn: Callable) -> Callable:
    """An ``out=`` overload from a functional implementation."""

    def dispatcher(*args, out, **kwargs):
        result = fast_fn(*args, **kwargs)
        if result is NOT_HANDLED:
            raise unsupported(op_name, args, kwargs)
        copy_into(_require(out), result)
        return out

    return dispatcher
