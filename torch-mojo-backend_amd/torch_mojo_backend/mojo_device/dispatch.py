"""The dispatch bracket between `__torch_dispatch__` and the op table.

Counterpart of the reference's deferred_compile.dispatch
(torch_mojo_backend/mojo_device/deferred_compile.py:77-90).  There is no
kernel-call queue here: every kernel is compiled ahead of time, so a launch
is never blocked on a build and ops are issued directly, in order, on the
device stream.  `drain()` therefore reduces to a stream synchronisation at
host reads (`synchronize`, `.item()`, `.cpu()`).
"""

from __future__ import annotations

import torch

from .. import eager_kernels as _ek
from ..eager_kernels import aten_fast as _aten_fast

# OpOverload -> python implementation (filled by register_mojo_devices)
DIRECT: dict = {}

_DISABLE = torch._C._DisableTorchDispatch


_MUTABLE: dict = {}  # OpOverload -> whether its schema writes an argument


def _is_mutable(func) -> bool:
    mutable = _MUTABLE.get(func)
    if mutable is None:
        mutable = _MUTABLE[func] = func._schema.is_mutable
    return mutable


_ADAMW = (torch.ops.aten._fused_adamw_.default, torch.ops.aten._fused_adamw_.tensor_lr)


def dispatch(func, args, kwargs):
    if _ek._lazy:  # work waiting for a first use: autocast layer-norm outputs, a clip scale
        if func in _ADAMW and len(args) > 1:
            # the fused step applies a pending scale on its gradients itself
            # (fast_aten__fused_adamw_); everything else it touches goes first
            _ek.materialize_touched(args[:1] + args[2:], kwargs, True)
        else:
            _ek.materialize_touched(args, kwargs, _is_mutable(func))
    if _aten_fast._param_low_by_holder and _is_mutable(func):  # parameter copies exist (autocast training)
        _aten_fast.drop_param_copies_written_by(func, args, kwargs)
    impl = DIRECT.get(func)
    if impl is not None:
        return impl(*args, **kwargs)
    # Not a direct entry: let the dispatcher pick the PrivateUse1 kernel (one
    # of ours, or a composite decomposition whose pieces come back here).
    with _DISABLE():
        return func(*args, **kwargs)
