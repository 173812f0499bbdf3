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


_VIEW: dict = {}  # OpOverload -> whether it reads no data (a view, or a fresh tensor shaped like an input)
# fresh tensors shaped like their input, whose values do not depend on it
_LIKE = ("aten::empty_like", "aten::zeros_like", "aten::ones_like", "aten::full_like", "aten::new_empty",
         "aten::new_empty_strided", "aten::new_zeros", "aten::new_ones", "aten::new_full")


def _is_view(func) -> bool:
    view = _VIEW.get(func)
    if view is None:
        sch = func._schema
        view = _VIEW[func] = sch.name in _LIKE or (
            not sch.is_mutable and bool(sch.returns) and all(r.alias_info is not None for r in sch.returns))
    return view


def dispatch(func, args, kwargs):
    # work waiting for a first use (autocast layer-norm outputs, a clip scale,
    # ...) runs before the op, unless the op reads no data: a view shares the
    # storage, so its own first use still finds the work pending, and an
    # `ones_like` (the engine's gradient of a loss) needs only the shape
    if _ek._lazy and not _is_view(func):
        _ek.materialize_touched(args, kwargs, _is_mutable(func), func)
    if _aten_fast._param_low_by_holder and _is_mutable(func):  # parameter copies exist (autocast training)
        _aten_fast.drop_param_copies_written_by(func, args, kwargs)
    impl = DIRECT.get(func)
    if impl is not None:
        return impl(*args, **kwargs)
    # Not a direct entry: let the dispatcher pick the PrivateUse1 kernel (one
    # of ours, or a composite decomposition whose pieces come back here).
    with _DISABLE():
        return func(*args, **kwargs)
