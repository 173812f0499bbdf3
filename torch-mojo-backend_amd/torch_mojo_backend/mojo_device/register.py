"""`register_mojo_devices()`: enable the `mojo` device and its ATen kernels.

Follows the reference's registration sequence (torch_mojo_backend/
mojo_device/register.py:217-275): swap-on-conversion so tied weights stay one
allocation, PrivateUse1 renamed to "mojo" with the backend module, the
accelerator synchronize hook, foreach/fused optimizer opt-in, the ATen op
table, the SDPA autograd kernel and the autocast policies.  The torch.compile
patches of the reference are out of scope (eager device only).
"""

from __future__ import annotations

from functools import wraps

import torch

from . import dispatch
from .mojo_device_aten_ops import _aten_ops_registry

_registered = False
_libraries: list = []


def _install_torch_accelerator_synchronize(module) -> None:
    original = torch.accelerator.synchronize
    if getattr(original, "_torch_mojo_backend", False):
        return

    @wraps(original)
    def synchronize(device=None):
        if torch.accelerator.current_accelerator() != torch.device("mojo"):
            return original(device)
        return module.synchronize(device)

    synchronize._torch_mojo_backend = True
    torch.accelerator.synchronize = synchronize


def _resolve_overload(qualname: str):
    ns, rest = qualname.split("::")
    name, _, overload = rest.partition(".")
    packet = getattr(getattr(torch.ops, ns), name)
    return getattr(packet, overload or "default")


def register_mojo_devices() -> None:
    """Enable the mojo device globally and register its ATen ops."""
    global _registered
    if _registered:
        return
    from torch.utils.backend_registration import _setup_privateuseone_for_python_backend

    from . import torch_mojo_device_module
    from ..eager_kernels import lib

    # Fail loudly now if the kernel library is absent: there is no fallback.
    if torch_mojo_device_module._tensor_mod.storage_kind() == "cuda":
        lib()

    torch.__future__.set_swap_module_params_on_conversion(True)
    _setup_privateuseone_for_python_backend("mojo", backend_module=torch_mojo_device_module)
    _install_torch_accelerator_synchronize(torch_mojo_device_module)

    import torch.optim.optimizer as optimizer_module
    import torch.utils._foreach_utils as foreach_utils

    from .torch_mojo_tensor import TorchMojoTensor

    for supported in (optimizer_module._foreach_supported_types, foreach_utils._foreach_supported_types):
        if TorchMojoTensor not in supported:
            supported.append(TorchMojoTensor)

    lib_obj = torch.library.Library("aten", "IMPL", "PrivateUse1")
    _libraries.append(lib_obj)
    for op_name, func in _aten_ops_registry:
        overload = _resolve_overload(op_name)
        # Composite-implicit ops decompose above the backend; registering a
        # backend kernel for them would bypass autograd.  Only SDPA is kept,
        # paired with its own AutogradPrivateUse1 kernel.
        if op_name != "aten::scaled_dot_product_attention" and torch._C._dispatch_has_kernel_for_dispatch_key(
            overload.name(), "CompositeImplicitAutograd"
        ):
            continue
        lib_obj.impl(overload, func)
        dispatch.DIRECT[overload] = func

    from .mojo_device_autograd import register_autograd_ops
    from .mojo_device_autocast import register_autocast_ops

    register_autograd_ops()
    register_autocast_ops()
    _registered = True
