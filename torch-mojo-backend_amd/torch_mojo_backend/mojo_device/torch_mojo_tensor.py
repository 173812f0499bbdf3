"""`TorchMojoTensor`: the eager `mojo` device tensor.

Mirrors the reference wrapper (torch_mojo_backend/mojo_device/
torch_mojo_tensor.py:309-612): a storage-less ``PrivateUse1`` wrapper
subclass whose payload is plain Python attributes

    _holder   object owning the device allocation (shared by views)
    _ptr      device address of element 0 of this view
    _shape, _strides (elements), _offset (elements from allocation start)
    _dtype (torch dtype), _itemsize, _numel, _device (int index),
    _is_contiguous, _torch_device

The difference is the holder: the reference holds a Mojo ``TensorHolder``;
here it is a byte tensor from PyTorch-ROCm's caching allocator on the GPU
the ``mojo:N`` device maps to (``cuda:N``).  PyTorch is used only for that
allocation and for host<->device byte copies; every computation on these
tensors goes through the gfx950 kernel library.

The wrapper's ``__torch_dispatch__`` looks the op up in the registered
kernel table and calls it directly (skipping a second trip through the
dispatcher); ops without a direct entry are redispatched to the
``PrivateUse1`` key, where composite decompositions land back in the table.
"""

from __future__ import annotations

import math

import torch

_MAX_RANK = 8

# torch dtype -> kernel-library dtype code (include/mi355x_kernels.h)
DTYPE_CODE = {
    torch.float32: 0,
    torch.bfloat16: 1,
    torch.float16: 2,
    torch.float64: 3,
    torch.int64: 4,
    torch.int32: 5,
    torch.int16: 6,
    torch.int8: 7,
    torch.uint8: 8,
    torch.bool: 9,
}

# Where holders live.  "cuda" on a GPU box; host-only tests swap in "cpu"
# together with a host stand-in for the kernel library.
_STORAGE_KIND = "cuda"
_STORAGE_DEVICES: dict[int, torch.device] = {}
_TORCH_DEVICES: dict[int, torch.device] = {}


def set_storage_kind_for_tests(kind: str) -> str:
    """Switch holder allocation between "cuda" and "cpu"; returns the old kind."""
    global _STORAGE_KIND
    previous = _STORAGE_KIND
    _STORAGE_KIND = kind
    _STORAGE_DEVICES.clear()
    return previous


def storage_kind() -> str:
    return _STORAGE_KIND


def storage_device(index: int) -> torch.device:
    dev = _STORAGE_DEVICES.get(index)
    if dev is None:
        if _STORAGE_KIND == "cuda":
            if not torch.cuda.is_available():
                raise RuntimeError(
                    "the mojo device needs a ROCm GPU (torch.cuda.is_available() is False)"
                )
            dev = torch.device("cuda", index)
        else:
            dev = torch.device("cpu")
        _STORAGE_DEVICES[index] = dev
    return dev


def torch_device_of(index: int) -> torch.device:
    dev = _TORCH_DEVICES.get(index)
    if dev is None:
        dev = torch.device("mojo", index)
        _TORCH_DEVICES[index] = dev
    return dev


def row_major_strides(shape) -> tuple[int, ...]:
    strides = []
    acc = 1
    for s in reversed(shape):
        strides.append(acc)
        acc *= max(s, 1)
    return tuple(reversed(strides))


def compute_contiguous(shape, strides) -> bool:
    expected = 1
    for s, st in zip(reversed(shape), reversed(strides)):
        if s == 1:
            continue
        if st != expected:
            return False
        expected *= s
    return True


def _alloc_bytes(nbytes: int, device: int) -> torch.Tensor:
    """Allocate `nbytes` (at least 1) on the storage device.

    On OOM the caching allocator's free blocks are released and the
    allocation retried once, the counterpart of the reference's
    drain-and-retry (torch_mojo_tensor.py:213-244)."""
    dev = storage_device(device)
    size = max(int(nbytes), 1)
    try:
        return torch.empty(size, dtype=torch.uint8, device=dev)
    except torch.OutOfMemoryError:
        if dev.type == "cuda":
            torch.cuda.synchronize(dev)
            torch.cuda.empty_cache()
        return torch.empty(size, dtype=torch.uint8, device=dev)


_DISPATCH = None


def _dispatch_module():
    """The dispatch module, imported on first use (it imports this one)."""
    global _DISPATCH
    if _DISPATCH is None:
        from . import dispatch

        _DISPATCH = dispatch
    return _DISPATCH


class TorchMojoTensor(torch.Tensor):
    """Eager mojo tensor (storage-less PrivateUse1 wrapper subclass)."""

    @classmethod
    def __torch_dispatch__(cls, func, types, args=(), kwargs=None):
        if len(types) != 1 or types[0] is not cls:
            for t in types:
                if not issubclass(cls, t):
                    return NotImplemented
        return (_DISPATCH or _dispatch_module()).dispatch(func, args, kwargs or {})

    __torch_function__ = torch._C._disabled_torch_function_impl

    @classmethod
    def _make(cls, holder, ptr, shape, strides, offset, dtype, device, contiguous=None):
        shape = tuple(shape)
        strides = tuple(strides)
        tdev = torch_device_of(device)
        res = torch.Tensor._make_wrapper_subclass(
            cls,
            shape,
            strides=strides,
            storage_offset=offset,
            dtype=dtype,
            layout=torch.strided,
            device=tdev,
            requires_grad=False,
        )
        res._holder = holder
        res._ptr = ptr
        res._shape = shape
        res._strides = strides
        res._offset = offset
        res._dtype = dtype
        res._itemsize = dtype.itemsize
        res._numel = math.prod(shape)
        res._device = device
        res._torch_device = tdev
        res._is_contiguous = (
            compute_contiguous(shape, strides) if contiguous is None else contiguous
        )
        return res

    @classmethod
    def _alloc(cls, shape, dtype, device: int) -> "TorchMojoTensor":
        """A new contiguous uninitialised tensor (one allocation)."""
        shape = tuple(int(s) for s in shape)
        if len(shape) > _MAX_RANK:
            raise NotImplementedError(
                f"mojo tensors support at most rank {_MAX_RANK}, got {len(shape)}"
            )
        numel = math.prod(shape)
        holder = _alloc_bytes(numel * dtype.itemsize, device)
        return cls._make(
            holder, holder.data_ptr(), shape, row_major_strides(shape), 0, dtype, device, True
        )

    @classmethod
    def _alloc_strided(cls, shape, strides, dtype, device: int) -> "TorchMojoTensor":
        """A new uninitialised tensor with explicit (non-negative) strides."""
        shape = tuple(int(s) for s in shape)
        strides = tuple(int(s) for s in strides)
        if any(st < 0 for st in strides):
            raise NotImplementedError("negative strides are not supported on mojo tensors")
        extent = 1 + sum((s - 1) * st for s, st in zip(shape, strides)) if all(shape) else 0
        holder = _alloc_bytes(extent * dtype.itemsize, device)
        return cls._make(holder, holder.data_ptr(), shape, strides, 0, dtype, device)

    @classmethod
    def _view_of(cls, base, shape, strides, offset, contiguous=None) -> "TorchMojoTensor":
        """Zero-copy view sharing `base`'s holder; `offset` is absolute."""
        ptr = base._ptr + (offset - base._offset) * base._itemsize
        return cls._make(
            base._holder, ptr, shape, strides, offset, base._dtype, base._device, contiguous
        )

    @classmethod
    def _from_cpu(cls, cpu_tensor: torch.Tensor, device: int) -> "TorchMojoTensor":
        """H2D: allocate and copy a CPU tensor's bytes."""
        t = cpu_tensor.detach()
        if t.device.type != "cpu":
            raise RuntimeError(
                f"TorchMojoTensor._from_cpu requires a CPU source tensor, got {t.device}"
            )
        if not t.is_contiguous():
            t = t.contiguous()
        out = cls._alloc(tuple(t.shape), t.dtype, device)
        nbytes = t.numel() * t.element_size()
        if nbytes:
            src = t.reshape(-1).view(torch.uint8)
            out._holder[:nbytes].copy_(src)
        return out

    def _to_cpu_tensor(self) -> torch.Tensor:
        """D2H copy into a new CPU tensor (waits for pending device work).
        A bounds error that a kernel flagged since the last host read is
        raised here."""
        from ..eager_kernels import aten_fast, flush_pending, materialize

        materialize(self)  # an output whose kernel waits for its first use
        flush_pending()  # launches held back for fusion write what is read here
        aten_fast.raise_pending_device_errors()
        src = self._contig()
        out = torch.empty(src._shape, dtype=src._dtype)
        nbytes = src._numel * src._itemsize
        if nbytes:
            begin = src._offset * src._itemsize
            out.reshape(-1).view(torch.uint8).copy_(src._holder[begin : begin + nbytes])
        return out

    def _contig(self) -> "TorchMojoTensor":
        """self if contiguous, else a materialised contiguous copy."""
        if self._is_contiguous:
            return self
        from ..eager_kernels import aten_fast

        return aten_fast.materialize_contiguous(self)

    def __reduce_ex__(self, protocol):
        """Pickle as a plain CPU tensor (torch_mojo_tensor.py:572-583), so
        checkpoints load without this backend."""
        if hasattr(self, "_holder"):
            return self._to_cpu_tensor().__reduce_ex__(protocol)
        return super().__reduce_ex__(protocol)

    def __repr__(self, *, tensor_contents=None):
        if hasattr(self, "_holder"):
            return f"TorchMojoTensor({self._to_cpu_tensor()!r}, device='{self.device}')"
        return super().__repr__()

    @property
    def device(self):
        if hasattr(self, "_torch_device"):
            return self._torch_device
        return super().device
