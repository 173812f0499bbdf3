"""ATen-semantics host wrappers: ``fast_aten_<op>`` over the gfx950 library.

Counterpart of the reference's L2 layer (torch_mojo_backend/eager_kernels/
aten_fast.py): each function validates metadata, allocates outputs with the
device allocator, and issues one or a few kernel calls through the C ABI
(`include/mi355x_kernels.h`).  A function returns ``NOT_HANDLED`` (the
reference's sentinel, aten_fast.py:159) for inputs it cannot serve; the
registry turns that into a ``NotImplementedError`` naming the op.

Ownership follows the reference's "Into" ABI (docs/kernel_call_queue.md:
164-180): Python allocates every output and workspace before the call, the
kernels never allocate and never synchronise.  All launches go to the null
stream of the device, which is also PyTorch's default stream, so the caching
allocator's stream-ordered reuse keeps freed buffers safe.
"""

from __future__ import annotations

import ctypes
import math
import numbers
import os

import torch

from . import AdamWTensor, Deferred, check, defer, flush_pending, lazy, lazy_scale, lib, take_pending
from . import lazy_live as _lazy_pending
from . import pending_scale as _pending_scale
from ..mojo_device.torch_mojo_tensor import (
    DTYPE_CODE,
    TorchMojoTensor,
    _alloc_bytes,
    compute_contiguous,
    row_major_strides,
)

NOT_HANDLED = object()

MT = TorchMojoTensor
_STREAM = None  # the device's null stream (PyTorch's default stream)
_FLOAT_DTYPES = (torch.float32, torch.bfloat16, torch.float16)
_MFMA_DTYPES = (torch.bfloat16, torch.float16)

# opcode constants (include/mi355x_kernels.h)
OP = dict(
    add=0, sub=1, mul=2, div=3, maximum=4, minimum=5, pow=6, eq=7, ne=8, lt=9, le=10,
    gt=11, ge=12, logical_and=13, logical_or=14, logical_xor=15, bitwise_and=16,
    bitwise_or=17, bitwise_xor=18, remainder=19, floor_divide=20, div_trunc=21,
    div_floor=22, where=40, addcmul=41, addcdiv=42, lerp=43, identity=60, neg=61,
    abs=62, exp=63, log=64, sqrt=65, rsqrt=66, reciprocal=67, sin=68, cos=69, tanh=70,
    sigmoid=71, erf=72, relu=73, silu=74, log1p=75, expm1=76, floor=77, ceil=78,
    round=79, trunc=80, sign=81, pow_scalar=82, clamp=83, logical_not=84,
    bitwise_not=85, isnan=86, isinf=87, isfinite=88, tan=89, atan=90, asin=91,
    acos=92, sinh=93, cosh=94, asinh=95, acosh=96, atanh=97, log2=98, exp2=99,
    log10=100, square=101, clamp_min=102, clamp_max=103, rsub=104,
)
RED = dict(sum=0, mean=1, max=2, min=3, norm2=4, sumsq=5, amax=6, prod=7, any=8, all=9, norm1=10)


# ---------------------------------------------------------------------------
# small helpers
# ---------------------------------------------------------------------------
def _i64(values) -> ctypes.Array:
    values = tuple(int(v) for v in values)
    return (ctypes.c_int64 * max(len(values), 1))(*values)


def _t(x):
    """x as a mojo tensor with a payload, else None."""
    if isinstance(x, MT) and hasattr(x, "_holder"):
        return x
    return None


def _is_mojo(x) -> bool:
    return isinstance(x, MT)


def _require(x, what="tensor"):
    t = _t(x)
    if t is None:
        raise RuntimeError(f"expected a mojo tensor for {what}, got {type(x).__name__}")
    return t


def _alloc(shape, dtype, device: int) -> MT:
    return MT._alloc(shape, dtype, device)


def _workspace(nbytes: int, device: int):
    """Scratch buffer; returns (holder, pointer).  Stream-ordered reuse of
    the caching allocator makes dropping it after the launch safe."""
    if nbytes <= 0:
        return None, None
    holder = _alloc_bytes(nbytes, device)
    return holder, holder.data_ptr()


def _code(dtype) -> int:
    code = DTYPE_CODE.get(dtype)
    if code is None:
        raise NotImplementedError(f"dtype {dtype} is not supported on the mojo device")
    return code


def _contig(t: MT) -> MT:
    return t if t._is_contiguous else materialize_contiguous(t)


def _norm_dim(dim: int, rank: int) -> int:
    r = max(rank, 1)
    if dim < -r or dim >= r:
        raise IndexError(f"Dimension out of range (expected to be in range of [{-r}, {r - 1}], but got {dim})")
    return dim % r if rank > 0 else 0


def _scalar_value(x):
    if isinstance(x, torch.Tensor):
        return x.item()
    return x


def _scalar_dtype(x):
    if isinstance(x, bool):
        return torch.bool
    if isinstance(x, numbers.Integral):
        return torch.int64
    if isinstance(x, complex):
        raise NotImplementedError("complex scalars are not supported on the mojo device")
    return torch.float32


def _broadcast_strides(t: MT, shape) -> tuple[int, ...]:
    """t's strides expanded to `shape` (0 along broadcast dims)."""
    nd = len(shape)
    pad = nd - len(t._shape)
    out = []
    for i in range(nd):
        j = i - pad
        if j < 0 or t._shape[j] == 1 and shape[i] != 1:
            out.append(0)
        elif t._shape[j] == 1:
            out.append(0)
        else:
            out.append(t._strides[j])
    return tuple(out)


def _device_of(*xs) -> int:
    for x in xs:
        t = _t(x)
        if t is not None:
            return t._device
    raise RuntimeError("no mojo tensor among the operands")


# ---------------------------------------------------------------------------
# copies
# ---------------------------------------------------------------------------
def copy_into(dst: MT, src: MT) -> MT:
    """dst[...] = src (broadcast, dtype conversion) on the device."""
    shape = dst._shape
    if dst._numel == 0:
        return dst
    st = _broadcast_strides(src, shape)
    check(
        "mi355x_copy",
        lib().mi355x_copy(
            dst._ptr, _code(dst._dtype), _i64(dst._strides), src._ptr, _code(src._dtype),
            _i64(st), _i64(shape), len(shape), _STREAM,
        ),
    )
    return dst


def materialize_contiguous(t: MT, dtype=None) -> MT:
    out = _alloc(t._shape, dtype or t._dtype, t._device)
    return copy_into(out, t)


def _dense_permutation(t: MT):
    """Strides that keep t's memory order for a new dense tensor (the
    preserve_format rule), or None to use row-major."""
    if t._is_contiguous:
        return None
    nd = len(t._shape)
    order = sorted(range(nd), key=lambda i: (-t._strides[i], i))
    shape_p = [t._shape[i] for i in order]
    strides_p = [t._strides[i] for i in order]
    if not compute_contiguous(shape_p, strides_p):
        return None
    dense = row_major_strides(shape_p)
    strides = [0] * nd
    for k, i in enumerate(order):
        strides[i] = dense[k]
    return tuple(strides)


def _empty_like_layout(t: MT, dtype=None) -> MT:
    strides = _dense_permutation(t)
    if strides is None:
        return _alloc(t._shape, dtype or t._dtype, t._device)
    return MT._alloc_strided(t._shape, strides, dtype or t._dtype, t._device)


def upload(cpu: torch.Tensor, device: int) -> MT:
    return MT._from_cpu(cpu, device)


def fast_aten_copy_(self, src, non_blocking=False):
    dst = _t(self)
    s = _t(src)
    if dst is not None and s is not None:
        if dst._device != s._device:
            s = upload(s._to_cpu_tensor(), dst._device)
        copy_into(dst, s)
        return self
    if dst is not None and isinstance(src, torch.Tensor):
        # host -> device
        cpu = src.detach()
        if dst._is_contiguous and cpu.dtype == dst._dtype and tuple(cpu.shape) == dst._shape:
            cpu = cpu.contiguous()
            nbytes = cpu.numel() * cpu.element_size()
            if nbytes:
                begin = dst._offset * dst._itemsize
                flush_pending()
                dst._holder[begin : begin + nbytes].copy_(cpu.reshape(-1).view(torch.uint8))
            return self
        tmp = upload(cpu.contiguous(), dst._device)
        copy_into(dst, tmp)
        return self
    if s is not None and isinstance(self, torch.Tensor) and self.device.type == "cpu":
        # device -> host
        host = s._to_cpu_tensor()
        self.copy_(host)
        return self
    return NOT_HANDLED


def fast_aten__copy_from(self, dst, non_blocking=False):
    fast_aten_copy_(dst, self, non_blocking)
    return dst


def fast_aten__to_copy(
    self, *, dtype=None, layout=None, device=None, pin_memory=None, non_blocking=False,
    memory_format=None,
):
    t = _t(self)
    target = torch.device(device) if device is not None else None
    dtype = dtype or self.dtype
    if t is None:
        if isinstance(self, torch.Tensor) and self.device.type == "cpu" and target is not None \
                and target.type == "mojo":
            # host -> device: convert on the host (exact, as torch does), then upload
            src = self.detach()
            if src.dtype != dtype:
                src = src.to(dtype)
            return upload(src, _dev_index(target))
        return NOT_HANDLED
    if target is not None and target.type == "cpu":
        src = t if dtype == t._dtype else fast_aten__to_copy(t, dtype=dtype)
        return src._to_cpu_tensor()
    dev = t._device
    if target is not None and target.type == "mojo" and target.index is not None:
        if target.index != dev:
            host = t._to_cpu_tensor()
            return upload(host.to(dtype), target.index)
    if dtype != t._dtype and memory_format in (None, torch.preserve_format, torch.contiguous_format):
        low = _take_low_copy(t, dtype)
        if low is not None:
            return low
        if dtype in (torch.bfloat16, torch.float16) and t._dtype == torch.float32:
            # a held-back residual-gradient sum cast to the autocast dtype
            # (the autograd engine's cast to a bf16 input's dtype)
            low = _add_then_cast(t, dtype)
            if low is not None:
                return low
    if memory_format in (None, torch.preserve_format):
        out = _empty_like_layout(t, dtype)
    else:
        out = _alloc(t._shape, dtype, dev)
    return copy_into(out, t)


def fast_aten_clone(self, *, memory_format=None):
    t = _require(self)
    if memory_format in (None, torch.preserve_format):
        out = _empty_like_layout(t)
    else:
        out = _alloc(t._shape, t._dtype, t._device)
    return copy_into(out, t)


def fast_aten__local_scalar_dense(self):
    t = _require(self)
    return t._to_cpu_tensor().item()


# ---------------------------------------------------------------------------
# factories
# ---------------------------------------------------------------------------
def _dev_index(device) -> int:
    if device is None:
        from ..mojo_device import torch_mojo_device_module as mod

        return mod.current_device()
    d = torch.device(device)
    if d.type != "mojo":
        raise RuntimeError(f"expected a mojo device, got {d}")
    if d.index is None:
        from ..mojo_device import torch_mojo_device_module as mod

        return mod.current_device()
    return d.index


def fill_(t: MT, value) -> MT:
    if t._numel:
        check(
            "mi355x_fill",
            lib().mi355x_fill(
                t._ptr, _code(t._dtype), _i64(t._strides), _i64(t._shape), len(t._shape),
                float(value), _STREAM,
            ),
        )
    return t


def fast_aten_empty_memory_format(
    size, *, dtype=None, layout=None, device=None, pin_memory=None, memory_format=None
):
    return _alloc(tuple(size), dtype or torch.get_default_dtype(), _dev_index(device))


def fast_aten_empty_strided(
    size, stride, *, dtype=None, layout=None, device=None, pin_memory=None
):
    size, stride = tuple(size), tuple(stride)
    dtype = dtype or torch.get_default_dtype()
    if stride == row_major_strides(size):
        return _alloc(size, dtype, _dev_index(device))
    return MT._alloc_strided(size, stride, dtype, _dev_index(device))


def fast_aten_empty_like(
    self, *, dtype=None, layout=None, device=None, pin_memory=None, memory_format=None
):
    t = _require(self)
    dev = t._device if device is None else _dev_index(device)
    if memory_format in (None, torch.preserve_format) and dev == t._device:
        return _empty_like_layout(t, dtype)
    return _alloc(t._shape, dtype or t._dtype, dev)


def fast_aten_full(size, fill_value, *, dtype=None, layout=None, device=None, pin_memory=None):
    if dtype is None:
        dtype = _scalar_dtype(fill_value) if not isinstance(fill_value, float) else torch.get_default_dtype()
    return fill_(_alloc(tuple(size), dtype, _dev_index(device)), fill_value)


def fast_aten_zeros(size, *, dtype=None, layout=None, device=None, pin_memory=None):
    return fill_(_alloc(tuple(size), dtype or torch.get_default_dtype(), _dev_index(device)), 0)


def fast_aten_ones(size, *, dtype=None, layout=None, device=None, pin_memory=None):
    return fill_(_alloc(tuple(size), dtype or torch.get_default_dtype(), _dev_index(device)), 1)


def _like(self, value, dtype, device, memory_format):
    out = fast_aten_empty_like(self, dtype=dtype, device=device, memory_format=memory_format)
    return fill_(out, value)


def fast_aten_zeros_like(self, *, dtype=None, layout=None, device=None, pin_memory=None, memory_format=None):
    return _like(self, 0, dtype, device, memory_format)


def fast_aten_ones_like(self, *, dtype=None, layout=None, device=None, pin_memory=None, memory_format=None):
    return _like(self, 1, dtype, device, memory_format)


def fast_aten_full_like(self, fill_value, *, dtype=None, layout=None, device=None, pin_memory=None, memory_format=None):
    return _like(self, fill_value, dtype, device, memory_format)


def _new(self, size, dtype, device):
    t = _require(self)
    return _alloc(tuple(size), dtype or t._dtype, t._device if device is None else _dev_index(device))


def fast_aten_new_empty(self, size, *, dtype=None, layout=None, device=None, pin_memory=None):
    return _new(self, size, dtype, device)


def fast_aten_new_empty_strided(self, size, stride, *, dtype=None, layout=None, device=None, pin_memory=None):
    t = _require(self)
    return fast_aten_empty_strided(size, stride, dtype=dtype or t._dtype,
                                   device=device if device is not None else t.device)


def fast_aten_new_zeros(self, size, *, dtype=None, layout=None, device=None, pin_memory=None):
    return fill_(_new(self, size, dtype, device), 0)


def fast_aten_new_ones(self, size, *, dtype=None, layout=None, device=None, pin_memory=None):
    return fill_(_new(self, size, dtype, device), 1)


def fast_aten_new_full(self, size, fill_value, *, dtype=None, layout=None, device=None, pin_memory=None):
    return fill_(_new(self, size, dtype, device), fill_value)


def fast_aten_scalar_tensor(s, *, dtype=None, layout=None, device=None, pin_memory=None):
    return fill_(_alloc((), dtype or torch.get_default_dtype(), _dev_index(device)), s)


def fast_aten_arange(end, *, dtype=None, layout=None, device=None, pin_memory=None):
    return fast_aten_arange_start_step(0, end, 1, dtype=dtype, device=device)


def fast_aten_arange_start(start, end, *, dtype=None, layout=None, device=None, pin_memory=None):
    return fast_aten_arange_start_step(start, end, 1, dtype=dtype, device=device)


def fast_aten_arange_start_step(start, end, step=1, *, dtype=None, layout=None, device=None, pin_memory=None):
    start, end, step = (_scalar_value(v) for v in (start, end, step))
    if dtype is None:
        if all(isinstance(v, numbers.Integral) for v in (start, end, step)):
            dtype = torch.int64
        else:
            dtype = torch.get_default_dtype()
    if step == 0:
        raise RuntimeError("step must be nonzero")
    n = max(0, math.ceil((end - start) / step))
    out = _alloc((n,), dtype, _dev_index(device))
    if n:
        check("mi355x_arange", lib().mi355x_arange(out._ptr, _code(dtype), n, float(start), float(step), _STREAM))
    return out


def fast_aten_fill__scalar(self, value):
    fill_(_require(self), _scalar_value(value))
    return self


def fast_aten_fill__tensor(self, value):
    t = _require(self)
    v = _t(value)
    if v is not None:
        copy_into(t, v)
    else:
        fill_(t, _scalar_value(value))
    return self


def fast_aten_zero_(self):
    fill_(_require(self), 0)
    return self


# ---------------------------------------------------------------------------
# views (metadata only)
# ---------------------------------------------------------------------------
def _infer_size(shape, numel):
    shape = list(shape)
    neg = [i for i, s in enumerate(shape) if s == -1]
    if len(neg) > 1:
        raise RuntimeError("only one dimension can be inferred")
    if neg:
        rest = math.prod(s for s in shape if s != -1)
        if rest == 0 or numel % rest:
            raise RuntimeError(f"shape '{list(shape)}' is invalid for input of size {numel}")
        shape[neg[0]] = numel // rest
    if math.prod(shape) != numel:
        raise RuntimeError(f"shape '{list(shape)}' is invalid for input of size {numel}")
    return tuple(shape)


def _view_strides(old_shape, old_strides, new_shape):
    """ATen's computeStride: strides of a view, or None if impossible."""
    numel = math.prod(old_shape)
    if numel == 0:
        return row_major_strides(new_shape) if old_shape != new_shape else tuple(old_strides)
    new_strides = [0] * len(new_shape)
    view_d = len(new_shape) - 1
    chunk_base_stride = old_strides[-1] if old_strides else 1
    tensor_numel = 1
    view_numel = 1
    for tensor_d in range(len(old_shape) - 1, -1, -1):
        tensor_numel *= old_shape[tensor_d]
        if tensor_d == 0 or (
            old_shape[tensor_d - 1] != 1
            and old_strides[tensor_d - 1] != tensor_numel * chunk_base_stride
        ):
            while view_d >= 0 and (view_numel < tensor_numel or new_shape[view_d] == 1):
                new_strides[view_d] = view_numel * chunk_base_stride
                view_numel *= new_shape[view_d]
                view_d -= 1
            if view_numel != tensor_numel:
                return None
            if tensor_d > 0:
                chunk_base_stride = old_strides[tensor_d - 1]
                tensor_numel = 1
                view_numel = 1
    if view_d != -1:
        return None
    return tuple(new_strides)


def fast_aten_view(self, size):
    t = _require(self)
    shape = _infer_size(size, t._numel)
    if t._is_contiguous:
        return MT._view_of(t, shape, row_major_strides(shape), t._offset, True)
    strides = _view_strides(t._shape, t._strides, shape)
    if strides is None:
        raise RuntimeError(
            "view size is not compatible with input tensor's size and stride (at least one"
            " dimension spans across two contiguous subspaces). Use .reshape(...) instead."
        )
    return MT._view_of(t, shape, strides, t._offset)


def fast_aten__unsafe_view(self, size):
    return fast_aten_view(self, size)


def fast_aten__reshape_alias(self, size, stride):
    t = _require(self)
    return MT._view_of(t, tuple(size), tuple(stride), t._offset)


def fast_aten_as_strided(self, size, stride, storage_offset=None):
    t = _require(self)
    off = t._offset if storage_offset is None else int(storage_offset)
    return MT._view_of(t, tuple(size), tuple(stride), off)


def fast_aten_alias(self):
    t = _require(self)
    return MT._view_of(t, t._shape, t._strides, t._offset, t._is_contiguous)


fast_aten_detach = fast_aten_alias


def fast_aten_t(self):
    t = _require(self)
    if len(t._shape) < 2:
        return fast_aten_alias(t)
    return fast_aten_transpose(t, 0, 1)


def fast_aten_transpose(self, dim0, dim1):
    t = _require(self)
    nd = len(t._shape)
    if nd == 0:
        return fast_aten_alias(t)
    d0, d1 = _norm_dim(dim0, nd), _norm_dim(dim1, nd)
    shape, strides = list(t._shape), list(t._strides)
    shape[d0], shape[d1] = shape[d1], shape[d0]
    strides[d0], strides[d1] = strides[d1], strides[d0]
    return MT._view_of(t, shape, strides, t._offset)


def fast_aten_permute(self, dims):
    t = _require(self)
    nd = len(t._shape)
    dims = [_norm_dim(d, nd) for d in dims]
    return MT._view_of(t, [t._shape[d] for d in dims], [t._strides[d] for d in dims], t._offset)


def fast_aten_expand(self, size, *, implicit=False):
    t = _require(self)
    size = list(size)
    nd = len(size)
    pad = nd - len(t._shape)
    if pad < 0:
        raise RuntimeError("expand: the number of sizes must be >= the tensor rank")
    shape, strides = [], []
    for i in range(nd):
        j = i - pad
        if j < 0:
            if size[i] < 0:
                raise RuntimeError("expand: -1 is not allowed in a leading, non-existing dimension")
            shape.append(size[i])
            strides.append(0)
        else:
            s = size[i]
            if s == -1:
                s = t._shape[j]
            if t._shape[j] == s:
                shape.append(s)
                strides.append(t._strides[j])
            elif t._shape[j] == 1:
                shape.append(s)
                strides.append(0)
            else:
                raise RuntimeError(
                    f"The expanded size of the tensor ({s}) must match the existing size"
                    f" ({t._shape[j]}) at non-singleton dimension {i}"
                )
    return MT._view_of(t, shape, strides, t._offset)


def fast_aten_slice(self, dim=0, start=None, end=None, step=1):
    t = _require(self)
    nd = len(t._shape)
    d = _norm_dim(dim, nd)
    n = t._shape[d]
    start = 0 if start is None else start
    end = n if end is None else end
    if start < 0:
        start += n
    if end < 0:
        end += n
    start = min(max(start, 0), n)
    end = min(max(end, start), n)
    if step <= 0:
        raise RuntimeError("slice step must be positive")
    length = (end - start + step - 1) // step
    shape, strides = list(t._shape), list(t._strides)
    shape[d] = length
    strides[d] = t._strides[d] * step
    return MT._view_of(t, shape, strides, t._offset + start * t._strides[d])


def fast_aten_select(self, dim, index):
    t = _require(self)
    nd = len(t._shape)
    d = _norm_dim(dim, nd)
    n = t._shape[d]
    if index < -n or index >= n:
        raise IndexError(f"select(): index {index} out of range for tensor of size {t._shape} at dimension {d}")
    index %= n
    shape = t._shape[:d] + t._shape[d + 1 :]
    strides = t._strides[:d] + t._strides[d + 1 :]
    return MT._view_of(t, shape, strides, t._offset + index * t._strides[d])


def fast_aten_split_with_sizes(self, split_sizes, dim=0):
    t = _require(self)
    d = _norm_dim(dim, len(t._shape))
    if sum(split_sizes) != t._shape[d]:
        raise RuntimeError("split_with_sizes expects split_sizes to sum exactly to the dim size")
    outs, start = [], 0
    for s in split_sizes:
        outs.append(fast_aten_slice(t, d, start, start + s))
        start += s
    return outs


def fast_aten_split(self, split_size, dim=0):
    t = _require(self)
    d = _norm_dim(dim, len(t._shape))
    n = t._shape[d]
    if split_size <= 0:
        return [fast_aten_alias(t)]
    sizes = [split_size] * (n // split_size)
    if n % split_size or n == 0:
        sizes.append(n % split_size)
    return fast_aten_split_with_sizes(t, sizes, d)


def fast_aten_unbind(self, dim=0):
    t = _require(self)
    d = _norm_dim(dim, len(t._shape))
    return [fast_aten_select(t, d, i) for i in range(t._shape[d])]


def fast_aten_squeeze(self):
    t = _require(self)
    keep = [i for i, s in enumerate(t._shape) if s != 1]
    return MT._view_of(t, [t._shape[i] for i in keep], [t._strides[i] for i in keep], t._offset)


def fast_aten_squeeze_dims(self, dims):
    t = _require(self)
    nd = len(t._shape)
    if isinstance(dims, int):
        dims = [dims]
    ds = {_norm_dim(d, nd) for d in dims} if nd else set()
    keep = [i for i in range(nd) if not (i in ds and t._shape[i] == 1)]
    return MT._view_of(t, [t._shape[i] for i in keep], [t._strides[i] for i in keep], t._offset)


def fast_aten_unsqueeze(self, dim):
    t = _require(self)
    nd = len(t._shape)
    d = _norm_dim(dim, nd + 1)
    shape, strides = list(t._shape), list(t._strides)
    st = shape[d] * strides[d] if d < nd else 1
    shape.insert(d, 1)
    strides.insert(d, st)
    return MT._view_of(t, shape, strides, t._offset)


# ---------------------------------------------------------------------------
# elementwise
# ---------------------------------------------------------------------------
def _map_call(opcode, out: MT, inputs, s0=0.0, s1=0.0):
    """inputs: list of (MT or None-for-scalar-s1, dtype)."""
    shape = out._shape
    if out._numel == 0:
        return out
    nin = len(inputs)
    ptrs = (ctypes.c_void_p * 3)()
    dts = (ctypes.c_int * 3)()
    strides = list(out._strides)
    for j, (x, dt) in enumerate(inputs):
        if x is None:
            ptrs[j] = None
            dts[j] = _code(dt)
            strides.extend([0] * len(shape))
        else:
            ptrs[j] = x._ptr
            dts[j] = _code(x._dtype)
            strides.extend(_broadcast_strides(x, shape))
    check(
        "mi355x_map",
        lib().mi355x_map(
            opcode, out._ptr, _code(out._dtype), nin, ptrs, dts, _i64(strides), _i64(shape),
            len(shape), float(s0), float(s1), _STREAM,
        ),
    )
    return out


def _operand(x):
    """(mojo tensor | None, scalar value | None, dtype, shape)."""
    t = _t(x)
    if t is not None:
        return t, None, t._dtype, t._shape
    if isinstance(x, torch.Tensor):
        if x.dim() != 0:
            raise RuntimeError(
                f"expected all tensors to be on the same device, got a {x.device} tensor of"
                f" shape {tuple(x.shape)} with a mojo tensor"
            )
        return None, x.item(), x.dtype, ()
    return None, x, _scalar_dtype(x), ()


_COMPARE = {"eq", "ne", "lt", "le", "gt", "ge", "logical_and", "logical_or", "logical_xor"}
_FLOAT_RESULT = {"div", "pow"}


def _binary(name, a, b, alpha=1, *, out=None, inplace=False, mode=None):
    ta, sa, da, sha = _operand(a)
    tb, sb, db, shb = _operand(b)
    if ta is None and tb is None:
        return NOT_HANDLED
    if name == "add" and out is None and ta is not None and tb is not None and _lazy_pending():
        r = _add_lazy(ta, tb, alpha, inplace)
        if r is not None:
            return r
    opcode = OP[name]
    if name == "div" and mode == "trunc":
        opcode = OP["div_trunc"]
    elif name == "div" and mode == "floor":
        opcode = OP["div_floor"]
    # result dtype by torch's promotion rules (scalars are "wrapped numbers";
    # two tensors of rank >= 1 promote by dtype alone)
    if ta is not None and tb is not None and sha and shb:
        rtype = torch.promote_types(da, db)
    else:
        rtype = torch.result_type(a, b)
    if name in _COMPARE:
        out_dtype = torch.bool
    elif name in _FLOAT_RESULT and mode is None and not rtype.is_floating_point:
        out_dtype = torch.get_default_dtype()
    else:
        out_dtype = rtype
    shape = tuple(sha) if tuple(sha) == tuple(shb) else tuple(torch.broadcast_shapes(sha, shb))
    if inplace:
        target = ta
        if tuple(target._shape) != shape:
            raise RuntimeError(
                f"output with shape {list(target._shape)} doesn't match the broadcast shape {list(shape)}"
            )
        if not torch.can_cast(out_dtype, target._dtype) and name not in _COMPARE:
            raise RuntimeError(f"result type {out_dtype} can't be cast to the desired output type {target._dtype}")
        res = target
    elif out is not None:
        res = _require(out)
    else:
        dev = (ta if ta is not None else tb)._device
        res = _alloc(shape, out_dtype, dev)
    s0 = float(_scalar_value(alpha)) if name in ("add", "sub") else 0.0
    if ta is None:
        # scalar first operand: only for commutative ops or via rsub forms
        if name in ("add", "mul", "maximum", "minimum", "eq", "ne", "logical_and", "logical_or",
                    "logical_xor", "bitwise_and", "bitwise_or", "bitwise_xor"):
            return _map_call(opcode, res, [(tb, db), (None, da)], s0, sa) if name != "add" else \
                _map_call(OP["rsub"], res, [(tb, db)], sa, -s0)
        swapped = {"lt": "gt", "le": "ge", "gt": "lt", "ge": "le"}
        if name in swapped:
            return _map_call(OP[swapped[name]], res, [(tb, db), (None, da)], 0.0, sa)
        if name == "sub":
            return _map_call(OP["rsub"], res, [(tb, db)], sa, s0)
        # general: materialise the scalar
        fill_val = fill_(_alloc((), da, tb._device), sa)
        return _map_call(opcode, res, [(fill_val, da), (tb, db)], s0, 0.0)
    if tb is None:
        return _map_call(opcode, res, [(ta, da), (None, db)], s0, sb)
    if name == "add" and not inplace and out is None and s0 == 1.0 and _residual_add(res, ta, tb):
        # x + f(...) of a pre-norm block: held back so that the LayerNorm
        # reading the sum can compute it in the same pass (any other
        # consumer issues it first).  The record keeps the storages, not
        # the tensors: a held reference to the sum would stop autograd from
        # taking it as a leaf's .grad without a copy.
        r_out, r_a, r_b = _Ref(res), _Ref(ta), _Ref(tb)
        defer(Deferred(r_out, (r_a, r_b), lambda: _map_call(opcode, r_out, [(r_a, da), (r_b, db)], s0, 0.0)))
        return res
    return _map_call(opcode, res, [(ta, da), (tb, db)], s0, 0.0)


class _Ref:
    """What a held-back launch needs of a mojo tensor (pointer, layout,
    dtype, and the storage holder that keeps the memory alive), without a
    reference to the tensor object itself."""

    __slots__ = ("_holder", "_ptr", "_shape", "_strides", "_offset", "_dtype", "_numel", "_is_contiguous",
                 "_device", "_itemsize")

    def __init__(self, t: MT):
        self._holder, self._ptr, self._shape, self._strides = t._holder, t._ptr, t._shape, t._strides
        self._offset, self._dtype, self._numel = t._offset, t._dtype, t._numel
        self._is_contiguous, self._device, self._itemsize = t._is_contiguous, t._device, t._itemsize


_RESIDUAL_MIN_NUMEL = 1 << 16


def _residual_add(res: MT, a: MT, b: MT) -> bool:
    """Whether res = a + b has the shape a fused residual-add LayerNorm
    takes: f32 a and res, f32/bf16/f16 b, one shape, contiguous rows of a
    multiple of 4 (at most 2048) elements, 16-byte aligned."""
    if res._dtype != torch.float32 or a._dtype != torch.float32 or b._dtype not in _FLOAT_DTYPES:
        return False
    if tuple(a._shape) != tuple(res._shape) or tuple(b._shape) != tuple(res._shape):
        return False
    if not (a._is_contiguous and b._is_contiguous and res._is_contiguous) or res._numel < _RESIDUAL_MIN_NUMEL:
        return False
    cols = res._shape[-1]
    return cols % 4 == 0 and cols <= 2048 and a._ptr % 16 == 0 and b._ptr % 16 == 0 and res._ptr % 16 == 0


def _unary(name, a, *, out=None, inplace=False, s0=0.0, s1=0.0, float_result=True):
    t = _require(a)
    if inplace:
        res = t
    elif out is not None:
        res = _require(out)
    else:
        dt = t._dtype
        if float_result and not dt.is_floating_point:
            dt = torch.get_default_dtype()
        if name in ("isnan", "isinf", "isfinite", "logical_not"):
            dt = torch.bool
        res = _alloc(t._shape, dt, t._device)
    return _map_call(OP[name], res, [(t, t._dtype)], s0, s1)


def fast_aten_where(condition, self, other):
    tc, _, _, shc = _operand(condition)
    ta, sa, da, sha = _operand(self)
    tb, sb, db, shb = _operand(other)
    shape = tuple(torch.broadcast_shapes(shc, sha, shb))
    out_dtype = torch.result_type(self, other)
    dev = _device_of(condition, self, other)
    res = _alloc(shape, out_dtype, dev)
    if tc is None:
        tc = fill_(_alloc((), torch.bool, dev), bool(_scalar_value(condition)))
    if ta is None:
        ta = fill_(_alloc((), out_dtype, dev), sa)
    if tb is None:
        tb = fill_(_alloc((), out_dtype, dev), sb)
    return _map_call(OP["where"], res, [(tc, tc._dtype), (ta, ta._dtype), (tb, tb._dtype)])


def fast_aten_masked_fill(self, mask, value, *, inplace=False):
    t = _require(self)
    m = _require(mask)
    v = _t(value)
    res = t if inplace else _alloc(t._shape, t._dtype, t._device)
    if v is not None:
        return _map_call(OP["where"], res, [(m, m._dtype), (v, v._dtype), (t, t._dtype)])
    val = _scalar_value(value)
    return _map_call(OP["where"], res, [(m, m._dtype), (None, _scalar_dtype(val)), (t, t._dtype)], 0.0, val)


def _ternary(name, self, t1, t2, value, inplace=False):
    a = _require(self)
    b, c = _require(t1), _require(t2)
    shape = tuple(torch.broadcast_shapes(a._shape, b._shape, c._shape))
    res = a if inplace else _alloc(shape, torch.result_type(torch.result_type(self, t1), t2), a._device)
    return _map_call(OP[name], res, [(a, a._dtype), (b, b._dtype), (c, c._dtype)], float(_scalar_value(value)))


def fast_aten_lerp(self, end, weight, *, inplace=False):
    a, b = _require(self), _require(end)
    w = _t(weight)
    if w is not None:
        # a + w*(b-a) with a tensor weight: (b-a)*w + a
        diff = _binary("sub", b, a)
        prod = _binary("mul", diff, w)
        res = a if inplace else _alloc(a._shape, a._dtype, a._device)
        return _map_call(OP["add"], res, [(a, a._dtype), (prod, prod._dtype)], 1.0)
    shape = tuple(torch.broadcast_shapes(a._shape, b._shape))
    res = a if inplace else _alloc(shape, a._dtype, a._device)
    return _map_call(OP["lerp"], res, [(a, a._dtype), (b, b._dtype)], float(_scalar_value(weight)))


def fast_aten_clamp(self, min=None, max=None, *, inplace=False, out=None):
    t = _require(self)
    tmin, tmax = _t(min), _t(max)
    if tmin is not None or tmax is not None:
        r = t
        if tmin is not None:
            r = _binary("maximum", r, tmin)
        if tmax is not None:
            r = _binary("minimum", r, tmax)
        if inplace:
            return copy_into(t, r)
        return r
    lo = -math.inf if min is None else _scalar_value(min)
    hi = math.inf if max is None else _scalar_value(max)
    dt = t._dtype
    if not dt.is_floating_point and (isinstance(lo, float) and math.isfinite(lo) or isinstance(hi, float) and math.isfinite(hi)):
        dt = torch.get_default_dtype()
    if not dt.is_floating_point:
        lo = -(2**62) if min is None else lo
        hi = 2**62 if max is None else hi
    res = t if inplace else (_require(out) if out is not None else _alloc(t._shape, dt, t._device))
    return _map_call(OP["clamp"], res, [(t, t._dtype)], lo, hi)


def fast_aten_pow_tensor_scalar(self, exponent, *, inplace=False):
    t = _require(self)
    e = _scalar_value(exponent)
    dt = t._dtype
    if not dt.is_floating_point and (isinstance(e, float) or e < 0):
        dt = torch.get_default_dtype()
    res = t if inplace else _alloc(t._shape, dt, t._device)
    if not dt.is_floating_point:
        if e == 2:
            return _map_call(OP["square"], res, [(t, t._dtype)])
        if e == 1:
            return _map_call(OP["identity"], res, [(t, t._dtype)])
        if e == 0:
            return fill_(res, 1)
    return _map_call(OP["pow_scalar"], res, [(t, t._dtype)], float(e))


def fast_aten_pow_scalar(self, exponent):
    base = _scalar_value(self)
    e = _require(exponent)
    dt = e._dtype if e._dtype.is_floating_point else torch.get_default_dtype()
    res = _alloc(e._shape, dt, e._device)
    b = fill_(_alloc((), dt, e._device), base)
    return _map_call(OP["pow"], res, [(b, dt), (e, e._dtype)])


def fast_aten_rsub(self, other, alpha=1):
    """other - alpha*self"""
    t = _require(self)
    to = _t(other)
    if to is not None:
        return _binary("sub", to, t, alpha)
    o = _scalar_value(other)
    dt = torch.result_type(self, other)
    res = _alloc(t._shape, dt, t._device)
    return _map_call(OP["rsub"], res, [(t, t._dtype)], float(o), float(_scalar_value(alpha)))


# ---------------------------------------------------------------------------
# reductions
# ---------------------------------------------------------------------------
def _reduce_plan(t: MT, dims):
    """(tensor, outer, r, inner, s_o, s_r, s_i, kept_shape) for reducing
    `dims` of t; materialises a permuted copy when the reduced dims cannot be
    expressed as one strided axis."""
    nd = len(t._shape)
    if dims is None or (isinstance(dims, (list, tuple)) and len(dims) == 0):
        dims = list(range(nd))
    elif isinstance(dims, int):
        dims = [dims]
    red = sorted({_norm_dim(d, nd) for d in dims}) if nd else []
    kept = [i for i in range(nd) if i not in red]
    kept_shape = [t._shape[i] for i in kept]
    src = _contig(t)
    shape = src._shape
    r = math.prod(shape[i] for i in red) if red else 1
    if red and red == list(range(red[0], red[-1] + 1)):
        outer = math.prod(shape[: red[0]])
        inner = math.prod(shape[red[-1] + 1 :])
        return src, outer, r, inner, r * inner, inner, 1, kept_shape
    if not red:
        n = math.prod(shape)
        return src, n, 1, 1, 1, 1, 1, kept_shape
    perm = kept + red
    permuted = materialize_contiguous(fast_aten_permute(src, perm))
    outer = math.prod(kept_shape)
    return permuted, outer, r, 1, r, 1, 1, kept_shape


def _reduce(op, self, dims, keepdim, out_dtype, *, out=None):
    t = _require(self)
    nd = len(t._shape)
    src, outer, r, inner, so, sr, si, kept_shape = _reduce_plan(t, dims)
    if keepdim:
        if dims is None or (isinstance(dims, (list, tuple)) and len(dims) == 0):
            dset = set(range(nd))
        else:
            dset = {_norm_dim(d, nd) for d in ([dims] if isinstance(dims, int) else dims)}
        out_shape = tuple(1 if i in dset else t._shape[i] for i in range(nd))
    else:
        out_shape = tuple(kept_shape)
    res = _require(out) if out is not None else _alloc(out_shape, out_dtype, t._device)
    dst = res if res._is_contiguous else _alloc(out_shape, out_dtype, t._device)
    if r == 0 and op in (RED["max"], RED["min"], RED["amax"]) and outer * inner:
        raise IndexError("max(): Expected reduction dim to be specified for input.numel() == 0")
    ws = lib().mi355x_reduce_workspace_bytes(outer, r, inner)
    hold, wptr = _workspace(ws, t._device)
    check(
        "mi355x_reduce",
        lib().mi355x_reduce(op, dst._ptr, _code(dst._dtype), src._ptr, _code(src._dtype),
                            outer, r, inner, so, sr, si, wptr, ws, _STREAM),
    )
    if dst is not res:
        copy_into(res, dst)
    return res


def _sum_dtype(t, dtype):
    if dtype is not None:
        return dtype
    if t.dtype.is_floating_point:
        return t.dtype
    return torch.int64


def fast_aten_sum(self, dim=None, keepdim=False, *, dtype=None):
    return _reduce(RED["sum"], self, dim, keepdim, _sum_dtype(self, dtype))


def fast_aten_sum_default(self, *, dtype=None):
    return _reduce(RED["sum"], self, None, False, _sum_dtype(self, dtype))


def fast_aten_mean(self, dim=None, keepdim=False, *, dtype=None):
    dt = dtype or self.dtype
    if not dt.is_floating_point:
        raise RuntimeError(
            f"mean(): could not infer output dtype. Input dtype must be either a floating point"
            f" or complex dtype. Got: {self.dtype}"
        )
    return _reduce(RED["mean"], self, dim, keepdim, dt)


def fast_aten_mean_default(self, *, dtype=None):
    return fast_aten_mean(self, None, False, dtype=dtype)


def fast_aten_amax(self, dim=(), keepdim=False):
    return _reduce(RED["max"], self, dim, keepdim, self.dtype)


def fast_aten_amin(self, dim=(), keepdim=False):
    return _reduce(RED["min"], self, dim, keepdim, self.dtype)


def fast_aten_max_default(self):
    return _reduce(RED["max"], self, None, False, self.dtype)


def fast_aten_min_default(self):
    return _reduce(RED["min"], self, None, False, self.dtype)


def fast_aten_any(self, dim=None, keepdim=False):
    return _reduce(RED["any"], self, dim, keepdim, torch.bool)


def fast_aten_all(self, dim=None, keepdim=False):
    return _reduce(RED["all"], self, dim, keepdim, torch.bool)


def fast_aten_linalg_vector_norm(self, ord=2, dim=None, keepdim=False, *, dtype=None):
    t = _require(self)
    out_dtype = dtype or t._dtype
    if ord == 2:
        return _reduce(RED["norm2"], t, dim, keepdim, out_dtype)
    if ord == 1:
        return _reduce(RED["norm1"], t, dim, keepdim, out_dtype)
    if ord == math.inf:
        return _reduce(RED["amax"], t, dim, keepdim, out_dtype)
    if ord == 0:
        nz = _binary("ne", t, 0)
        return _reduce(RED["sum"], nz, dim, keepdim, out_dtype)
    # general p-norm: (sum |x|^p)^(1/p)
    a = _unary("abs", t)
    p = fast_aten_pow_tensor_scalar(a, float(ord))
    s = _reduce(RED["sum"], p, dim, keepdim, out_dtype)
    return fast_aten_pow_tensor_scalar(s, 1.0 / float(ord))


def _argreduce(is_min, self, dim, keepdim, with_values):
    t = _require(self)
    nd = len(t._shape)
    if dim is None:
        flat = _contig(t)
        src, outer, r, inner, so, sr, si = flat, 1, flat._numel, 1, flat._numel, 1, 1
        out_shape = (1,) * nd if keepdim else ()
    else:
        d = _norm_dim(dim, nd)
        src, outer, r, inner, so, sr, si, kept = _reduce_plan(t, [d])
        out_shape = tuple(1 if i == d else t._shape[i] for i in range(nd)) if keepdim else tuple(kept)
    if r == 0:
        raise IndexError("argmax(): Expected reduction dim to be specified for input.numel() == 0.")
    idx = _alloc(out_shape, torch.int64, t._device)
    vals = _alloc(out_shape, t._dtype, t._device) if with_values else None
    check(
        "mi355x_argreduce",
        lib().mi355x_argreduce(int(is_min), idx._ptr, vals._ptr if vals is not None else None,
                               src._ptr, _code(src._dtype), outer, r, inner, so, sr, si, _STREAM),
    )
    return (vals, idx) if with_values else idx


def fast_aten_argmax(self, dim=None, keepdim=False):
    return _argreduce(False, self, dim, keepdim, False)


def fast_aten_argmin(self, dim=None, keepdim=False):
    return _argreduce(True, self, dim, keepdim, False)


def fast_aten_max_dim(self, dim, keepdim=False):
    return _argreduce(False, self, dim, keepdim, True)


def fast_aten_min_dim(self, dim, keepdim=False):
    return _argreduce(True, self, dim, keepdim, True)


# ---------------------------------------------------------------------------
# cat / index
# ---------------------------------------------------------------------------
_FOREACH_DTYPES = (torch.float32, torch.bfloat16, torch.float16)


_CAT_READY = "_mojo_cat_ready"


def _mark_cat_ready(t: MT) -> None:
    """Mark a fresh buffer whose slices are handed out as separate results
    (the attention gradients): one cat of its adjacent slices may return a
    view of it instead of a copy."""
    setattr(t._holder, _CAT_READY, True)


def _cat_in_place(ts, d, shape):
    """A view of the buffer when `ts` are adjacent slices of one cat-ready
    buffer laid out exactly as their concatenation along d (same strides,
    equal to the result's contiguous strides; offsets one piece after the
    other), else None.  The mark is consumed."""
    first = ts[0]
    holder = first._holder
    if not getattr(holder, _CAT_READY, False):
        return None
    strides = [1] * len(shape)
    for j in range(len(shape) - 2, -1, -1):
        strides[j] = strides[j + 1] * shape[j + 1]
    off = first._offset
    for x in ts:
        if x._holder is not holder or x._dtype != first._dtype or tuple(x._strides) != tuple(strides):
            return None
        if x._offset != off:
            return None
        off += x._shape[d] * strides[d]
    setattr(holder, _CAT_READY, False)
    return MT._view_of(first, tuple(shape), tuple(strides), first._offset, True)


def _stack_in_place(ts):
    """A view of the buffer when `ts` are equal-shape contiguous slices of
    one cat-ready buffer lying one after the other (the per-tensor results
    of `_foreach_norm`), i.e. already laid out as their stack along dim 0,
    else None.  The mark is consumed."""
    first = ts[0]
    holder = first._holder
    if not getattr(holder, _CAT_READY, False) or not first._is_contiguous:
        return None
    shape, step, off = first._shape, first._numel, first._offset
    for x in ts:
        if (x._holder is not holder or x._offset != off or x._shape != shape or x._dtype != first._dtype
                or not x._is_contiguous):
            return None
        off += step
    setattr(holder, _CAT_READY, False)
    out_shape = (len(ts),) + tuple(shape)
    return MT._view_of(first, out_shape, row_major_strides(out_shape), first._offset, True)


def fast_aten_cat(tensors, dim=0):
    ts = [_require(x) for x in tensors]
    ts_nonempty = [x for x in ts if not (len(x._shape) == 1 and x._shape[0] == 0)]
    if not ts_nonempty:
        return _alloc((0,), ts[0]._dtype if ts else torch.float32, ts[0]._device if ts else 0)
    ref = ts_nonempty[0]
    nd = len(ref._shape)
    d = _norm_dim(dim, nd)
    dtype = ts_nonempty[0]._dtype
    for x in ts_nonempty[1:]:
        dtype = torch.promote_types(dtype, x._dtype)
    # torch.cat's own checks (a __torch_dispatch__ subclass gets no meta
    # shape check first): same rank, same size in every dim but d
    for i, x in enumerate(ts):
        if len(x._shape) == 1 and x._shape[0] == 0:
            continue  # torch.cat skips legacy empty 1-D pieces
        if len(x._shape) != nd:
            raise RuntimeError(
                f"Tensors must have same number of dimensions: got {nd} and {len(x._shape)}"
            )
        for j in range(nd):
            if j != d and x._shape[j] != ref._shape[j]:
                raise RuntimeError(
                    f"Sizes of tensors must match except in dimension {d}. Expected size"
                    f" {ref._shape[j]} but got size {x._shape[j]} for tensor number {i}"
                    " in the list."
                )
    shape = list(ref._shape)
    shape[d] = sum(x._shape[d] for x in ts_nonempty)
    if len(ts_nonempty) > 1 and all(x._dtype == dtype for x in ts_nonempty):
        view = _cat_in_place(ts_nonempty, d, shape)
        if view is not None:
            return view
    out = _alloc(shape, dtype, ref._device)
    if (len(ts_nonempty) >= 8 and math.prod(shape[:d]) == 1 and dtype in _FOREACH_DTYPES
            and all(x._dtype == dtype and x._is_contiguous for x in ts_nonempty)):
        # Many pieces that are whole contiguous chunks of the output (e.g.
        # clip_grad_norm_'s stack of per-parameter norms): one multi-tensor
        # launch instead of one copy per piece.  chunk_i = -0.0 + 1 * x_i
        # equals x_i for every finite or infinite x_i and for signed zeros; a
        # NaN stays NaN (a signalling NaN comes out quieted).
        fill_(out, -0.0)
        ptrs, off = [], 0
        for x in ts_nonempty:
            ptrs.append(out._ptr + off * out._itemsize)
            off += x._numel
        check(
            "mi355x_foreach_apply",
            lib().mi355x_foreach_apply(
                0, _ptr_array(ptrs), _ptr_array([x._ptr for x in ts_nonempty]), None, None,
                _i64([x._numel for x in ts_nonempty]), len(ts_nonempty), _code(dtype), 1.0, None, _STREAM,
            ),
        )
        return out
    start = 0
    for x in ts_nonempty:
        n = x._shape[d]
        if n:
            copy_into(fast_aten_slice(out, d, start, start + n), x)
        start += n
    return out


def fast_aten_stack(tensors, dim=0):
    ts = [_require(x) for x in tensors]
    d = _norm_dim(dim, len(ts[0]._shape) + 1)
    if d == 0:
        view = _stack_in_place(ts)
        if view is not None:
            return view
    return fast_aten_cat([fast_aten_unsqueeze(x, d) for x in ts], d)


def fast_aten_index_select(self, dim, index):
    t = _require(self)
    idx = _contig(_require(index))
    if idx._dtype not in (torch.int64,):
        idx = materialize_contiguous(idx, torch.int64)
    nd = len(t._shape)
    d = _norm_dim(dim, nd)
    src = _contig(t)
    n_idx = idx._numel
    outer = math.prod(src._shape[:d])
    inner = math.prod(src._shape[d + 1 :])
    rows = src._shape[d] if nd else 1
    shape = list(src._shape)
    if nd:
        shape[d] = n_idx
    out = _alloc(shape, t._dtype, t._device)
    if out._numel:
        eptr = _error_slot(t._device, _INDEX_ERROR)
        check(
            "mi355x_index_select",
            lib().mi355x_index_select(out._ptr, src._ptr, _code(src._dtype), idx._ptr, outer,
                                      n_idx, rows, inner, rows * inner, inner, eptr, _STREAM),
        )
    return out


# Device-side bounds errors.  Kernels that validate indices store 1 into an
# int32 slot of a persistent per-device flag buffer instead of faulting;
# nothing synchronises at launch.  The flags are read (and cleared) at the
# next device->host read, which waits for the queue anyway, and the error is
# raised there, like the reference's queued errors that surface at the next
# drain (eager_kernels/call_queue.py).
_ERROR_KINDS = (
    (IndexError, "index out of range in self"),
    (IndexError, "Target is out of bounds"),
)
_INDEX_ERROR, _TARGET_ERROR = 0, 1
_error_flags: dict = {}      # device index -> int32 [len(_ERROR_KINDS)] flag tensor
_errors_pending: set = set()  # devices with a flag launch since the last read


def _error_slot(device, kind):
    """Pointer to `kind`'s flag on `device`; the next host read checks it."""
    flags = _error_flags.get(device)
    if flags is None:
        flags = _alloc((len(_ERROR_KINDS),), torch.int32, device)
        fill_(flags, 0)
        _error_flags[device] = flags
    _errors_pending.add(device)
    return flags._ptr + 4 * kind


def raise_pending_device_errors():
    """Read the flags of every device with flagged launches since the last
    call, clear them, and raise the first recorded error.  Called before
    each device->host copy."""
    if not _errors_pending:
        return
    devices = list(_errors_pending)
    _errors_pending.clear()
    for dev in devices:
        flags = _error_flags[dev]
        host = flags._holder[: 4 * len(_ERROR_KINDS)].to("cpu", copy=True).view(torch.int32)
        if host.any():
            fill_(flags, 0)
            exc, message = _ERROR_KINDS[int(host.nonzero()[0, 0])]
            raise exc(message)


def fast_aten_index_tensor(self, indices):
    t = _require(self)
    idx = [i for i in indices]
    # Supported: a single integer index tensor on one dim (others None).
    nonnull = [(k, i) for k, i in enumerate(idx) if i is not None]
    if len(nonnull) == 1:
        k, it = nonnull[0]
        ti = _require(it)
        if ti._dtype == torch.bool:
            return NOT_HANDLED
        flat = fast_aten_view(_contig(ti), (-1,)) if ti._numel else ti
        sel = fast_aten_index_select(t, k, flat)
        shape = list(t._shape[:k]) + list(ti._shape) + list(t._shape[k + 1 :])
        return fast_aten_view(sel, shape)
    return NOT_HANDLED


# ---------------------------------------------------------------------------
# matmul family (fast_aten_mm / addmm / bmm, aten_fast.py:8713-8935)
# ---------------------------------------------------------------------------
def _gemm_operand(x: MT, rank: int):
    """(tensor, rs, cs, bs) with a unit row or column stride."""
    rs, cs = x._strides[-2], x._strides[-1]
    m, k = x._shape[-2], x._shape[-1]
    if cs == 1 or k == 1:
        cs = 1
        if m == 1:
            rs = k
    elif rs == 1 or m == 1:
        rs = 1
        if k == 1:
            cs = m
    else:
        x = materialize_contiguous(x)
        rs, cs = x._strides[-2], x._strides[-1]
    bs = x._strides[0] if rank == 3 else 0
    if rank == 3 and x._shape[0] == 1:
        bs = 0
    return x, rs, cs, bs


def _gemm(out: MT, a: MT, b: MT, bias=None, beta=0, batch=1, round_out=False, rowsum=None):
    """out = a @ b (+ bias) (+ out if beta); round_out rounds the result to
    the operands' 16-bit dtype before storing it in a wider out; rowsum
    (optional [m] or [batch, m] tensor) receives the row sums of a."""
    m, k = a._shape[-2], a._shape[-1]
    n = b._shape[-1]
    if out._numel == 0:
        return out
    if k == 0:
        if rowsum is not None:
            fill_(rowsum, 0)
        if beta:
            return out
        fill_(out, 0)
        if bias is not None:
            copy_into(out, bias)
        return out
    if a._dtype != b._dtype:
        raise RuntimeError(
            f"expected m1 and m2 to have the same dtype, but got: {a._dtype} != {b._dtype}"
        )
    if a._dtype not in _FLOAT_DTYPES:
        raise NotImplementedError(f"mm on the mojo device needs a floating dtype, got {a._dtype}")
    rank = len(a._shape)
    a, ars, acs, abs_ = _gemm_operand(a, rank)
    b, brs, bcs, bbs = _gemm_operand(b, rank)
    c_rs = out._strides[-2] if m > 1 else n
    c_bs = out._strides[0] if rank == 3 else 0
    ws = lib().mi355x_gemm_workspace_bytes(a._ptr, ars, acs, abs_, b._ptr, brs, bcs, bbs,
                                           _code(a._dtype), batch, m, n, k)
    hold, wptr = _workspace(ws, a._device)
    flags = (1 if beta else 0) | (2 if round_out else 0)
    check(
        "mi355x_gemm",
        lib().mi355x_gemm_ex(
            out._ptr, _code(out._dtype), c_rs, c_bs,
            a._ptr, ars, acs, abs_,
            b._ptr, brs, bcs, bbs,
            _code(a._dtype), bias._ptr if bias is not None else None,
            _code(bias._dtype) if bias is not None else 0, flags,
            rowsum._ptr if rowsum is not None else None, _code(rowsum._dtype) if rowsum is not None else 0,
            batch, m, n, k, ws_ptr_or_none(wptr), ws, _STREAM,
        ),
    )
    return out


def ws_ptr_or_none(p):
    return p if p else None


# ---------------------------------------------------------------------------
# fused linear (the autocast linear path: casts, GEMMs and the bias
# gradient as direct kernel calls, without per-view dispatches)
# ---------------------------------------------------------------------------
_LOW_ATTR = "_mojo_low_copy"
# MI355X_LAZY_LN_OUT=0 writes the f32 layer-norm output eagerly (A/B measurement)
_LAZY_LN_OUT = os.environ.get("MI355X_LAZY_LN_OUT", "1") != "0"
# MI355X_LAZY_CE=0 runs the fused cross-entropy forward at once (A/B measurement)
_LAZY_CE = os.environ.get("MI355X_LAZY_CE", "1") != "0"
# MI355X_LAZY_EMB_GRAD=0 writes the dense embedding gradient at once (A/B measurement)
_LAZY_EMB_GRAD = os.environ.get("MI355X_LAZY_EMB_GRAD", "1") != "0"
# MI355X_LAZY_GRAD_SCALE=0 runs a scalar-tensor _foreach_mul_ at once (A/B measurement)
_LAZY_GRAD_SCALE = os.environ.get("MI355X_LAZY_GRAD_SCALE", "1") != "0"


def _take_low_copy(t: MT, dtype):
    """The 16-bit copy of t that the kernel producing t wrote alongside it (a
    layer norm under autocast, whose f32 output the next linear casts), if t
    has not been modified since.  Each copy is handed out once, so the caller
    owns it like a fresh cast."""
    low = t.__dict__.pop(_LOW_ATTR, None) if hasattr(t, "__dict__") else None
    if low is None:
        return None
    copy, version = low
    if copy._dtype != dtype or t._version != version:
        return None
    return copy


# The autocast lower-precision dtype while an f32-policy op (layer norm) runs
# under autocast; set by the AutocastPrivateUse1 wrapper, since autocast
# reads as off below the Python dispatch key.
_autocast_low = None


def autocast_low_scope(dtype):
    """Context manager that marks an f32-policy op as running under autocast
    with lower-precision dtype `dtype`."""
    import contextlib

    @contextlib.contextmanager
    def scope():
        global _autocast_low
        prev, _autocast_low = _autocast_low, dtype
        try:
            yield
        finally:
            _autocast_low = prev

    return scope()


def _autocast_low_dtype():
    return _autocast_low if _autocast_low in (torch.bfloat16, torch.float16) else None


# Parameters the autocast forward casts (leaves that require grad): the
# fused AdamW step also writes each one's 16-bit copy, and the next forward's
# cast returns that copy.  A copy is dropped by any op that writes into the
# parameter's storage (see drop_param_copies_written_by) and is checked
# against the parameter's storage, address and version before each use.
_CAST_DTYPE_ATTR = "_mojo_autocast_dtype"
_PARAM_LOW_ATTR = "_mojo_param_low"
_param_low_by_holder: dict = {}  # id(storage holder) -> weakref to the parameter


def _param_low_copy(t: MT, dtype):
    rec = t.__dict__.get(_PARAM_LOW_ATTR) if hasattr(t, "__dict__") else None
    if rec is None:
        return None
    copy, holder, ptr, version = rec
    if copy._dtype != dtype or t._holder is not holder or t._ptr != ptr or t._version != version:
        drop_param_copy(t)
        return None
    return copy


def drop_param_copy(t) -> None:
    rec = t.__dict__.pop(_PARAM_LOW_ATTR, None)
    if rec is not None:
        _param_low_by_holder.pop(id(rec[1]), None)


def _set_param_copy(p: MT, copy: MT) -> None:
    import weakref

    drop_param_copy(p)
    p.__dict__[_PARAM_LOW_ATTR] = (copy, p._holder, p._ptr, p._version)
    _param_low_by_holder[id(p._holder)] = weakref.ref(p)


_written_args: dict = {}  # OpOverload -> tuple of (position, name) of written arguments


def drop_param_copies_written_by(func, args, kwargs) -> None:
    """Drop the parameter copies whose storage the op `func` writes."""
    spec = _written_args.get(func)
    if spec is None:
        spec = tuple(
            (i, a.name) for i, a in enumerate(func._schema.arguments)
            if a.alias_info is not None and a.alias_info.is_write
        )
        if func._schema.name in ("aten::_fused_adamw_", "aten::_fused_adam_"):
            # only the parameter list can hold parameter storage: the other
            # written lists are gradients, moments and step counters
            spec = tuple(x for x in spec if x[0] == 0)
        _written_args[func] = spec
    for i, name in spec:
        v = args[i] if i < len(args) else kwargs.get(name)
        for t in (v if isinstance(v, (list, tuple)) else (v,)):
            holder = getattr(t, "_holder", None)
            if holder is not None:
                ref = _param_low_by_holder.get(id(holder))
                if ref is not None:
                    prm = ref()
                    if prm is None:
                        _param_low_by_holder.pop(id(holder), None)
                    else:
                        drop_param_copy(prm)


def param_copies_active() -> bool:
    return bool(_param_low_by_holder)


def cast_to(t: MT, dtype) -> MT:
    """t in `dtype` (t itself when it already is)."""
    if t._dtype == dtype:
        return t
    low = _take_low_copy(t, dtype)
    if low is not None:
        return low
    if dtype in (torch.bfloat16, torch.float16) and t._dtype == torch.float32:
        low = _add_then_cast(t, dtype)
        if low is not None:
            return low
    if dtype in (torch.bfloat16, torch.float16) and t.requires_grad and t.is_leaf:
        low = _param_low_copy(t, dtype)
        if low is not None:
            return low
        t.__dict__[_CAST_DTYPE_ATTR] = dtype
    out = _alloc(t._shape, dtype, t._device)
    return copy_into(out, t)


def _add_then_cast(t: MT, dtype):
    """When t is a held-back f32 sum a + r (f32 or bf16 r), compute it and
    its `dtype` copy in one pass (mi355x_add_cast) and return the copy."""
    rec = take_pending(lambda r: r.out._holder is t._holder and r.out._ptr == t._ptr
                       and tuple(r.out._shape) == tuple(t._shape) and t._is_contiguous)
    if rec is None:
        return None
    ra, rr = rec.inputs
    if rr._dtype not in (torch.float32, torch.bfloat16):
        rec.launch()
        return None
    low = _alloc(t._shape, dtype, t._device)
    rc = lib().mi355x_add_cast(t._ptr, low._ptr, _code(dtype), ra._ptr, rr._ptr, _code(rr._dtype), t._numel, _STREAM)
    if rc:
        rec.launch()
        return None
    return low


def _rows_view(t: MT) -> MT:
    """[..., K] as a 2-D [M, K] view (materialised when the leading dims
    do not collapse)."""
    if len(t._shape) == 2:
        return t
    k = t._shape[-1]
    m = t._numel // k if k else 0
    if t._is_contiguous:
        return MT._view_of(t, (m, k), (k, 1), t._offset, True)
    lead_ok = t._strides[-1] == 1 or k == 1
    if lead_ok:
        # leading dims collapse when each stride equals the next one times its size
        st = t._strides[-2] if len(t._shape) >= 2 else k
        ok = True
        for i in range(len(t._shape) - 2):
            if t._shape[i] != 1 and t._strides[i] != t._strides[i + 1] * t._shape[i + 1]:
                ok = False
                break
        if ok:
            return MT._view_of(t, (m, k), (st, 1), t._offset)
    c = materialize_contiguous(t)
    return MT._view_of(c, (m, k), (k, 1), c._offset, True)


def linear_forward(x: MT, w: MT, b) -> MT:
    """out[..., N] = x[..., K] @ w[N, K]^T (+ b), one GEMM with the bias
    in its epilogue (aten_fast.py:8755-8812 counterpart)."""
    n, k = w._shape
    x2 = _rows_view(x)
    out = _alloc(tuple(x._shape[:-1]) + (n,), x._dtype, x._device)
    o2 = MT._view_of(out, (x2._shape[0], n), (n, 1), 0, True)
    wt = MT._view_of(w, (k, n), (w._strides[1], w._strides[0]), w._offset)
    if b is not None and b._strides[-1] == 1:
        _gemm(o2, x2, wt, bias=b)
    else:
        _gemm(o2, x2, wt)
        if b is not None:
            _map_call(OP["add"], o2, [(o2, o2._dtype), (b, b._dtype)], 1.0, 0.0)
    return out


def linear_backward(dy: MT, x: MT, w: MT, need_x: bool, need_w: bool, need_b: bool,
                    x_dtype, w_dtype, b_dtype):
    """(dx, dw, db) of linear_forward (aten_fast.py:8815-8907): dx = dy w,
    dw = dy^T x, db = sum(dy, 0), computed in the forward's 16-bit dtype and
    delivered in x_dtype / w_dtype / b_dtype: a wider dtype gets the 16-bit
    result widened (the GEMM rounds before storing), as the autocast casts'
    own backward would produce.  db comes out of the dW GEMM as the row sums
    of dy^T, so dy is read once for both."""
    n, k = w._shape
    d2 = _rows_view(dy)
    m = d2._shape[0]
    cdt = dy._dtype
    dx = dw = db = None
    if need_x:
        dx = _alloc(tuple(dy._shape[:-1]) + (k,), x_dtype, dy._device)
        _gemm(MT._view_of(dx, (m, k), (k, 1), 0, True), d2, w, round_out=x_dtype != cdt)
    if need_b:
        db = _alloc((n,), b_dtype, dy._device)
    if need_w:
        x2 = _rows_view(x)
        dw = _alloc((n, k), w_dtype, dy._device)
        dyt = MT._view_of(d2, (n, m), (d2._strides[1], d2._strides[0]), d2._offset)
        _gemm(dw, dyt, x2, round_out=w_dtype != cdt or (need_b and b_dtype != cdt), rowsum=db)
    elif need_b:
        r = _reduce(RED["sum"], d2, [0], False, cdt)
        db = cast_to(r, b_dtype)
    return dx, dw, db


def fast_aten_mm(self, mat2):
    a, b = _require(self), _require(mat2)
    if len(a._shape) != 2 or len(b._shape) != 2:
        raise RuntimeError("mm: both arguments must be 2-D")
    if a._shape[1] != b._shape[0]:
        raise RuntimeError(
            f"mat1 and mat2 shapes cannot be multiplied ({a._shape[0]}x{a._shape[1]} and"
            f" {b._shape[0]}x{b._shape[1]})"
        )
    out = _alloc((a._shape[0], b._shape[1]), a._dtype, a._device)
    return _gemm(out, a, b)


def fast_aten_addmm(self, mat1, mat2, *, beta=1, alpha=1):
    bias, a, b = _require(self), _require(mat1), _require(mat2)
    if len(a._shape) != 2 or len(b._shape) != 2 or a._shape[1] != b._shape[0]:
        raise RuntimeError(
            f"mat1 and mat2 shapes cannot be multiplied ({a._shape[0]}x{a._shape[1]} and"
            f" {b._shape[0]}x{b._shape[1]})"
        )
    m, n = a._shape[0], b._shape[1]
    out = _alloc((m, n), a._dtype, a._device)
    if alpha == 1 and beta == 1:
        if bias._shape in ((n,), (1, n)) and (bias._numel == 1 or bias._strides[-1] == 1):
            return _gemm(out, a, b, bias=bias)
        copy_into(out, bias)
        return _gemm(out, a, b, beta=1)
    prod = _gemm(out, a, b)
    if alpha != 1:
        prod = _map_call(OP["mul"], prod, [(prod, prod._dtype), (None, torch.float32)], 0.0, float(alpha))
    if beta == 0:
        return prod
    return _map_call(OP["add"], prod, [(prod, prod._dtype), (bias, bias._dtype)], float(beta))


def fast_aten_bmm(self, mat2):
    a, b = _require(self), _require(mat2)
    if len(a._shape) != 3 or len(b._shape) != 3 or a._shape[0] != b._shape[0] or a._shape[2] != b._shape[1]:
        raise RuntimeError(f"bmm: shape mismatch {a._shape} x {b._shape}")
    out = _alloc((a._shape[0], a._shape[1], b._shape[2]), a._dtype, a._device)
    return _gemm(out, a, b, batch=a._shape[0])


# ---------------------------------------------------------------------------
# layer norm (aten_fast.py:5248-5517)
# ---------------------------------------------------------------------------
def fast_aten_native_layer_norm(input, normalized_shape, weight, bias, eps):
    a = _require(input)
    normalized_shape = tuple(normalized_shape)
    k = len(normalized_shape)
    if a._dtype not in _FLOAT_DTYPES or k < 1 or tuple(a._shape[-k:]) != normalized_shape:
        return NOT_HANDLED
    cols = math.prod(normalized_shape)
    rows = a._numel // cols if cols else 0
    g = _t(weight) if weight is not None else None
    b = _t(bias) if bias is not None else None
    for p in (g, b):
        if p is not None and (tuple(p._shape) != normalized_shape):
            return NOT_HANDLED
    x = _contig(a)
    g = None if g is None else (_contig(g) if g._dtype == a._dtype else materialize_contiguous(g, a._dtype))
    b = None if b is None else (_contig(b) if b._dtype == a._dtype else materialize_contiguous(b, a._dtype))
    out = _alloc(a._shape, a._dtype, a._device)
    stat_shape = tuple(a._shape[:-k]) + (1,) * k
    mean = _alloc(stat_shape, torch.float32, a._device)
    rstd = _alloc(stat_shape, torch.float32, a._device)
    # Under autocast an f32 layer norm feeds a lower-precision matmul: the
    # kernel also writes y in that dtype, which the cast then takes.
    low_dt = _autocast_low_dtype() if a._dtype == torch.float32 else None
    low = _alloc(a._shape, low_dt, a._device) if (low_dt is not None and rows and cols) else None
    # With the 16-bit copy written, the f32 y is left to a lazy launch: in an
    # autocast step only the copy is read (the next linear takes it).
    defer_y = low is not None and _LAZY_LN_OUT
    y_ptr = None if defer_y else out._ptr
    # the input is a held-back residual add: compute it in the norm's pass
    rec = take_pending(lambda r: r.out._holder is x._holder and r.out._ptr == x._ptr
                       and tuple(r.out._shape) == tuple(x._shape)) if rows and cols else None
    fused = False
    if rec is not None:
        ra, rr = rec.inputs
        rc = lib().mi355x_layer_norm_fwd_add(
            y_ptr, low._ptr if low is not None else None, _code(low_dt) if low is not None else 0,
            mean._ptr, rstd._ptr, x._ptr, ra._ptr, rr._ptr, _code(rr._dtype), g._ptr if g is not None else None,
            b._ptr if b is not None else None, rows, cols, float(eps), _code(a._dtype), _STREAM,
        )
        fused = rc == 0
        if not fused:
            rec.launch()  # shape the fused kernel does not take: the add, then the norm
    if rows and cols and not fused:
        check(
            "mi355x_layer_norm_fwd_ex",
            lib().mi355x_layer_norm_fwd_ex(
                y_ptr, low._ptr if low is not None else None, _code(low_dt) if low is not None else 0,
                mean._ptr, rstd._ptr, x._ptr, g._ptr if g is not None else None,
                b._ptr if b is not None else None, rows, cols, float(eps), _code(a._dtype), _STREAM,
            ),
        )
    if low is not None:
        setattr(out, _LOW_ATTR, (low, out._version))
    if defer_y:
        def fill(y=out._ptr, x=x, mean=mean, rstd=rstd, g=g, b=b, code=_code(a._dtype)):
            check("mi355x_layer_norm_apply", lib().mi355x_layer_norm_apply(
                y, x._ptr, mean._ptr, rstd._ptr, g._ptr if g is not None else None,
                b._ptr if b is not None else None, rows, cols, code, _STREAM))

        lazy(out, [t for t in (x, mean, rstd, g, b) if t is not None], fill)
    if a._dtype != torch.float32:
        # ATen returns the statistics in the input dtype (aten_fast.py:5228-5245)
        mean = materialize_contiguous(mean, a._dtype)
        rstd = materialize_contiguous(rstd, a._dtype)
    return out, mean, rstd


def fast_aten_native_layer_norm_backward(
    grad_out, input, normalized_shape, mean, rstd, weight, bias, output_mask
):
    a = _require(input)
    dy = _contig(_require(grad_out))
    normalized_shape = tuple(normalized_shape)
    k = len(normalized_shape)
    cols = math.prod(normalized_shape)
    rows = a._numel // cols if cols else 0
    x = _contig(a)
    if dy._dtype != a._dtype:
        dy = materialize_contiguous(dy, a._dtype)
    mu = _require(mean)
    rs = _require(rstd)
    mu = _contig(mu) if mu._dtype == torch.float32 else materialize_contiguous(mu, torch.float32)
    rs = _contig(rs) if rs._dtype == torch.float32 else materialize_contiguous(rs, torch.float32)
    g = _t(weight) if weight is not None else None
    if g is not None and g._dtype != a._dtype:
        g = materialize_contiguous(g, a._dtype)
    elif g is not None:
        g = _contig(g)
    want_dx, want_dw, want_db = (bool(m) for m in output_mask)
    dx = _alloc(a._shape, a._dtype, a._device) if want_dx else None
    pdt = g._dtype if g is not None else a._dtype
    dw = _alloc(normalized_shape, a._dtype, a._device) if (want_dw and weight is not None) else None
    db = _alloc(normalized_shape, a._dtype, a._device) if (want_db and bias is not None) else None
    ws = lib().mi355x_layer_norm_bwd_workspace_bytes(rows, cols) if (dw is not None or db is not None) else 0
    hold, wptr = _workspace(ws, a._device)
    check(
        "mi355x_layer_norm_bwd",
        lib().mi355x_layer_norm_bwd(
            dx._ptr if dx is not None else None, dw._ptr if dw is not None else None,
            db._ptr if db is not None else None, dy._ptr, x._ptr, mu._ptr, rs._ptr,
            g._ptr if g is not None else None, rows, cols, _code(a._dtype), wptr, ws, _STREAM,
        ),
    )
    if dw is not None and weight is not None and weight.dtype != dw._dtype:
        dw = materialize_contiguous(dw, weight.dtype)
    if db is not None and bias is not None and bias.dtype != db._dtype:
        db = materialize_contiguous(db, bias.dtype)
    del pdt
    return dx, dw, db


# ---------------------------------------------------------------------------
# GELU (aten_fast.py:2940-3009)
# ---------------------------------------------------------------------------
def _approx_code(approximate):
    if approximate in (None, "none"):
        return 0
    if approximate == "tanh":
        return 1
    raise RuntimeError(f"approximate argument must be either none or tanh, got {approximate}")


def fast_aten_gelu(self, *, approximate="none", out=None):
    t = _require(self)
    if t._dtype not in _FLOAT_DTYPES:
        return NOT_HANDLED
    x = _contig(t)
    y = _alloc(t._shape, t._dtype, t._device)
    if y._numel:
        check("mi355x_gelu_fwd", lib().mi355x_gelu_fwd(y._ptr, x._ptr, y._numel, _approx_code(approximate), _code(t._dtype), _STREAM))
    if out is not None:
        return copy_into(_require(out), y)
    return y


def fast_aten_gelu_(self, *, approximate="none"):
    t = _require(self)
    y = fast_aten_gelu(t, approximate=approximate)
    copy_into(t, y)
    return self


def fast_aten_gelu_backward(grad_output, self, *, approximate="none"):
    t = _require(self)
    dy = _require(grad_output)
    if t._dtype not in _FLOAT_DTYPES:
        return NOT_HANDLED
    x = _contig(t)
    if dy._dtype != t._dtype or tuple(dy._shape) != tuple(t._shape):
        dy = materialize_contiguous(fast_aten_expand(dy, t._shape), t._dtype)
    dy = _contig(dy)
    dx = _alloc(t._shape, t._dtype, t._device)
    if dx._numel:
        check("mi355x_gelu_bwd", lib().mi355x_gelu_bwd(dx._ptr, dy._ptr, x._ptr, dx._numel, _approx_code(approximate), _code(t._dtype), _STREAM))
    return dx


# ---------------------------------------------------------------------------
# softmax / log_softmax (aten_fast.py:5792-5971, 9220-9254)
# ---------------------------------------------------------------------------
def _lastdim_view(t: MT, dim):
    nd = len(t._shape)
    d = _norm_dim(dim, nd)
    if d == nd - 1 or nd == 0:
        return _contig(t), None
    perm = [i for i in range(nd) if i != d] + [d]
    return materialize_contiguous(fast_aten_permute(t, perm)), perm


def _restore_dim(y: MT, perm, shape):
    if perm is None:
        return y
    inv = [0] * len(perm)
    for i, p in enumerate(perm):
        inv[p] = i
    return materialize_contiguous(fast_aten_permute(y, inv))


def _softmax_impl(self, dim, half_to_float, log):
    t = _require(self)
    if t._dtype not in _FLOAT_DTYPES:
        return NOT_HANDLED
    out_dtype = torch.float32 if half_to_float else t._dtype
    x, perm = _lastdim_view(t, dim)
    cols = x._shape[-1] if x._shape else 1
    rows = x._numel // cols if cols else 0
    y = _alloc(x._shape, out_dtype, t._device)
    if y._numel:
        check("mi355x_softmax_fwd", lib().mi355x_softmax_fwd(y._ptr, _code(out_dtype), x._ptr, _code(x._dtype), rows, cols, int(log), _STREAM))
    return _restore_dim(y, perm, t._shape)


def fast_aten__softmax(self, dim, half_to_float):
    return _softmax_impl(self, dim, half_to_float, False)


def fast_aten__log_softmax(self, dim, half_to_float):
    return _softmax_impl(self, dim, half_to_float, True)


def _softmax_bwd_impl(grad_output, output, dim, input_dtype, log):
    dy_t, y_t = _require(grad_output), _require(output)
    dy, perm = _lastdim_view(dy_t, dim)
    y, _ = _lastdim_view(y_t, dim)
    cols = y._shape[-1] if y._shape else 1
    rows = y._numel // cols if cols else 0
    dx = _alloc(y._shape, input_dtype, y._device)
    if dx._numel:
        check("mi355x_softmax_bwd", lib().mi355x_softmax_bwd(dx._ptr, _code(input_dtype), dy._ptr, _code(dy._dtype), y._ptr, _code(y._dtype), rows, cols, int(log), _STREAM))
    return _restore_dim(dx, perm, y_t._shape)


def fast_aten__softmax_backward_data(grad_output, output, dim, input_dtype):
    return _softmax_bwd_impl(grad_output, output, dim, input_dtype, False)


def fast_aten__log_softmax_backward_data(grad_output, output, dim, input_dtype):
    return _softmax_bwd_impl(grad_output, output, dim, input_dtype, True)


# ---------------------------------------------------------------------------
# NLL loss (aten_fast.py:5974-6130)
# ---------------------------------------------------------------------------
def _nll_shapes(lp: MT, target: MT):
    if len(lp._shape) == 1:
        return 1, lp._shape[0]
    if len(lp._shape) == 2:
        return lp._shape[0], lp._shape[1]
    return None


def fast_aten_nll_loss_forward(self, target, weight, reduction, ignore_index):
    lp = _require(self)
    tg = _require(target)
    shp = _nll_shapes(lp, tg)
    if shp is None or lp._dtype not in _FLOAT_DTYPES:
        return NOT_HANDLED
    n, c = shp
    if tg._numel != n:
        raise ValueError(f"Expected input batch_size ({n}) to match target batch_size ({tg._numel}).")
    x = _contig(lp)
    tgt = _contig(tg) if tg._dtype == torch.int64 else materialize_contiguous(tg, torch.int64)
    w = None
    if weight is not None:
        w = _require(weight)
        w = _contig(w) if w._dtype == lp._dtype else materialize_contiguous(w, lp._dtype)
    out_shape = (n,) if (reduction == 0 and len(lp._shape) == 2) else ()
    out = _alloc(out_shape, lp._dtype, lp._device)
    total = _alloc((), lp._dtype, lp._device)
    ws = lib().mi355x_nll_workspace_bytes(n)
    hold, wptr = _workspace(ws, lp._device)
    eptr = _error_slot(lp._device, _TARGET_ERROR)
    check(
        "mi355x_nll_fwd",
        lib().mi355x_nll_fwd(out._ptr, total._ptr, x._ptr, _code(lp._dtype), tgt._ptr,
                             w._ptr if w is not None else None, n, c, int(reduction),
                             int(ignore_index), eptr, wptr, ws, _STREAM),
    )
    return out, total


def fast_aten_nll_loss_backward(grad_output, self, target, weight, reduction, ignore_index, total_weight):
    lp = _require(self)
    tg = _require(target)
    shp = _nll_shapes(lp, tg)
    if shp is None:
        return NOT_HANDLED
    n, c = shp
    go = _contig(_require(grad_output))
    if go._dtype != lp._dtype:
        go = materialize_contiguous(go, lp._dtype)
    tgt = _contig(tg) if tg._dtype == torch.int64 else materialize_contiguous(tg, torch.int64)
    w = None
    if weight is not None:
        w = _require(weight)
        w = _contig(w) if w._dtype == lp._dtype else materialize_contiguous(w, lp._dtype)
    tw = _require(total_weight)
    if tw._dtype != lp._dtype:
        tw = materialize_contiguous(tw, lp._dtype)
    gi = _alloc(lp._shape, lp._dtype, lp._device)
    if gi._numel:
        check(
            "mi355x_nll_bwd",
            lib().mi355x_nll_bwd(gi._ptr, go._ptr, tgt._ptr, w._ptr if w is not None else None,
                                 tw._ptr, n, c, int(reduction), int(ignore_index), _code(lp._dtype), _STREAM),
        )
    return gi


# ---------------------------------------------------------------------------
# embedding (aten_fast.py:9262-9368)
# ---------------------------------------------------------------------------
def fast_aten_embedding(weight, indices, padding_idx=-1, scale_grad_by_freq=False, sparse=False):
    w = _require(weight)
    idx = _require(indices)
    if len(w._shape) != 2:
        return NOT_HANDLED
    if idx._dtype not in (torch.int64, torch.int32):
        raise RuntimeError(
            "Expected tensor for argument #1 'indices' to have one of the following scalar types:"
            f" Long, Int; but got {idx._dtype} instead"
        )
    ids = _contig(idx) if idx._dtype == torch.int64 else materialize_contiguous(idx, torch.int64)
    num, dim = w._shape
    wsrc = w if w._strides[1] == 1 else materialize_contiguous(w)
    out = _alloc(tuple(idx._shape) + (dim,), w._dtype, w._device)
    if out._numel:
        eptr = _error_slot(w._device, _INDEX_ERROR)
        check(
            "mi355x_embedding_fwd",
            lib().mi355x_embedding_fwd(out._ptr, wsrc._ptr, _code(w._dtype), ids._ptr, ids._numel,
                                       num, dim, wsrc._strides[0], eptr, _STREAM),
        )
    return out


def fast_aten_embedding_dense_backward(grad_output, indices, num_weights, padding_idx, scale_grad_by_freq):
    if scale_grad_by_freq:
        return NOT_HANDLED
    go = _require(grad_output)
    idx = _require(indices)
    ids = _contig(idx) if idx._dtype == torch.int64 else materialize_contiguous(idx, torch.int64)
    dim = go._shape[-1]
    g = _contig(go)
    gw = _alloc((num_weights, dim), go._dtype, go._device)

    def run(dst, base=None, g=g, ids=ids, pad=int(padding_idx), code=_code(go._dtype), dev=go._device):
        ws = lib().mi355x_embedding_bwd_workspace_bytes(ids._numel, num_weights)
        hold, wptr = _workspace(ws, dev)
        if base is None:
            check("mi355x_embedding_bwd", lib().mi355x_embedding_bwd(
                dst, g._ptr, code, ids._ptr, ids._numel, num_weights, dim, pad, wptr, ws, _STREAM))
        else:
            check("mi355x_embedding_bwd_accumulate", lib().mi355x_embedding_bwd_accumulate(
                dst, base, g._ptr, code, ids._ptr, ids._numel, num_weights, dim, pad, wptr, ws, _STREAM))

    if _LAZY_EMB_GRAD:
        # A tied embedding's gradient is added to the output projection's by
        # autograd (`a + this` in its input buffer, or `grad += this`): left
        # lazy, that add takes it as a scatter-add of the named rows (no
        # dense gradient written, no dense add of it).
        lazy(gw, [g, ids], lambda y=gw._ptr: run(y),
             consumers={torch.ops.aten.add.Tensor: {0, 1}, torch.ops.aten.add_.Tensor: {1}},
             accumulate=lambda dst, base: run(dst._ptr, base._ptr))
    else:
        run(gw._ptr)
    return gw


def _add_lazy(a: MT, b: MT, alpha, inplace: bool):
    """a + alpha*b (into a when `inplace`) when one operand is a lazy output
    that can add itself onto the other (see fast_aten_embedding_dense_backward):
    the result, written by that record's accumulate.  Otherwise the lazy
    operands are materialized and None returned (the caller adds as usual)."""
    from . import lazy_record, materialize

    ra, rb = lazy_record(a), lazy_record(b)
    if ra is None and rb is None:
        return None
    # the operand whose record can add itself onto the other (b first: in
    # place, only b can); the other operand's own pending work runs first
    if rb is not None and rb.accumulate is not None:
        rec, base = rb, a
    elif ra is not None and ra.accumulate is not None and not inplace:
        rec, base = ra, b
    else:
        rec = base = None
    if (rec is not None and rec is not lazy_record(base) and float(_scalar_value(alpha)) == 1.0
            and a._dtype == b._dtype and tuple(a._shape) == tuple(b._shape) and a._is_contiguous
            and b._is_contiguous and a._holder is not b._holder):
        materialize(base)
        dst = a if inplace else _alloc(a._shape, a._dtype, a._device)
        rec.accumulate(dst, base)
        return dst
    for t in (a, b):
        materialize(t)
    return None


# ---------------------------------------------------------------------------
# scaled dot-product attention (aten_fast.py:7462-7839, 9102-9211)
# ---------------------------------------------------------------------------
def _bhs(t: MT):
    return _i64(t._strides[:3])


_FUSED_FA_HEAD_DIMS = (32, 64, 128)  # the MFMA forward + backward
_MFMA_EX_HEAD_DIMS = (64, 128, 256)   # the MFMA forward with grouped K/V heads / a window
_FUSED_FA_MAX_HEAD_DIM = 256          # the fused gate (aten_fast.py:7420)


def fused_fa_inputs(query, key, value, attn_mask, dropout_p, is_causal, scale, enable_gqa):
    """Eligible [B,H,S,D] q/k/v for the fused flash pair, or None (metadata
    only; the gate of aten_fast.py:7462-7530 minus its gfx942 check: f32,
    bf16 or f16, head_dim up to 256, no mask, dropout or grouped heads).
    bf16/f16 at head_dim 32, 64 or 128 run on MFMA; the rest on the f32
    kernels of csrc/attention_generic.hip."""
    q, k, v = _t(query), _t(key), _t(value)
    if (
        q is None or k is None or v is None
        or attn_mask is not None or enable_gqa
        or float(dropout_p) != 0.0
        or q._device != k._device or q._device != v._device
        or q._dtype not in _FLOAT_DTYPES
        or q._dtype != k._dtype or q._dtype != v._dtype
        or len(q._shape) != 4 or len(k._shape) != 4 or len(v._shape) != 4
    ):
        return None
    if tuple(q._shape[:2]) != tuple(k._shape[:2]) or tuple(k._shape) != tuple(v._shape) or q._shape[3] != k._shape[3]:
        return None
    b, h, sq, d = q._shape
    skv = k._shape[2]
    if min(b, h, sq, skv, d) <= 0 or d > _FUSED_FA_MAX_HEAD_DIM:
        return None
    if scale is not None and not math.isfinite(float(scale)):
        return None
    return q, k, v


def _fa_head_contig(t: MT) -> MT:
    """t itself when the MFMA kernels can read it in place (unit head_dim
    stride, 16-byte aligned base, (b, h, s) strides multiples of 8
    elements), else a contiguous copy."""
    st = t._strides
    if st[3] == 1 and t._ptr % 16 == 0 and st[0] % 8 == 0 and st[1] % 8 == 0 and st[2] % 8 == 0:
        return t
    return materialize_contiguous(t)


def _unit_head_stride(t: MT) -> MT:
    """t itself when its head_dim stride is 1 (all the f32 kernels need), else
    a contiguous copy."""
    return t if t._strides[3] == 1 or t._shape[3] == 1 else materialize_contiguous(t)


def alloc_bthd(b, h, s, d, dtype, device) -> MT:
    """[B,H,S,D] view over dense [B,S,H,D] storage (aten_fast.py:7433-7459):
    `out.transpose(1, 2)` is then a free contiguous [B,S,H,D]."""
    dense = _alloc((b, s, h, d), dtype, device)
    return MT._view_of(dense, (b, h, s, d), (s * h * d, d, h * d, 1), 0)


def _mfma_fwd_ok(q: MT, group, window) -> bool:
    d = q._shape[3]
    if q._dtype not in _MFMA_DTYPES:
        return False
    if group == 1 and window == 0 and d in _FUSED_FA_HEAD_DIMS:
        return True
    return d in _MFMA_EX_HEAD_DIMS


def _mfma_bwd_ok(q: MT, group, window) -> bool:
    return q._dtype in _MFMA_DTYPES and group == 1 and window == 0 and q._shape[3] in _FUSED_FA_HEAD_DIMS


def attention_forward(q: MT, k: MT, v: MT, causal, window, scale):
    """(out [B,H,Sq,D] over BTHD storage, lse f32 [B,H,Sq]) of causal / full
    attention with optional grouped K/V heads (k, v with H / g heads) and a
    causal sliding window: MFMA kernels where they apply, else the f32
    kernels."""
    b, h, sq, d = q._shape
    hk, skv = k._shape[1], k._shape[2]
    scale_value = float(scale) if scale is not None else 1.0 / math.sqrt(d)
    out = alloc_bthd(b, h, sq, d, q._dtype, q._device)
    lse = _alloc((b, h, sq), torch.float32, q._device)
    if _mfma_fwd_ok(q, h // hk, window):
        q, k, v = _fa_head_contig(q), _fa_head_contig(k), _fa_head_contig(v)
        check(
            "mi355x_attn_fwd_ex",
            lib().mi355x_attn_fwd_ex(out._ptr, _bhs(out), lse._ptr, q._ptr, _bhs(q), k._ptr, _bhs(k),
                                     v._ptr, _bhs(v), b, h, hk, sq, skv, d, scale_value, int(bool(causal)),
                                     int(window), _code(q._dtype), _STREAM),
        )
    else:
        q, k, v = _unit_head_stride(q), _unit_head_stride(k), _unit_head_stride(v)
        check(
            "mi355x_attn_fwd_gen",
            lib().mi355x_attn_fwd_gen(out._ptr, _bhs(out), lse._ptr, q._ptr, _bhs(q), k._ptr, _bhs(k),
                                      v._ptr, _bhs(v), b, h, hk, sq, skv, d, scale_value, int(bool(causal)),
                                      int(window), _code(q._dtype), _STREAM),
        )
    return out, lse


def attention_backward(grad_out, q: MT, k: MT, v: MT, out: MT, lse: MT, causal, window, scale):
    """(dq, dk, dv) of attention_forward: dk/dv have k's heads (the query
    heads of each group summed)."""
    b, h, sq, d = q._shape
    hk, skv = k._shape[1], k._shape[2]
    scale_value = float(scale) if scale is not None else 1.0 / math.sqrt(d)
    if grad_out._dtype != q._dtype:
        grad_out = materialize_contiguous(grad_out, q._dtype)
    lse = _contig(lse)
    if hk == h and skv == sq:
        # dQ, dK, dV side by side in one [B, S, 3, H, D] buffer: the backward of
        # the fused qkv projection's split is then a cat of adjacent slices,
        # which fast_aten_cat returns as a view of this buffer (no copies)
        dense = _alloc((b, sq, 3, h, d), q._dtype, q._device)
        st = (sq * 3 * h * d, d, 3 * h * d, 1)
        dq, dk, dv = (MT._view_of(dense, (b, h, sq, d), st, i * h * d) for i in range(3))
        _mark_cat_ready(dense)
    else:
        dq = alloc_bthd(b, h, sq, d, q._dtype, q._device)
        dk = alloc_bthd(b, hk, skv, d, q._dtype, q._device)
        dv = alloc_bthd(b, hk, skv, d, q._dtype, q._device)
    if _mfma_bwd_ok(q, h // hk, window):
        q, k, v = _fa_head_contig(q), _fa_head_contig(k), _fa_head_contig(v)
        out, dout = _fa_head_contig(out), _fa_head_contig(grad_out)
        ws = lib().mi355x_attn_bwd_workspace_bytes(b, h, sq, skv, d)
        hold, wptr = _workspace(ws, q._device)
        check(
            "mi355x_attn_bwd",
            lib().mi355x_attn_bwd(
                dq._ptr, _bhs(dq), dk._ptr, _bhs(dk), dv._ptr, _bhs(dv), dout._ptr, _bhs(dout),
                q._ptr, _bhs(q), k._ptr, _bhs(k), v._ptr, _bhs(v), out._ptr, _bhs(out), lse._ptr,
                b, h, sq, skv, d, scale_value, int(bool(causal)), _code(q._dtype), wptr, ws, _STREAM,
            ),
        )
    else:
        q, k, v = _unit_head_stride(q), _unit_head_stride(k), _unit_head_stride(v)
        out, dout = _unit_head_stride(out), _unit_head_stride(grad_out)
        ws = lib().mi355x_attn_bwd_gen_workspace_bytes(b, h, hk, sq, skv, d)
        hold, wptr = _workspace(ws, q._device)
        check(
            "mi355x_attn_bwd_gen",
            lib().mi355x_attn_bwd_gen(
                dq._ptr, _bhs(dq), dk._ptr, _bhs(dk), dv._ptr, _bhs(dv), dout._ptr, _bhs(dout),
                q._ptr, _bhs(q), k._ptr, _bhs(k), v._ptr, _bhs(v), out._ptr, _bhs(out), lse._ptr,
                b, h, hk, sq, skv, d, scale_value, int(bool(causal)), int(window), _code(q._dtype),
                wptr, ws, _STREAM,
            ),
        )
    return dq, dk, dv


def fused_flash_attention_forward(q: MT, k: MT, v: MT, is_causal, scale):
    return attention_forward(q, k, v, is_causal, 0, scale)


def fused_flash_attention_backward(grad_out, q, k, v, out, lse, is_causal, scale):
    return attention_backward(grad_out, q, k, v, out, lse, is_causal, 0, scale)


def fast_aten__scaled_dot_product_flash_attention(
    query, key, value, dropout_p=0.0, is_causal=False, return_debug_mask=False, *, scale=None
):
    """The ATen flash-pair forward contract (aten_fast.py:7699-7734):
    (out, lse f32 [B,H,Sq], cum_seq_q, cum_seq_k, Sq, Sk, rng_state u64[2],
    unused u64[], debug_attn_mask)."""
    if dropout_p != 0.0 or return_debug_mask:
        return NOT_HANDLED
    inputs = fused_fa_inputs(query, key, value, None, dropout_p, is_causal, scale, False)
    if inputs is None:
        return NOT_HANDLED
    q, k, v = inputs
    out, lse = fused_flash_attention_forward(q, k, v, is_causal, scale)
    dev = q._device
    rng_state = fill_(_alloc((2,), torch.uint64, dev), 0) if hasattr(torch, "uint64") and torch.uint64 in DTYPE_CODE else _alloc((2,), torch.int64, dev)
    unused = _alloc((0,), rng_state._dtype, dev)
    debug_attn_mask = _alloc((0,), q._dtype, dev)
    return (out, lse, None, None, q._shape[2], k._shape[2], rng_state, unused, debug_attn_mask)


def fast_aten__scaled_dot_product_flash_attention_backward(
    grad_out, query, key, value, out, logsumexp, cum_seq_q, cum_seq_k, max_q, max_k,
    dropout_p, is_causal, philox_seed, philox_offset, *, scale=None,
):
    if dropout_p != 0.0 or cum_seq_q is not None and _t(cum_seq_q) is not None and cum_seq_q.numel():
        return NOT_HANDLED
    inputs = fused_fa_inputs(query, key, value, None, 0.0, is_causal, scale, False)
    if inputs is None:
        return NOT_HANDLED
    q, k, v = inputs
    o = _t(out)
    lse = _t(logsumexp)
    if o is None or lse is None:
        o, lse = fused_flash_attention_forward(q, k, v, is_causal, scale)
    return fused_flash_attention_backward(_require(grad_out), q, k, v, o, lse, is_causal, scale)


def sdpa_math(query, key, value, attn_mask=None, dropout_p=0.0, is_causal=False, scale=None, enable_gqa=False):
    """Decomposed SDPA built from device ops (differentiable through them)."""
    if dropout_p != 0.0:
        raise NotImplementedError("scaled_dot_product_attention with dropout is not supported on the mojo device")
    d = query.shape[-1]
    s = scale if scale is not None else 1.0 / math.sqrt(d)
    if enable_gqa and key.shape[-3] != query.shape[-3]:
        rep = query.shape[-3] // key.shape[-3]
        key = key.repeat_interleave(rep, dim=-3)
        value = value.repeat_interleave(rep, dim=-3)
    scores = torch.matmul(query, key.transpose(-2, -1)) * s
    if is_causal:
        sq, skv = query.shape[-2], key.shape[-2]
        rows = torch.arange(sq, device=query.device).view(sq, 1)
        cols = torch.arange(skv, device=query.device).view(1, skv)
        keep = rows >= cols  # top-left aligned causal mask
        scores = scores.masked_fill(keep.logical_not(), float("-inf"))
    if attn_mask is not None:
        if attn_mask.dtype == torch.bool:
            scores = scores.masked_fill(attn_mask.logical_not(), float("-inf"))
        else:
            scores = scores + attn_mask
    probs = torch.softmax(scores, dim=-1)
    return torch.matmul(probs, value)


def fused_fa_ex_inputs(query, key, value, attn_mask, dropout_p, is_causal, scale, enable_gqa):
    """Fused attention beyond the flash-pair gate: grouped K/V heads
    (enable_gqa) and a sliding-window causal mask built by
    torch_mojo_backend.masks.  Returns (q, k, v, causal, window) or None."""
    from ..masks import window_of

    q, k, v = _t(query), _t(key), _t(value)
    if (
        q is None or k is None or v is None
        or float(dropout_p) != 0.0
        or q._device != k._device or q._device != v._device
        or q._dtype not in _FLOAT_DTYPES
        or q._dtype != k._dtype or q._dtype != v._dtype
        or len(q._shape) != 4 or len(k._shape) != 4 or len(v._shape) != 4
    ):
        return None
    b, h, sq, d = q._shape
    hk, skv = k._shape[1], k._shape[2]
    if k._shape[0] != b or tuple(k._shape) != tuple(v._shape) or k._shape[3] != d:
        return None
    if hk != h and not (enable_gqa and hk > 0 and h % hk == 0):
        return None
    if min(b, h, sq, skv, d) <= 0 or d > _FUSED_FA_MAX_HEAD_DIM:
        return None
    if scale is not None and not math.isfinite(float(scale)):
        return None
    causal, window = bool(is_causal), 0
    if attn_mask is not None:
        w = window_of(attn_mask)
        if w is None or is_causal or sq != skv:
            return None
        causal, window = True, w
    return q, k, v, causal, window


def fast_aten_scaled_dot_product_attention(
    query, key, value, attn_mask=None, dropout_p=0.0, is_causal=False, *, scale=None, enable_gqa=False
):
    """No-grad SDPA (aten_fast.py:9102-9211): fused kernels when eligible
    (including grouped K/V heads, f32, head_dim up to 256 and sliding-window
    masks from torch_mojo_backend.masks), otherwise the decomposition."""
    ex = fused_fa_ex_inputs(query, key, value, attn_mask, dropout_p, is_causal, scale, enable_gqa)
    if ex is not None:
        q, k, v, causal, window = ex
        out, _ = attention_forward(q, k, v, causal, window, scale)
        return out
    return sdpa_math(query, key, value, attn_mask, dropout_p, is_causal, scale, enable_gqa)


def rms_norm_inputs(x, normalized_shape, weight) -> bool:
    """Whether the fused RMSNorm kernel takes these inputs (metadata only)."""
    t = _t(x)
    if t is None or t._dtype not in (torch.float32, torch.bfloat16, torch.float16) or not normalized_shape:
        return False
    if tuple(t._shape[len(t._shape) - len(normalized_shape):]) != tuple(normalized_shape):
        return False
    n = math.prod(normalized_shape)
    if weight is not None:
        w = _t(weight)
        if w is None or w._numel != n or w._dtype not in (torch.float32, t._dtype):
            return False
    return n > 0


def rms_norm_forward(x: MT, normalized_shape, weight, eps, weight_offset=0.0):
    """(y, rstd [rows] f32) of rms_norm over the trailing `normalized_shape`
    dims (scale weight + weight_offset), or NOT_HANDLED."""
    n = math.prod(normalized_shape) if normalized_shape else 1
    if tuple(x._shape[len(x._shape) - len(normalized_shape):]) != tuple(normalized_shape) or n <= 0:
        return NOT_HANDLED
    if x._dtype not in (torch.float32, torch.bfloat16, torch.float16):
        return NOT_HANDLED
    w = None
    if weight is not None:
        w = _require(weight)
        if w._numel != n or w._dtype not in (torch.float32, x._dtype):
            return NOT_HANDLED
        w = _contig(w)
    xc = _contig(x)
    rows = xc._numel // n
    y = _alloc(x._shape, x._dtype, x._device)
    rstd = _alloc((rows,), torch.float32, x._device)
    check(
        "mi355x_rms_norm_fwd",
        lib().mi355x_rms_norm_fwd(y._ptr, rstd._ptr, xc._ptr, w._ptr if w is not None else None,
                                  _code(w._dtype) if w is not None else 0, float(weight_offset), rows, n,
                                  float(eps), _code(x._dtype), _STREAM),
    )
    return y, rstd


_EUNSUPPORTED = 3  # MI355X_EUNSUPPORTED


def rms_norm_backward(grad, x, normalized_shape, weight, rstd, weight_offset, need_x, need_w):
    """(dx, dweight) of rms_norm_forward in one kernel (mi355x_rms_norm_bwd),
    or NOT_HANDLED for inputs it does not take (a weight of another dtype
    than x, rows that are not 4-element multiples of at most 2048)."""
    n = math.prod(normalized_shape) if normalized_shape else 1
    g, xt = _require(grad), _require(x)
    w = _require(weight) if weight is not None else None
    if w is not None and w._dtype != xt._dtype:
        return NOT_HANDLED
    if n % 4 or n > 2048 or g._dtype != xt._dtype or tuple(g._shape) != tuple(xt._shape):
        return NOT_HANDLED
    gc, xc = _contig(g), _contig(xt)
    wc = _contig(w) if w is not None else None
    rows = xc._numel // n
    dx = _alloc(xt._shape, xt._dtype, xt._device)
    dw = _alloc(w._shape, w._dtype, w._device) if (w is not None and need_w) else None
    hold, wptr, ws = None, None, 0
    if dw is not None:
        ws = lib().mi355x_layer_norm_bwd_workspace_bytes(rows, n)
        hold, wptr = _workspace(ws, xt._device)
    rc = lib().mi355x_rms_norm_bwd(dx._ptr, dw._ptr if dw is not None else None, gc._ptr, xc._ptr, _require(rstd)._ptr,
                                   wc._ptr if wc is not None else None, float(weight_offset), rows, n,
                                   _code(xt._dtype), wptr, ws, _STREAM)
    if rc == _EUNSUPPORTED:
        return NOT_HANDLED
    check("mi355x_rms_norm_bwd", rc)
    return (dx if need_x else None), dw


def rope_forward(x: MT, cos: MT, sin: MT, inverse=False) -> MT:
    """Rotary embedding of x [B, H, T, D] with dense [T, D] tables; the output
    is allocated [B, T, H, D]-dense (as the attention kernels' inputs are) and
    returned as a [B, H, T, D] view."""
    b, h, t, d = x._shape
    if x._strides[3] != 1 or any(st % 4 for st in x._strides[:3]) or x._ptr % (4 * x._itemsize):
        x = materialize_contiguous(x)
    c = _contig(cos) if cos._dtype == x._dtype else materialize_contiguous(cos, x._dtype)
    sn = _contig(sin) if sin._dtype == x._dtype else materialize_contiguous(sin, x._dtype)
    out = alloc_bthd(b, h, t, d, x._dtype, x._device)
    strides = lambda v: _i64(v._strides[:3])  # noqa: E731
    check(
        "mi355x_rope",
        lib().mi355x_rope(out._ptr, strides(out), x._ptr, strides(x), c._ptr, sn._ptr, b, h, t, d, int(inverse),
                          _code(x._dtype), _STREAM),
    )
    return out


def geglu_forward(gate: MT, up: MT, approximate: str) -> MT:
    g, u = _contig(gate), _contig(up)
    out = _alloc(g._shape, g._dtype, g._device)
    check(
        "mi355x_geglu_fwd",
        lib().mi355x_geglu_fwd(out._ptr, g._ptr, u._ptr, g._numel, 1 if approximate == "tanh" else 0,
                               _code(g._dtype), _STREAM),
    )
    return out


def geglu_backward(grad: MT, gate: MT, up: MT, approximate: str):
    """(d_gate, d_up) of geglu_forward in one pass (mi355x_geglu_bwd)."""
    gr, g, u = _contig(_require(grad)), _contig(gate), _contig(up)
    dg = _alloc(g._shape, g._dtype, g._device)
    du = _alloc(g._shape, g._dtype, g._device)
    check(
        "mi355x_geglu_bwd",
        lib().mi355x_geglu_bwd(dg._ptr, du._ptr, gr._ptr, g._ptr, u._ptr, g._numel, 1 if approximate == "tanh" else 0,
                               _code(g._dtype), _STREAM),
    )
    return dg, du


# ---------------------------------------------------------------------------
# optimizer: fused AdamW and foreach (aten_fast.py:515-1162)
# ---------------------------------------------------------------------------
def _ptr_array(ptrs):
    arr = (ctypes.c_void_p * max(len(ptrs), 1))()
    for i, p in enumerate(ptrs):
        arr[i] = p
    return arr


def fast_aten__fused_adamw_(
    self, grads, exp_avgs, exp_avg_sqs, max_exp_avg_sqs, state_steps, *, lr, beta1, beta2,
    weight_decay, eps, amsgrad, maximize, grad_scale=None, found_inf=None,
):
    params = list(self)
    n = len(params)
    if not n:
        return None
    lists = [params, list(grads), list(exp_avgs), list(exp_avg_sqs), list(state_steps)]
    if any(len(x) != n for x in lists):
        raise RuntimeError("_fused_adamw_: all tensor lists must have the same length")
    if amsgrad and len(max_exp_avg_sqs) != n:
        raise RuntimeError("_fused_adamw_: max_exp_avg_sqs must match params when amsgrad=True")
    f32 = torch.float32
    P, G, M, V, S = ([_require(t) for t in lst] for lst in lists)
    # a gradient-clipping scale still pending on the gradients is applied as
    # they are read (they stay logically scaled; the multiply runs only if
    # something else reads them)
    gmul = _pending_scale(G)
    fields = []  # AdamWTensor records, flattened (seven 8-byte fields each)
    for i in range(n):
        p, g, m, v, s = P[i], G[i], M[i], V[i], S[i]
        pn = p._numel
        if not (p._dtype == f32 and g._dtype == f32 and m._dtype == f32 and v._dtype == f32
                and p._is_contiguous and g._is_contiguous and m._is_contiguous and v._is_contiguous):
            return NOT_HANDLED
        if g._numel != pn or m._numel != pn or v._numel != pn:
            name, t = next((nm, t) for nm, t in (("grad", g), ("exp_avg", m), ("exp_avg_sq", v)) if t._numel != pn)
            raise RuntimeError(f"_fused_adamw_: {name} {i} has {t._numel} elements, param has {pn}")
        if s._dtype != f32 or s._numel != 1:
            return NOT_HANDLED
        mx_ptr = 0
        if amsgrad:
            mx = _require(max_exp_avg_sqs[i])
            if mx._dtype != f32 or not mx._is_contiguous:
                return NOT_HANDLED
            if mx._numel != pn:
                raise RuntimeError(f"_fused_adamw_: max_exp_avg_sq {i} has {mx._numel} elements, param has {pn}")
            mx_ptr = mx._ptr
        fields += (p._ptr, g._ptr, m._ptr, v._ptr, mx_ptr, s._ptr, pn)
    assert ctypes.sizeof(AdamWTensor) == 7 * 8
    raw = (ctypes.c_uint64 * len(fields))(*fields)
    descs = (AdamWTensor * n).from_buffer(raw)
    lr_t = _t(lr)
    lr_value = 0.0 if lr_t is not None else float(lr)
    if lr_t is not None and lr_t._dtype != torch.float32:
        lr_t = materialize_contiguous(lr_t, torch.float32)
    flags = (1 if amsgrad else 0) | (2 if maximize else 0)
    gs = _t(grad_scale) if grad_scale is not None else None
    fi = _t(found_inf) if found_inf is not None else None
    if gs is not None and gs._dtype != torch.float32:
        gs = materialize_contiguous(gs, torch.float32)
    if fi is not None and fi._dtype != torch.float32:
        fi = materialize_contiguous(fi, torch.float32)
    # parameters the autocast forward casts get their 16-bit copy from this step
    low_dt = None
    lows = [None] * n
    take = []
    for i, prm in enumerate(params):
        dt = prm.__dict__.get(_CAST_DTYPE_ATTR) if hasattr(prm, "__dict__") else None
        if dt is not None and (low_dt is None or dt == low_dt):
            low_dt = dt
            take.append(i)
    if take:
        # the copies are slices of one allocation, each 256-byte aligned
        align = 256 // low_dt.itemsize
        offs, total = [], 0
        for i in take:
            offs.append(total)
            total += -(-P[i]._numel // align) * align
        buf = _alloc((total,), low_dt, P[take[0]]._device)
        for i, off in zip(take, offs):
            shp = P[i]._shape
            lows[i] = MT._view_of(buf, shp, row_major_strides(shp), off, True)
    low_ptrs = (ctypes.c_void_p * n)(*[x._ptr if x is not None else None for x in lows]) if low_dt else None
    check(
        "mi355x_fused_adamw_ex",
        lib().mi355x_fused_adamw_ex(
            descs, low_ptrs, _code(low_dt) if low_dt else 0, n, lr_value, lr_t._ptr if lr_t is not None else None,
            float(beta1), float(beta2), float(weight_decay), float(eps), flags,
            gs._ptr if gs is not None else None, fi._ptr if fi is not None else None,
            gmul._ptr if gmul is not None else None, _STREAM,
        ),
    )
    if fi is not None:
        # a skipped step (found_inf) leaves the copies unwritten: do not publish them
        lows = [None] * n
    for prm, low in zip(params, lows):
        if low is not None:
            _set_param_copy(prm, low)
    return None


def _foreach_ok(tensors, dtype=None):
    ts = [_t(x) for x in tensors]
    if any(t is None or not t._is_contiguous for t in ts):
        return None
    dt = dtype or ts[0]._dtype
    if any(t._dtype != dt for t in ts) or dt not in (torch.float32, torch.bfloat16, torch.float16):
        return None
    return ts


def foreach_apply(opname, a_list, b_list=None, c_list=None, scalars=None, s0=0.0, tensor_scalar=None):
    a = _foreach_ok(a_list)
    if a is None:
        return NOT_HANDLED
    dt = a[0]._dtype
    b = c = None
    if b_list is not None:
        b = _foreach_ok(b_list, dt)
        if b is None or any(x._numel != y._numel for x, y in zip(a, b)):
            return NOT_HANDLED
    if c_list is not None:
        c = _foreach_ok(c_list, dt)
        if c is None or any(x._numel != y._numel for x, y in zip(a, c)):
            return NOT_HANDLED
    n = len(a)
    if n == 0:
        return None
    opcode = {"add": 0, "mul": 2, "div": 3, "lerp": 43, "addcmul": 41, "addcdiv": 42, "sqrt": 65}[opname]
    sc = None
    if scalars is not None:
        sc = (ctypes.c_double * n)(*[float(_scalar_value(x)) for x in scalars])
    ts = None
    if tensor_scalar is not None:
        ts = _t(tensor_scalar)
        if ts is None:
            return NOT_HANDLED
        if ts._dtype != torch.float32:
            ts = materialize_contiguous(ts, torch.float32)
    check(
        "mi355x_foreach_apply",
        lib().mi355x_foreach_apply(
            opcode, _ptr_array([x._ptr for x in a]),
            _ptr_array([x._ptr for x in b]) if b is not None else None,
            _ptr_array([x._ptr for x in c]) if c is not None else None,
            sc, _i64([x._numel for x in a]), n, _code(dt), float(s0),
            ts._ptr if ts is not None else None, _STREAM,
        ),
    )
    return None


def _storage_ref(t: MT):
    """A callable returning a tensor with t's layout over t's storage while
    that storage lives (None after): a weak reference that survives the
    death of t's own wrapper when views of the storage remain."""
    import weakref

    href = weakref.ref(t._holder)
    meta = (t._ptr, tuple(t._shape), tuple(t._strides), t._offset, t._dtype, t._device, t._is_contiguous)

    def get():
        h = href()
        if h is None:
            return None
        ptr, shape, strides, offset, dtype, device, contig = meta
        return MT._make(h, ptr, shape, strides, offset, dtype, device, contig)

    return get


def foreach_mul_deferred(a_list, tensor_scalar):
    """_foreach_mul_(tensors, scalar tensor) held as pending work (see
    `lazy_scale`) when every tensor is contiguous f32 and the scalar an f32
    device scalar: gradient clipping's scale, which the fused AdamW step that
    follows applies as it reads the gradients, so the gradients need no pass
    of their own.  NOT_HANDLED otherwise."""
    if not _LAZY_GRAD_SCALE:
        return NOT_HANDLED
    a = _foreach_ok(a_list, torch.float32)
    ts = _t(tensor_scalar)
    if a is None or not a or ts is None or ts._dtype != torch.float32 or ts._numel != 1:
        return NOT_HANDLED
    refs = [_storage_ref(t) for t in a]

    def run(refs=refs, ts=ts):
        alive = [t for t in (r() for r in refs) if t is not None]
        if alive:
            foreach_apply("mul", alive, tensor_scalar=ts)

    lazy_scale(a, ts, run, consumers={torch.ops.aten._fused_adamw_.default: {1},
                                      torch.ops.aten._fused_adamw_.tensor_lr: {1}})
    return None


def fast_aten__foreach_norm(self, ord=2, dtype=None):
    ts = _foreach_ok(self)
    if ts is None or ord not in (1, 2, math.inf, float("inf")):
        return NOT_HANDLED
    n = len(ts)
    out_dtype = dtype or ts[0]._dtype
    if n == 0:
        return []
    # one buffer, one 0-d view per tensor: the stack of the norms that
    # clip_grad_norm_ takes next is then a view of it
    buf = _alloc((n,), out_dtype, ts[0]._device)
    _mark_cat_ready(buf)
    outs = [MT._view_of(buf, (), (), i, True) for i in range(n)]
    numels = _i64([t._numel for t in ts])
    ws = lib().mi355x_foreach_norm_workspace_bytes(numels, n)
    hold, wptr = _workspace(ws, ts[0]._device)
    check(
        "mi355x_foreach_norm",
        lib().mi355x_foreach_norm(
            _ptr_array([o._ptr for o in outs]), _code(out_dtype), _ptr_array([t._ptr for t in ts]),
            _code(ts[0]._dtype), numels, n, float(ord), wptr, ws, _STREAM,
        ),
    )
    return outs


# ---------------------------------------------------------------------------
# fused cross-entropy (the log_softmax + nll_loss chain, aten_fast.py:5792-6130)
# ---------------------------------------------------------------------------
_REDUCTION = {0: 0, 1: 1, 2: 2}


def fused_cross_entropy_inputs(input, target, weight, reduction, ignore_index, label_smoothing):
    """(logits, target) when the fused kernels serve the call, else None."""
    x, t = _t(input), _t(target)
    if (
        x is None or t is None or weight is not None or float(label_smoothing) != 0.0
        or reduction not in _REDUCTION or x._dtype not in _FLOAT_DTYPES
        or len(x._shape) != 2 or t._dtype != torch.int64 or len(t._shape) != 1
        or t._shape[0] != x._shape[0] or x._strides[1] != 1 or x._shape[1] == 0
    ):
        return None
    return x, t


def fused_cross_entropy_forward(x: MT, t: MT, reduction, ignore_index):
    """(loss f32, lse f32 [n], total_weight f32 scalar)."""
    n, c = x._shape
    ld = x._strides[0] if n > 1 else c
    tgt = _contig(t)
    out = _alloc((n,) if reduction == 0 else (), torch.float32, x._device)
    lse = _alloc((n,), torch.float32, x._device)
    total = _alloc((), torch.float32, x._device)
    ws = lib().mi355x_cross_entropy_workspace_bytes(n)
    hold, wptr = _workspace(ws, x._device)
    eptr = _error_slot(x._device, _TARGET_ERROR)
    check(
        "mi355x_cross_entropy_fwd",
        lib().mi355x_cross_entropy_fwd(out._ptr, total._ptr, lse._ptr, x._ptr, _code(x._dtype), ld,
                                       tgt._ptr, n, c, int(reduction), int(ignore_index), eptr, wptr,
                                       ws, _STREAM),
    )
    return out, lse, total


def fused_cross_entropy_forward_deferred(x: MT, t: MT, reduction, ignore_index):
    """fused_cross_entropy_forward left lazy: (loss, lse, total) are filled by
    the backward's single pass over the logits (mi355x_cross_entropy_fwd_bwd),
    or by the forward kernels if anything reads them first.  None when that
    pass does not take the shape (the caller runs the forward now)."""
    import weakref

    from . import _run, is_pending, lazy_outputs

    global _last_ce_rec
    prev = _last_ce_rec() if _last_ce_rec is not None else None
    if prev is not None and is_pending(prev):
        _run(prev)  # at most one deferred forward (each holds its logits)
    n, c = x._shape
    ld = x._strides[0] if n > 1 else c
    es = x._itemsize
    v = 16 // es
    if (not _LAZY_CE or reduction not in (1, 2) or n == 0 or x._dtype not in _FLOAT_DTYPES
            or max((c + 2 * v - 2) // v, ((c + 7) // 8 * 8) // v) > 32 * 256):
        return None
    tgt = _contig(t)
    out = _alloc((), torch.float32, x._device)
    lse = _alloc((n,), torch.float32, x._device)
    total = _alloc((), torch.float32, x._device)
    ptrs = (out._ptr, total._ptr, lse._ptr)

    def forward(x=x, tgt=tgt):
        o, tw, l_ = ptrs
        ws = lib().mi355x_cross_entropy_workspace_bytes(n)
        hold, wptr = _workspace(ws, x._device)
        check("mi355x_cross_entropy_fwd", lib().mi355x_cross_entropy_fwd(
            o, tw, l_, x._ptr, _code(x._dtype), ld, tgt._ptr, n, c, int(reduction), int(ignore_index),
            _error_slot(x._device, _TARGET_ERROR), wptr, ws, _STREAM))

    out_ref = weakref.ref(out._holder)

    def both(dx: MT, ld_dx, g: MT, x=x, tgt=tgt):
        o, tw, l_ = ptrs
        hold_o = None
        if out_ref() is None:  # the loss tensor is gone: its value goes to scratch
            hold_o = _alloc((), torch.float32, x._device)
            o = hold_o._ptr
        ws = lib().mi355x_cross_entropy_workspace_bytes(n)
        hold, wptr = _workspace(ws, x._device)
        return lib().mi355x_cross_entropy_fwd_bwd(
            o, tw, l_, dx._ptr, ld_dx, x._ptr, _code(x._dtype), ld, tgt._ptr, g._ptr, n, c, int(reduction),
            int(ignore_index), _error_slot(x._device, _TARGET_ERROR), wptr, ws, _STREAM)

    rec = lazy_outputs((out, lse, total), (x, tgt), forward, fused=both)
    _last_ce_rec = weakref.ref(rec)
    return out, lse, total


_last_ce_rec = None  # weak reference to the last deferred cross-entropy forward


def fused_cross_entropy_backward(grad, x: MT, t: MT, lse: MT, total: MT, reduction, ignore_index):
    """dlogits in x's dtype, stored with rows padded to a multiple of 8
    elements (16-byte aligned rows for the lm_head GEMMs that consume it).
    When the forward is still pending (fused_cross_entropy_forward_deferred),
    one pass computes the loss, lse and dlogits together."""
    from . import lazy_record, materialize, retire

    n, c = x._shape
    ld = x._strides[0] if n > 1 else c
    g = _require(grad)
    g = _contig(g) if g._dtype == torch.float32 else materialize_contiguous(g, torch.float32)
    ld_dx = (c + 7) // 8 * 8
    dense = _alloc((n, ld_dx), x._dtype, x._device)
    dx = MT._view_of(dense, (n, c), (ld_dx, 1), 0, ld_dx == c)
    rec = lazy_record(lse)
    if rec is not None and rec.fused is not None and g._numel == 1:
        rc = rec.fused(dense, ld_dx, g)
        if rc == 0:
            retire(rec)
            return dx
        if rc != 3:  # anything but MI355X_EUNSUPPORTED (a shape it does not take) is an error
            check("mi355x_cross_entropy_fwd_bwd", rc)
    materialize(lse)
    check(
        "mi355x_cross_entropy_bwd",
        lib().mi355x_cross_entropy_bwd(dx._ptr, _code(x._dtype), ld_dx, x._ptr, _code(x._dtype), ld,
                                       lse._ptr, _contig(t)._ptr, g._ptr, int(reduction), total._ptr,
                                       n, c, int(ignore_index), _STREAM),
    )
    return dx
