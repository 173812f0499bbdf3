"""Loader for the gfx950 kernel library (`libmi355x_kernels.so`).

The reference builds one CPython extension per (op, dtype) variant with the
Mojo compiler and caches it (torch_mojo_backend/eager_kernels/__init__.py:
409-418, 463-510).  Here every kernel is compiled ahead of time by hipcc into
one shared library with a C ABI (`include/mi355x_kernels.h`), so there is no
JIT, no variant cache and no background build pool: loading is a single
`ctypes.CDLL`.

`lib()` returns the loaded library with argtypes/restype set for every
exported function.  A missing or stale library raises `KernelLibraryError`
with the build command: there is no fallback path.
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

LIB_NAME = "libmi355x_kernels.so"
LIB_PATH = Path(__file__).resolve().parent / LIB_NAME
ABI_VERSION = 6

c_int = ctypes.c_int
c_i64 = ctypes.c_int64
c_double = ctypes.c_double
c_vp = ctypes.c_void_p
c_char_p = ctypes.c_char_p
P_i64 = ctypes.POINTER(ctypes.c_int64)
P_int = ctypes.POINTER(ctypes.c_int)
P_vp = ctypes.POINTER(ctypes.c_void_p)
P_double = ctypes.POINTER(ctypes.c_double)


class AdamWTensor(ctypes.Structure):
    """`mi355x_adamw_tensor` (layout of include/mi355x_kernels.h)."""

    _fields_ = [
        ("param", c_vp),
        ("grad", c_vp),
        ("exp_avg", c_vp),
        ("exp_avg_sq", c_vp),
        ("max_exp_avg_sq", c_vp),
        ("step", c_vp),
        ("numel", c_i64),
    ]


# name -> (restype, argtypes).  Kept in the order of the header.
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "mi355x_abi_version": (c_int, []),
    "mi355x_last_error": (c_char_p, []),
    "mi355x_target": (c_char_p, []),
    "mi355x_source_hash": (c_char_p, []),
    "mi355x_copy": (c_int, [c_vp, c_int, P_i64, c_vp, c_int, P_i64, P_i64, c_int, c_vp]),
    "mi355x_fill": (c_int, [c_vp, c_int, P_i64, P_i64, c_int, c_double, c_vp]),
    "mi355x_arange": (c_int, [c_vp, c_int, c_i64, c_double, c_double, c_vp]),
    "mi355x_map": (
        c_int,
        [c_int, c_vp, c_int, c_int, P_vp, P_int, P_i64, P_i64, c_int, c_double, c_double, c_vp],
    ),
    "mi355x_reduce_workspace_bytes": (c_i64, [c_i64, c_i64, c_i64]),
    "mi355x_reduce": (
        c_int,
        [c_int, c_vp, c_int, c_vp, c_int, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_vp, c_i64, c_vp],
    ),
    "mi355x_argreduce": (
        c_int,
        [c_int, c_vp, c_vp, c_vp, c_int, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_vp],
    ),
    "mi355x_index_select": (
        c_int,
        [c_vp, c_vp, c_int, c_vp, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_vp, c_vp],
    ),
    "mi355x_embedding_fwd": (
        c_int,
        [c_vp, c_vp, c_int, c_vp, c_i64, c_i64, c_i64, c_i64, c_vp, c_vp],
    ),
    "mi355x_embedding_bwd_workspace_bytes": (c_i64, [c_i64, c_i64]),
    "mi355x_embedding_bwd": (
        c_int,
        [c_vp, c_vp, c_int, c_vp, c_i64, c_i64, c_i64, c_i64, c_vp, c_i64, c_vp],
    ),
    "mi355x_embedding_bwd_accumulate": (
        c_int,
        [c_vp, c_vp, c_vp, c_int, c_vp, c_i64, c_i64, c_i64, c_i64, c_vp, c_i64, c_vp],
    ),
    "mi355x_layer_norm_fwd": (
        c_int,
        [c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_i64, c_i64, c_double, c_int, c_vp],
    ),
    "mi355x_layer_norm_fwd_ex": (
        c_int,
        [c_vp, c_vp, c_int, c_vp, c_vp, c_vp, c_vp, c_vp, c_i64, c_i64, c_double, c_int, c_vp],
    ),
    "mi355x_add_cast": (c_int, [c_vp, c_vp, c_int, c_vp, c_vp, c_int, c_i64, c_vp]),
    "mi355x_layer_norm_fwd_add": (
        c_int,
        [c_vp, c_vp, c_int, c_vp, c_vp, c_vp, c_vp, c_vp, c_int, c_vp, c_vp, c_i64, c_i64, c_double, c_int, c_vp],
    ),
    "mi355x_layer_norm_apply": (c_int, [c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_i64, c_i64, c_int, c_vp]),
    "mi355x_layer_norm_bwd_workspace_bytes": (c_i64, [c_i64, c_i64]),
    "mi355x_layer_norm_bwd": (
        c_int,
        [c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_i64, c_i64, c_int, c_vp, c_i64, c_vp],
    ),
    "mi355x_gelu_fwd": (c_int, [c_vp, c_vp, c_i64, c_int, c_int, c_vp]),
    "mi355x_gelu_bwd": (c_int, [c_vp, c_vp, c_vp, c_i64, c_int, c_int, c_vp]),
    "mi355x_softmax_fwd": (c_int, [c_vp, c_int, c_vp, c_int, c_i64, c_i64, c_int, c_vp]),
    "mi355x_softmax_bwd": (
        c_int,
        [c_vp, c_int, c_vp, c_int, c_vp, c_int, c_i64, c_i64, c_int, c_vp],
    ),
    "mi355x_nll_workspace_bytes": (c_i64, [c_i64]),
    "mi355x_nll_fwd": (
        c_int,
        [c_vp, c_vp, c_vp, c_int, c_vp, c_vp, c_i64, c_i64, c_int, c_i64, c_vp, c_vp, c_i64, c_vp],
    ),
    "mi355x_nll_bwd": (
        c_int,
        [c_vp, c_vp, c_vp, c_vp, c_vp, c_i64, c_i64, c_int, c_i64, c_int, c_vp],
    ),
    "mi355x_cross_entropy_workspace_bytes": (c_i64, [c_i64]),
    "mi355x_cross_entropy_fwd": (
        c_int,
        [c_vp, c_vp, c_vp, c_vp, c_int, c_i64, c_vp, c_i64, c_i64, c_int, c_i64, c_vp, c_vp, c_i64, c_vp],
    ),
    "mi355x_cross_entropy_bwd": (
        c_int,
        [c_vp, c_int, c_i64, c_vp, c_int, c_i64, c_vp, c_vp, c_vp, c_int, c_vp, c_i64, c_i64, c_i64, c_vp],
    ),
    "mi355x_cross_entropy_fwd_bwd": (
        c_int,
        [c_vp, c_vp, c_vp, c_vp, c_i64, c_vp, c_int, c_i64, c_vp, c_vp, c_i64, c_i64, c_int, c_i64, c_vp, c_vp,
         c_i64, c_vp],
    ),
    "mi355x_fused_adamw": (
        c_int,
        [
            ctypes.POINTER(AdamWTensor), c_int, c_double, c_vp, c_double, c_double,
            c_double, c_double, c_int, c_vp, c_vp, c_vp,
        ],
    ),
    "mi355x_fused_adamw_ex": (
        c_int,
        [
            ctypes.POINTER(AdamWTensor), c_vp, c_int, c_int, c_double, c_vp, c_double, c_double,
            c_double, c_double, c_int, c_vp, c_vp, c_vp, c_vp,
        ],
    ),
    "mi355x_foreach_norm_workspace_bytes": (c_i64, [P_i64, c_int]),
    "mi355x_foreach_norm": (
        c_int,
        [P_vp, c_int, P_vp, c_int, P_i64, c_int, c_double, c_vp, c_i64, c_vp],
    ),
    "mi355x_foreach_apply": (
        c_int,
        [c_int, P_vp, P_vp, P_vp, P_double, P_i64, c_int, c_int, c_double, c_vp, c_vp],
    ),
    "mi355x_gemm_workspace_bytes": (
        c_i64, [c_vp, c_i64, c_i64, c_i64, c_vp, c_i64, c_i64, c_i64, c_int, c_i64, c_i64, c_i64, c_i64],
    ),
    "mi355x_gemm": (
        c_int,
        [
            c_vp, c_int, c_i64, c_i64,
            c_vp, c_i64, c_i64, c_i64,
            c_vp, c_i64, c_i64, c_i64,
            c_int, c_vp, c_int, c_int,
            c_i64, c_i64, c_i64, c_i64,
            c_vp, c_i64, c_vp,
        ],
    ),
    "mi355x_gemm_ex": (
        c_int,
        [
            c_vp, c_int, c_i64, c_i64,
            c_vp, c_i64, c_i64, c_i64,
            c_vp, c_i64, c_i64, c_i64,
            c_int, c_vp, c_int, c_int, c_vp, c_int,
            c_i64, c_i64, c_i64, c_i64,
            c_vp, c_i64, c_vp,
        ],
    ),
    "mi355x_attn_fwd": (
        c_int,
        [
            c_vp, P_i64, c_vp, c_vp, P_i64, c_vp, P_i64, c_vp, P_i64,
            c_i64, c_i64, c_i64, c_i64, c_i64, c_double, c_int, c_int, c_vp,
        ],
    ),
    "mi355x_rms_norm_fwd": (c_int, [c_vp, c_vp, c_vp, c_vp, c_int, c_double, c_i64, c_i64, c_double, c_int, c_vp]),
    "mi355x_rms_norm_bwd": (
        c_int,
        [c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_double, c_i64, c_i64, c_int, c_vp, c_i64, c_vp],
    ),
    "mi355x_rope": (c_int, [c_vp, P_i64, c_vp, P_i64, c_vp, c_vp, c_i64, c_i64, c_i64, c_i64, c_int, c_int, c_vp]),
    "mi355x_geglu_fwd": (c_int, [c_vp, c_vp, c_vp, c_i64, c_int, c_int, c_vp]),
    "mi355x_geglu_bwd": (c_int, [c_vp, c_vp, c_vp, c_vp, c_vp, c_i64, c_int, c_int, c_vp]),
    "mi355x_attn_fwd_ex": (
        c_int,
        [
            c_vp, P_i64, c_vp, c_vp, P_i64, c_vp, P_i64, c_vp, P_i64,
            c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_double, c_int, c_i64, c_int, c_vp,
        ],
    ),
    "mi355x_attn_bwd_workspace_bytes": (c_i64, [c_i64, c_i64, c_i64, c_i64, c_i64]),
    "mi355x_attn_bwd": (
        c_int,
        [
            c_vp, P_i64, c_vp, P_i64, c_vp, P_i64, c_vp, P_i64,
            c_vp, P_i64, c_vp, P_i64, c_vp, P_i64, c_vp, P_i64, c_vp,
            c_i64, c_i64, c_i64, c_i64, c_i64, c_double, c_int, c_int,
            c_vp, c_i64, c_vp,
        ],
    ),
    "mi355x_attn_fwd_gen": (
        c_int,
        [
            c_vp, P_i64, c_vp, c_vp, P_i64, c_vp, P_i64, c_vp, P_i64,
            c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_double, c_int, c_i64, c_int, c_vp,
        ],
    ),
    "mi355x_attn_bwd_gen_workspace_bytes": (c_i64, [c_i64, c_i64, c_i64, c_i64, c_i64, c_i64]),
    "mi355x_attn_bwd_gen": (
        c_int,
        [
            c_vp, P_i64, c_vp, P_i64, c_vp, P_i64, c_vp, P_i64,
            c_vp, P_i64, c_vp, P_i64, c_vp, P_i64, c_vp, P_i64, c_vp,
            c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_double, c_int, c_i64, c_int,
            c_vp, c_i64, c_vp,
        ],
    ),
    "mi355x_attn_bwd_noalloc": (
        c_int,
        [
            c_vp, P_i64, c_vp, P_i64, c_vp, P_i64, c_vp, P_i64,
            c_vp, P_i64, c_vp, P_i64, c_vp, P_i64, c_vp, P_i64, c_vp,
            c_i64, c_i64, c_i64, c_i64, c_i64, c_double, c_int, c_int,
            c_vp,
        ],
    ),
}


class KernelLibraryError(RuntimeError):
    """The gfx950 kernel library is missing, stale or reported an error."""


class KernelCallError(RuntimeError):
    """A library call returned a nonzero status."""

    def __init__(self, name: str, code: int, message: str):
        super().__init__(f"{name} failed (status {code}): {message}")
        self.code = code


_LIB = None


def _load() -> ctypes.CDLL:
    path = Path(os.environ.get("MI355X_KERNELS_LIB", LIB_PATH))
    if not path.exists():
        raise KernelLibraryError(
            f"{path} is missing: build it with `python torch-mojo-backend_amd/build.py`"
            " (or __graft_entry__.build())"
        )
    lib = ctypes.CDLL(str(path))
    for name, (restype, argtypes) in SIGNATURES.items():
        try:
            fn = getattr(lib, name)
        except AttributeError as exc:
            raise KernelLibraryError(f"{path} does not export {name}: rebuild it") from exc
        fn.restype = restype
        fn.argtypes = argtypes
    version = lib.mi355x_abi_version()
    if version != ABI_VERSION:
        raise KernelLibraryError(f"{path} has ABI {version}, expected {ABI_VERSION}: rebuild it")
    built = lib.mi355x_source_hash().decode()
    # an explicitly named library (MI355X_KERNELS_LIB) is the caller's choice
    expected = None if "MI355X_KERNELS_LIB" in os.environ else _expected_source_hash()
    if expected is not None and built != expected:
        raise KernelLibraryError(
            f"{path} was built from other sources (digest {built}, sources {expected}): rebuild it with"
            " `python torch-mojo-backend_amd/build.py`"
        )
    return lib


def _expected_source_hash():
    """Digest of csrc/ + include/ beside the package (None when absent)."""
    from .._srchash import source_hash

    import importlib.util

    spec = importlib.util.spec_from_file_location("_mi355x_build_flags", Path(__file__).resolve().parents[2] / "build.py")
    if spec is None or not Path(spec.origin).exists():
        return None
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return source_hash(mod._hash_flags())


class Deferred:
    """A kernel launch held back so that the next kernel can absorb it (the
    residual add that the following LayerNorm reads): `out` is the result
    tensor it will write, `inputs` what it reads, `launch()` issues it."""

    __slots__ = ("out", "inputs", "launch")

    def __init__(self, out, inputs, launch):
        self.out, self.inputs, self.launch = out, inputs, launch


_pending: list = []
_pending_lock = threading.RLock()
_state = threading.local()  # .flushing: this thread is issuing deferred launches


def defer(record: Deferred) -> None:
    """Queue a launch; it runs before the next library call, host read or
    synchronize, in the order deferred."""
    with _pending_lock:
        _pending.append(record)


def _reads_storage_of(rec: Deferred, ref) -> bool:
    return any(inp._holder is ref._holder for inp in rec.inputs)


def take_pending(match):
    """Remove and return the first pending launch for which match(record)
    holds (the caller then performs its work itself), else None.

    The caller issues the taken work after the launches still pending
    (its next library call flushes them first), so a record is taken only
    when no later pending launch reads the storage it writes; otherwise the
    later launch would read that output before it exists, and None is
    returned (the caller's library call then issues everything in order)."""
    if not _pending:
        return None
    with _pending_lock:
        for i, rec in enumerate(_pending):
            if match(rec):
                if any(_reads_storage_of(later, rec.out) for later in _pending[i + 1:]):
                    return None
                return _pending.pop(i)
    return None


def flush_pending() -> None:
    """Issue every deferred launch, oldest first.  A launch issued from
    here calls lib() itself, which must not re-enter the flush; other
    threads wait on the lock until the flush has finished."""
    if not _pending or getattr(_state, "flushing", False):
        return
    with _pending_lock:
        _state.flushing = True
        try:
            while _pending:
                _pending.pop(0).launch()
        finally:
            _state.flushing = False


class Lazy:
    """Work on some storages that has not run yet: `launch()` runs it, `inputs`
    are the tensors it reads, `refs` maps the id of each storage holder it
    writes to a weak reference (the record never keeps a storage alive).
    Two kinds: an output the kernel has not filled (the layer norm's f32
    output under autocast), and an in-place scale not yet applied (the
    gradient-clipping `_foreach_mul_`), whose `scale` is the scalar tensor
    and which a fused optimizer step can apply on the fly.  `consumers` maps
    an op to the argument position through which that op takes the record
    over itself: a set of positions (it neither needs nor triggers the
    launch there); `accumulate(dst, base)`, when set, writes base + the
    output into dst without materializing the output (a tied embedding's
    gradient; dst may be base)."""

    __slots__ = ("refs", "inputs", "launch", "scale", "consumers", "accumulate", "fused", "__weakref__")

    def __init__(self, inputs, launch, scale=None, consumers=None, accumulate=None, fused=None):
        self.refs, self.inputs, self.launch, self.scale = {}, tuple(inputs), launch, scale
        self.consumers, self.accumulate, self.fused = consumers or {}, accumulate, fused


_lazy: dict = {}  # id(storage holder) -> Lazy, while the holder lives
_lazy_records: dict = {}  # id(Lazy) -> Lazy, the records with a live holder


def _register(rec: Lazy, tensors) -> None:
    import weakref

    def gone(ref, key, rec=rec):
        if _pending_lock is None:  # interpreter shutdown: module globals are gone
            return
        with _pending_lock:
            if rec.refs.get(key) is ref:
                del rec.refs[key]
                if _lazy.get(key) is rec:
                    del _lazy[key]
            if not rec.refs:
                _lazy_records.pop(id(rec), None)

    with _pending_lock:
        for t in tensors:
            key = id(t._holder)
            old = _lazy.get(key)
            if old is not None and old is not rec:
                _run(old)  # an earlier record on the same storage goes first
            rec.refs[key] = weakref.ref(t._holder, lambda ref, key=key: gone(ref, key))
            _lazy[key] = rec
        _lazy_records[id(rec)] = rec


def _run(rec: Lazy) -> None:
    with _pending_lock:
        for key in rec.refs:
            if _lazy.get(key) is rec:
                del _lazy[key]
        _lazy_records.pop(id(rec), None)
        if any(r() is not None for r in rec.refs.values()):
            rec.launch()


def lazy(out, inputs, launch, consumers=None, accumulate=None) -> None:
    """Register `out` (a fresh tensor) as filled by `launch` when first
    touched: `materialize_touched` runs it before any op that reads or writes
    out's storage, or that writes the storage of one of `inputs`; if out's
    storage dies first, the launch never runs (the allocator may reuse the
    memory then, so the record holds the storage only weakly)."""
    _register(Lazy(inputs, launch, consumers=consumers, accumulate=accumulate), (out,))


def lazy_outputs(outs, inputs, launch, fused=None) -> Lazy:
    """`lazy` for several outputs of one launch (all filled together).
    `fused` is the caller's own alternative (see `retire`)."""
    rec = Lazy(inputs, launch, fused=fused)
    _register(rec, outs)
    return rec


def retire(rec: Lazy) -> None:
    """Drop a record whose outputs were filled by other means (a launch that
    computes them along with more): it will not run."""
    with _pending_lock:
        for key in rec.refs:
            if _lazy.get(key) is rec:
                del _lazy[key]
        _lazy_records.pop(id(rec), None)


def is_pending(rec: Lazy) -> bool:
    return _lazy_records.get(id(rec)) is rec


def lazy_scale(tensors, scale, launch, consumers=None) -> None:
    """Register the in-place multiplication of every tensor in `tensors` by
    the device scalar `scale` as pending: it runs (all of it, by `launch`)
    before any op touches one of those storages or writes `scale`, except a
    fused optimizer step that applies it itself (`pending_scale`)."""
    _register(Lazy((scale,), launch, scale, consumers), tensors)


def lazy_record(t):
    """The pending record on t's storage, or None."""
    return _lazy.get(id(t._holder)) if _lazy and getattr(t, "_holder", None) is not None else None


def pending_scale(tensors):
    """The scalar of the one pending scale covering every tensor in
    `tensors`, else None (after running any pending work on them, so the
    caller then reads plain values)."""
    if not _lazy:
        return None
    with _pending_lock:
        recs = {id(_lazy.get(id(t._holder))): _lazy.get(id(t._holder)) for t in tensors}
        if len(recs) == 1:
            rec = next(iter(recs.values()))
            if rec is not None and rec.scale is not None:
                return rec.scale
    materialize_touched(tuple(tensors), None, False)
    return None


def lazy_live() -> bool:
    return bool(_lazy)


def _holders_of(args, kwargs) -> dict:
    """id(storage holder) -> the argument positions (kwargs: -1) holding it."""
    found: dict = {}

    def add(v, pos):
        h = getattr(v, "_holder", None)
        if h is not None:
            found.setdefault(id(h), set()).add(pos)

    for pos, v in enumerate(args):
        if isinstance(v, (list, tuple)):
            for e in v:
                add(e, pos)
        else:
            add(v, pos)
    if kwargs:
        for v in kwargs.values():
            if isinstance(v, (list, tuple)):
                for e in v:
                    add(e, -1)
            else:
                add(v, -1)
    return found


def materialize_touched(args, kwargs, writes: bool, func=None) -> None:
    """Run the lazy work that an op with these arguments depends on: records
    writing a storage it touches, and, when the op writes (`writes`), records
    reading a storage it touches (they must run before it changes).  A record
    that lists `func` as a consumer at the only position where it is touched
    is left to the op."""
    if not _lazy:
        return
    # fast exit (most ops): no argument storage is pending, and the op writes
    # nothing a record reads
    ids = set()
    for v in args:
        if isinstance(v, (list, tuple)):
            for e in v:
                h = getattr(e, "_holder", None)
                if h is not None:
                    ids.add(id(h))
        else:
            h = getattr(v, "_holder", None)
            if h is not None:
                ids.add(id(h))
    if kwargs:
        ids.update(_holders_of((), kwargs))
    if not ids:
        return
    if ids.isdisjoint(_lazy.keys()) and not (
            writes and any(id(t._holder) in ids for rec in list(_lazy_records.values()) for t in rec.inputs)):
        return
    hs = _holders_of(args, kwargs)
    with _pending_lock:
        due = {}
        for key, where in hs.items():
            rec = _lazy.get(key)
            if rec is not None:
                ok = rec.consumers.get(func) if func is not None else None
                if ok is not None and where <= ok:
                    continue
                due[id(rec)] = rec
        if writes:
            for rec in list(_lazy_records.values()):
                if any(id(t._holder) in hs for t in rec.inputs):
                    due[id(rec)] = rec
        for rec in due.values():
            if _lazy_records.get(id(rec)) is rec:
                _run(rec)


def materialize(t) -> None:
    """Run the lazy work on t's storage, if any is pending."""
    if _lazy:
        materialize_touched((t,), None, False)


def lib() -> ctypes.CDLL:
    """The loaded kernel library (loaded on first use).  Deferred launches
    are issued first, so every kernel sees them in stream order."""
    global _LIB
    if _pending:
        flush_pending()
    if _LIB is None:
        _LIB = _load()
    return _LIB


def set_library_for_tests(replacement) -> object:
    """Swap the library object (host-only tests); returns the previous one."""
    global _LIB
    previous = _LIB
    _LIB = replacement
    return previous


def last_error() -> str:
    msg = lib().mi355x_last_error()
    return msg.decode() if isinstance(msg, bytes) else str(msg)


def check(name: str, status: int) -> None:
    """Raise KernelCallError when a library call returned nonzero."""
    if status:
        raise KernelCallError(name, status, last_error())
