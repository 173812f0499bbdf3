"""`torch.mojo`: the backend module of the eager mojo device.

Mirrors the reference's device module (torch_mojo_backend/mojo_device/
torch_mojo_device_module.py): device count/current/set, `synchronize`, the
Philox-style (seed, counter) RNG state as a 16-byte uint8 tensor, and the
AMP dtype list.  `mojo:N` is the N-th ROCm GPU; synchronising waits for the
device's stream (there is no launch queue to drain: kernels are built ahead
of time and issued directly).
"""

from __future__ import annotations

import struct
import threading

import torch

from . import torch_mojo_tensor as _tensor_mod

_current_device = 0


def _is_in_bad_fork():
    return False


def device_count() -> int:
    if _tensor_mod.storage_kind() != "cuda":
        return 1
    return torch.cuda.device_count()


def is_available() -> bool:
    return device_count() > 0


def is_initialized() -> bool:
    return True


def _lazy_init() -> None:
    return None


def current_device() -> int:
    return _current_device


def set_device(device_idx) -> None:
    global _current_device
    if isinstance(device_idx, torch.device):
        device_idx = device_idx.index or 0
    if device_idx < 0 or device_idx >= device_count():
        raise ValueError(f"Invalid device index {device_idx}")
    _current_device = device_idx
    if _tensor_mod.storage_kind() == "cuda":
        torch.cuda.set_device(device_idx)


class device:
    """Context manager swapping the current mojo device (torch.cuda.device's
    counterpart; torch.serialization needs it for map_location="mojo")."""

    def __init__(self, device) -> None:
        if device is None:
            self.idx = -1
        elif isinstance(device, int):
            self.idx = device
        else:
            d = torch.device(device)
            self.idx = -1 if d.index is None else d.index

    def __enter__(self) -> None:
        self.prev_idx = _current_device
        if self.idx >= 0 and self.idx != _current_device:
            set_device(self.idx)

    def __exit__(self, *exc_info) -> bool:
        if self.idx >= 0 and self.prev_idx != _current_device:
            set_device(self.prev_idx)
        return False


def _index_of(device) -> int:
    if device is None:
        return _current_device
    if isinstance(device, int):
        return device
    d = torch.device(device)
    if d.type != "mojo":
        raise ValueError(f"expected a mojo device, got {d}")
    return _current_device if d.index is None else d.index


def synchronize(device=None) -> None:
    """Wait until every kernel issued on the device has finished."""
    from ..eager_kernels import flush_pending

    idx = _index_of(device)
    flush_pending()
    if _tensor_mod.storage_kind() == "cuda":
        torch.cuda.synchronize(idx)


class _Generator:
    """One device's RNG state: a 64-bit seed and a 64-bit offset counter,
    serialised as 16 little-endian bytes (seed, then counter) -- the state
    format of the reference's device module, so saved states interchange."""

    __slots__ = ("seed", "offset")
    _FMT = struct.Struct("<QQ")

    def __init__(self, seed: int, offset: int = 0) -> None:
        self.seed, self.offset = seed, offset

    def to_tensor(self) -> torch.Tensor:
        raw = self._FMT.pack(self.seed, self.offset)
        return torch.frombuffer(bytearray(raw), dtype=torch.uint8).clone()

    @classmethod
    def from_tensor(cls, t: torch.Tensor) -> "_Generator":
        raw = t.detach().to("cpu").contiguous().view(-1)
        if raw.dtype != torch.uint8 or raw.numel() != cls._FMT.size:
            raise ValueError(f"a mojo RNG state is {cls._FMT.size} uint8 values, got {raw.numel()} of {raw.dtype}")
        return cls(*cls._FMT.unpack(raw.numpy().tobytes()))


# Default seed of a device nobody seeded (the reference's value, so the
# initial states agree).
_DEFAULT_SEED = 67_280_421_310_721
_generators: dict[int, _Generator] = {}
_seed_for_new = _DEFAULT_SEED
_gen_lock = threading.Lock()


def _as_u64(seed) -> int:
    """A seed as torch.manual_seed takes it: any int in [-2^63, 2^64), kept
    modulo 2^64."""
    v = int(seed)
    if not -(1 << 63) <= v < (1 << 64):
        raise ValueError(f"seed {v} does not fit in 64 bits")
    return v % (1 << 64)


def _generator(index: int) -> _Generator:
    g = _generators.get(index)
    if g is None:
        g = _generators[index] = _Generator(_seed_for_new)
    return g


def manual_seed_all(seed) -> None:
    global _seed_for_new
    v = _as_u64(seed)
    with _gen_lock:
        _seed_for_new = v
        _generators.clear()
        for i in range(max(device_count(), 1)):
            _generators[i] = _Generator(v)


def manual_seed(seed) -> None:
    manual_seed_all(seed)


def get_rng_state(device=None) -> torch.Tensor:
    with _gen_lock:
        return _generator(_index_of(device)).to_tensor()


def set_rng_state(new_state, device=None) -> None:
    if not isinstance(new_state, torch.Tensor):
        raise TypeError(f"set_rng_state expects a torch.Tensor, got {type(new_state).__name__}")
    g = _Generator.from_tensor(new_state)
    with _gen_lock:
        _generators[_index_of(device)] = g


def get_amp_supported_dtype():
    return [torch.float16, torch.bfloat16]


def is_bf16_supported(including_emulation: bool = True) -> bool:
    return True


def get_device_name(device=None) -> str:
    if _tensor_mod.storage_kind() == "cuda":
        return torch.cuda.get_device_name(_index_of(device))
    return "mojo host stand-in"
