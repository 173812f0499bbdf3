"""`torch.mojo`: the backend module of the eager mojo device.

Mirrors the reference's device module (torch_mojo_backend/mojo_device/
torch_mojo_device_module.py): device count/current/set, `synchronize`, the
Philox-style (seed, counter) RNG state as a 16-byte uint8 tensor, and the
AMP dtype list.  `mojo:N` is the N-th ROCm GPU; synchronising waits for the
device's stream (there is no launch queue to drain: kernels are built ahead
of time and issued directly).
"""

from __future__ import annotations

import threading

import torch

from . import torch_mojo_tensor as _tensor_mod

_current_device = 0
_UINT64_MASK = (1 << 64) - 1
_DEFAULT_RNG_SEED = 67_280_421_310_721
_rng_default_seed = _DEFAULT_RNG_SEED
_rng_states: dict[int, tuple[int, int]] = {}
_rng_lock = threading.Lock()


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
    idx = _index_of(device)
    if _tensor_mod.storage_kind() == "cuda":
        torch.cuda.synchronize(idx)


def _normalize_rng_seed(seed) -> int:
    value = int(seed)
    if value < -(1 << 63) or value > _UINT64_MASK:
        raise ValueError("Overflow when unpacking long long")
    return value & _UINT64_MASK


def manual_seed_all(seed) -> None:
    global _rng_default_seed
    normalized = _normalize_rng_seed(seed)
    with _rng_lock:
        _rng_default_seed = normalized
        _rng_states.clear()
        for index in range(max(device_count(), 1)):
            _rng_states[index] = (normalized, 0)


def manual_seed(seed) -> None:
    manual_seed_all(seed)


def get_rng_state(device=None) -> torch.Tensor:
    index = _index_of(device)
    with _rng_lock:
        seed, counter = _rng_states.setdefault(index, (_rng_default_seed, 0))
    encoded = seed.to_bytes(8, "little") + counter.to_bytes(8, "little")
    return torch.tensor(list(encoded), dtype=torch.uint8)


def set_rng_state(new_state, device=None) -> None:
    if not isinstance(new_state, torch.Tensor):
        raise TypeError("Mojo RNG state must be a torch.Tensor")
    state = new_state.detach().cpu().contiguous()
    if state.dtype != torch.uint8 or state.numel() != 16:
        raise ValueError("Mojo RNG state must be a 16-element uint8 tensor")
    encoded = bytes(state.reshape(-1).tolist())
    index = _index_of(device)
    with _rng_lock:
        _rng_states[index] = (
            int.from_bytes(encoded[:8], "little"),
            int.from_bytes(encoded[8:], "little"),
        )


def get_amp_supported_dtype():
    return [torch.float16, torch.bfloat16]


def is_bf16_supported(including_emulation: bool = True) -> bool:
    return True


def get_device_name(device=None) -> str:
    if _tensor_mod.storage_kind() == "cuda":
        return torch.cuda.get_device_name(_index_of(device))
    return "mojo host stand-in"
