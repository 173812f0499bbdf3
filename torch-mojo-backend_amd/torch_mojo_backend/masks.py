"""Attention masks whose structure the mojo device can use.

Torch's SDPA has no sliding-window argument; a Gemma-3-style local layer
passes a boolean mask.  A mask built here on the mojo device records its
window (and the tensor's version counter, so an in-place edit voids it), and
SDPA then runs the flash kernel with that window (O(S*window) work) instead
of materialising the S x S scores.  The reference routes every masked SDPA
to its math decomposition (torch_mojo_backend/eager_kernels/aten_fast.py:
9112-9123, :6869); any other mask still takes that path here too.
"""

from __future__ import annotations

import torch

_WINDOW_ATTR = "_mojo_attn_window"


def sliding_window_causal_mask(seq_len: int, window: int, device="mojo") -> torch.Tensor:
    """bool [seq_len, seq_len]: True where query i may attend key j, i.e.
    i - window < j <= i (top-left aligned causal attention over the last
    `window` keys)."""
    if seq_len <= 0 or window <= 0:
        raise ValueError(f"sliding_window_causal_mask: seq_len {seq_len} and window {window} must be positive")
    i = torch.arange(seq_len).view(seq_len, 1)
    j = torch.arange(seq_len).view(1, seq_len)
    mask = ((j <= i) & (i - j < window)).to(device)
    if mask.device.type == "mojo":
        setattr(mask, _WINDOW_ATTR, (int(window), int(seq_len), mask._version))
    return mask


def window_of(mask) -> int | None:
    """The window of a mask built by sliding_window_causal_mask and not
    modified since, else None."""
    tag = getattr(mask, _WINDOW_ATTR, None)
    if tag is None:
        return None
    window, seq_len, version = tag
    if mask._version != version or mask.dtype != torch.bool or tuple(mask.shape) != (seq_len, seq_len):
        return None
    return window
