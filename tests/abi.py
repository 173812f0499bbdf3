"""Helpers for GPU parity tests that call the gfx950 library through its C ABI.

Device memory comes from PyTorch-ROCm tensors (plumbing only); every result
under test is produced by a library call.
"""

from __future__ import annotations

import ctypes

import numpy as np
import torch

from torch_mojo_backend.eager_kernels import AdamWTensor, check, lib  # noqa: F401

CODE = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2, torch.float64: 3, torch.int64: 4,
        torch.int32: 5, torch.int16: 6, torch.int8: 7, torch.uint8: 8, torch.bool: 9}
DEV = "cuda"


def i64(*vals):
    vals = [int(v) for v in vals]
    return (ctypes.c_int64 * max(len(vals), 1))(*vals)


def p(t):
    return None if t is None else t.data_ptr()


def dev(x, dtype=None):
    """numpy/torch CPU -> device tensor (optionally cast on the host first)."""
    t = torch.as_tensor(x)
    if dtype is not None:
        t = t.to(dtype)
    return t.contiguous().to(DEV)


def host(t):
    torch.cuda.synchronize()
    return t.detach().cpu()


def np64(t):
    return host(t).double().numpy()


def bhs(t):
    return i64(*t.stride()[:3])


def call(name, *args):
    check(name, getattr(lib(), name)(*args))


def workspace(nbytes):
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=DEV)


def tol_close(actual, expected, atol, rtol, what=""):
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    assert a.shape == e.shape, f"{what}: shape {a.shape} vs {e.shape}"
    bad = ~(np.abs(a - e) <= atol + rtol * np.abs(e))
    both_nan = np.isnan(a) & np.isnan(e)
    same_inf = np.isinf(a) & np.isinf(e) & (np.sign(a) == np.sign(e))
    bad &= ~(both_nan | same_inf)
    if bad.any():
        idx = np.argwhere(bad)[0]
        raise AssertionError(
            f"{what}: {bad.sum()} of {bad.size} elements outside atol={atol} rtol={rtol};"
            f" first at {tuple(idx)}: got {a[tuple(idx)]}, expected {e[tuple(idx)]};"
            f" max abs err {np.nanmax(np.abs(np.where(bad, a - e, 0))):.3e}"
        )
