"""Fused ops of the Gemma-3-shaped workload: rotary embedding, GeGLU and
RMSNorm with a weight offset.

Torch has no single aten op for these (a model writes them as chains of
slice / neg / cat / mul / add, gelu + mul, and rms_norm with `1 + w`); the
functions here keep those semantics, run one gfx950 kernel each on the mojo
device, and fall back to the plain formula elsewhere (the CPU reference),
so a model written with them runs unchanged on both.  All are
differentiable.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from .eager_kernels import aten_fast
from .mojo_device.torch_mojo_tensor import TorchMojoTensor


def _on_mojo(*ts) -> bool:
    return all(isinstance(t, TorchMojoTensor) for t in ts)


def _needs_grad(*ts) -> bool:
    """Whether autograd records this call (otherwise the forward kernel is
    called directly, without an autograd Function's per-call cost)."""
    return torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in ts)


class _Rope(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, cos, sin):
        ctx.save_for_backward(cos, sin)
        return aten_fast.rope_forward(x, cos, sin)

    @staticmethod
    def backward(ctx, grad):
        cos, sin = ctx.saved_tensors
        return aten_fast.rope_forward(grad, cos, sin, inverse=True), None, None


def rotary_embedding(x, cos, sin):
    """x * cos + rotate_half(x) * sin over the last dim of x [B, H, T, D], with
    rotate_half(x) = cat(-x[..., D/2:], x[..., :D/2]) and cos/sin [T, D]."""
    if (_on_mojo(x, cos, sin) and x.dim() == 4 and x.shape[-1] % 8 == 0
            and tuple(cos.shape) == (x.shape[2], x.shape[3]) and tuple(sin.shape) == tuple(cos.shape)
            and x.dtype in (torch.float32, torch.bfloat16, torch.float16)):
        if not _needs_grad(x, cos, sin):
            return aten_fast.rope_forward(x, cos, sin)
        return _Rope.apply(x, cos, sin)
    half = x.shape[-1] // 2
    return x * cos + torch.cat([-x[..., half:], x[..., :half]], dim=-1) * sin


class _GeGLU(torch.autograd.Function):
    @staticmethod
    def forward(ctx, gate, up, approximate):
        ctx.save_for_backward(gate, up)
        ctx.approximate = approximate
        return aten_fast.geglu_forward(gate, up, approximate)

    @staticmethod
    def backward(ctx, grad):
        gate, up = ctx.saved_tensors
        if _on_mojo(grad) and grad.shape == gate.shape and grad.dtype == gate.dtype:
            with torch._C._AutoDispatchBelowAutograd():
                d_gate, d_up = aten_fast.geglu_backward(grad, gate, up, ctx.approximate)
            return d_gate, d_up, None
        act = F.gelu(gate, approximate=ctx.approximate)
        d_up = grad * act
        d_gate = torch.ops.aten.gelu_backward(grad * up, gate, approximate=ctx.approximate)
        return d_gate, d_up, None


def geglu(gate, up, approximate="tanh"):
    """gelu(gate) * up."""
    if (_on_mojo(gate, up) and gate.shape == up.shape and gate.dtype == up.dtype
            and gate.dtype in (torch.float32, torch.bfloat16, torch.float16)):
        if not _needs_grad(gate, up):
            return aten_fast.geglu_forward(gate, up, approximate)
        return _GeGLU.apply(gate, up, approximate)
    return F.gelu(gate, approximate=approximate) * up


def rms_norm(x, weight, eps, weight_offset=0.0):
    """rms_norm over the last dim with scale (weight + weight_offset), the
    scale formed in f32 (Gemma: weight_offset = 1)."""
    from .mojo_device.mojo_device_autograd import _FusedRMSNorm

    shape = (x.shape[-1],)
    if _on_mojo(x, weight) and aten_fast.rms_norm_inputs(x, shape, weight):
        if not _needs_grad(x, weight):
            return aten_fast.rms_norm_forward(x, shape, weight, float(eps), float(weight_offset))[0]
        return _FusedRMSNorm.apply(x, shape, weight, float(eps), float(weight_offset))
    return F.rms_norm(x, shape, weight.float() + weight_offset, eps)
