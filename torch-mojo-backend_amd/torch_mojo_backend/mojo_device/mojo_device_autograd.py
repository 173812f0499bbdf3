"""Autograd kernels of the mojo device: ``aten::scaled_dot_product_attention``
and ``aten::cross_entropy_loss`` (AutogradPrivateUse1), and the fused
linear used by the autocast ``linear`` policy.

SDPA:

Routing follows the reference (torch_mojo_backend/mojo_device/
mojo_device_autograd.py:565-643), re-targeted at gfx950:

- grad needed and the fused kernels accept the inputs -> the ATen flash op
  pair ``_scaled_dot_product_flash_attention`` / ``..._backward``; generated
  autograd saves (q, k, v, out, logsumexp) and calls the backward op, which
  recomputes P from the saved natural-log LSE (never the S x S matrix);
- no grad -> ``scaled_dot_product_attention`` on the device (fused kernel or
  decomposition);
- grad needed with grouped K/V heads or a sliding-window mask from
  torch_mojo_backend.masks -> ``_FusedAttention`` (fused forward, fused
  backward with dK/dV summed over each group), where the reference takes
  the math decomposition;
- otherwise (other masks, dropout) -> the math decomposition built from
  device ops, differentiated through its pieces.

There is no queue to drain before these routes: kernels are issued directly.

Cross-entropy: one fused softmax-cross-entropy Function (row LSE saved,
dlogits written once) where the inputs allow it, else the log_softmax ->
nll_loss decomposition.

Linear under autocast (mojo_device_autocast.py:547-561 puts linear in the
lower-precision list): ``_FusedLinear`` casts x, w and b to the autocast
dtype and runs one GEMM with the bias in its epilogue; its backward runs
the dX and dW GEMMs and the bias column sum, each rounded to the autocast
dtype and then widened to the dtype of the input it is the gradient of,
exactly what the autocast casts' own backward passes produce.  It replaces
the per-op chain (three casts, t, view, addmm, view and their autograd
nodes) with one Python call in each direction.
"""

from __future__ import annotations

import torch

from ..eager_kernels import aten_fast
from .torch_mojo_tensor import TorchMojoTensor

_registered = False
_library = None


def _scaled_dot_product_attention_autograd(
    query, key, value, attn_mask=None, dropout_p=0.0, is_causal=False, *, scale=None,
    enable_gqa=False,
):
    needs_backward = torch.is_grad_enabled() and (
        query.requires_grad or key.requires_grad or value.requires_grad
    )
    fused = aten_fast.fused_fa_inputs(
        query, key, value, attn_mask, dropout_p, is_causal, scale, enable_gqa
    )
    if not needs_backward:
        with torch._C._AutoDispatchBelowAutograd():
            return torch.ops.aten.scaled_dot_product_attention.default(
                query, key, value, attn_mask, dropout_p, is_causal, scale=scale,
                enable_gqa=enable_gqa,
            )
    if fused is not None:
        return torch.ops.aten._scaled_dot_product_flash_attention.default(
            query, key, value, dropout_p, is_causal, False, scale=scale
        )[0]
    ex = aten_fast.fused_fa_ex_inputs(
        query, key, value, attn_mask, dropout_p, is_causal, scale, enable_gqa
    )
    if ex is not None:
        _, _, _, causal, window = ex
        return _FusedAttention.apply(query, key, value, causal, window, scale)
    return aten_fast.sdpa_math(
        query, key, value, attn_mask, dropout_p, is_causal, scale, enable_gqa
    )


class _FusedAttention(torch.autograd.Function):
    """Attention with grouped K/V heads and/or a sliding-window causal mask
    (the Gemma-3-shaped layers), which the ATen flash pair cannot express:
    the fused forward saves (q, k, v, out, lse) like the pair does, and the
    fused backward recomputes P from the LSE, summing dK/dV over each
    group's query heads.  The reference differentiates these through its
    masked-math decomposition (aten_fast.py:9112-9123)."""

    @staticmethod
    def forward(ctx, q, k, v, causal, window, scale):
        with torch._C._AutoDispatchBelowAutograd():
            out, lse = aten_fast.attention_forward(q, k, v, causal, window, scale)
        ctx.save_for_backward(q, k, v, out, lse)
        ctx.args = (causal, window, scale)
        return out

    @staticmethod
    def backward(ctx, grad):
        q, k, v, out, lse = ctx.saved_tensors
        causal, window, scale = ctx.args
        with torch._C._AutoDispatchBelowAutograd():
            dq, dk, dv = aten_fast.attention_backward(grad, q, k, v, out, lse, causal, window, scale)
        return dq, dk, dv, None, None, None


def register_autograd_ops() -> None:
    global _registered, _library
    if _registered:
        return
    _library = torch.library.Library("aten", "IMPL", "AutogradPrivateUse1")
    _library.impl("scaled_dot_product_attention", _scaled_dot_product_attention_autograd)
    _library.impl("cross_entropy_loss", _cross_entropy_loss_autograd)
    _library.impl("rms_norm", _rms_norm_autograd)
    _library.impl("linear", _linear_autograd)
    _registered = True


def _linear_autograd(input, weight, bias=None):
    """aten::linear on the device.  When autograd records nothing (no_grad
    or inputs without requires_grad) and the operands share a float dtype,
    one GEMM with the bias in its epilogue, instead of the composite's
    transpose + matmul (+ add) chain of dispatches; otherwise the composite
    itself (aten's CompositeImplicitAutograd kernel), so training graphs are
    unchanged."""
    ts = (input, weight) if bias is None else (input, weight, bias)
    if (
        not (torch.is_grad_enabled() and any(t.requires_grad for t in ts))
        and all(isinstance(t, TorchMojoTensor) and hasattr(t, "_holder") for t in ts)
        and input.dtype in (torch.float32, torch.bfloat16, torch.float16)
        and all(t.dtype == input.dtype for t in ts)
        and weight.dim() == 2 and input.dim() >= 1 and input.shape[-1] == weight.shape[1]
        and (bias is None or (bias.dim() == 1 and bias.shape[0] == weight.shape[0]))
    ):
        return aten_fast.linear_forward(input, weight, bias)
    return torch.ops.aten.linear.default.decompose(input, weight, bias)


class _FusedLinear(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, w, b, dt):
        xl = aten_fast.cast_to(x, dt)
        wl = aten_fast.cast_to(w, dt)
        bl = aten_fast.cast_to(b, dt) if b is not None else None
        ctx.save_for_backward(xl, wl)
        ctx.dtypes = (x.dtype, w.dtype, b.dtype if b is not None else None)
        return aten_fast.linear_forward(xl, wl, bl)

    @staticmethod
    def backward(ctx, grad):
        xl, wl = ctx.saved_tensors
        nx, nw, nb = ctx.needs_input_grad[:3]
        nb = nb and ctx.dtypes[2] is not None
        g = grad if grad.dtype == xl.dtype else aten_fast.cast_to(grad, xl.dtype)
        xd, wd, bd = ctx.dtypes
        dx, dw, db = aten_fast.linear_backward(g, xl, wl, nx, nw, nb, xd, wd, bd)
        return dx, dw, db, None


def fused_linear(x, w, b, dt):
    return _FusedLinear.apply(x, w, b, dt)


def fused_linear_inputs(x, w, b, dt) -> bool:
    """Whether the autocast linear can take the fused path."""
    def ok(t):
        return (
            isinstance(t, TorchMojoTensor)
            and t.dtype in (torch.float32, torch.bfloat16, torch.float16)
            and hasattr(t, "_holder")
        )
    return (
        dt in (torch.bfloat16, torch.float16)
        and ok(x) and ok(w) and (b is None or (ok(b) and b.dim() == 1))
        and w.dim() == 2 and x.dim() >= 1 and x.shape[-1] == w.shape[1]
        and (b is None or b.shape[0] == w.shape[0])
    )


class _FusedCrossEntropy(torch.autograd.Function):
    """Softmax cross-entropy with saved row log-sum-exp: the forward reads the
    logits once, the backward writes dlogits = (softmax - onehot) * g once,
    instead of the log_softmax -> nll_loss chain's log-probabilities and
    dense one-hot gradient."""

    @staticmethod
    def forward(ctx, logits, target, reduction, ignore_index, out_dtype):
        # under autograd the loss is normally read after the backward: the
        # forward is left to the backward's single pass when it takes the shape
        lazy = (aten_fast.fused_cross_entropy_forward_deferred(logits, target, reduction, ignore_index)
                if ctx.needs_input_grad[0] else None)
        loss, lse, total = lazy or aten_fast.fused_cross_entropy_forward(logits, target, reduction, ignore_index)
        ctx.save_for_backward(logits, target, lse, total)
        ctx.reduction = reduction
        ctx.ignore_index = ignore_index
        ctx.loss_dtype = loss.dtype
        if out_dtype != loss.dtype:
            loss = loss.to(out_dtype)
        return loss

    @staticmethod
    def backward(ctx, grad):
        logits, target, lse, total = ctx.saved_tensors
        dx = aten_fast.fused_cross_entropy_backward(grad, logits, target, lse, total, ctx.reduction,
                                                    ctx.ignore_index)
        return dx, None, None, None, None


def _cross_entropy_loss_autograd(input, target, weight=None, reduction=1, ignore_index=-100,
                                 label_smoothing=0.0):
    if aten_fast.fused_cross_entropy_inputs(input, target, weight, reduction, ignore_index,
                                            label_smoothing) is not None:
        low = input.dtype in (torch.bfloat16, torch.float16)
        out_dtype = torch.float32 if (low and torch.is_autocast_enabled("mojo")) else input.dtype
        return _FusedCrossEntropy.apply(input, target, reduction, ignore_index, out_dtype)
    if float(label_smoothing) != 0.0:
        raise NotImplementedError(
            "cross_entropy with label_smoothing is not supported by the mojo eager device"
        )
    # other regimes (class weights, N-d inputs): the log_softmax -> nll_loss
    # decomposition on the device
    logp = torch.log_softmax(input, dim=1 if input.dim() > 1 else 0)
    return torch.nn.functional.nll_loss(
        logp, target, weight, reduction={0: "none", 1: "mean", 2: "sum"}[reduction],
        ignore_index=ignore_index,
    )


class _FusedRMSNorm(torch.autograd.Function):
    """rms_norm (the Gemma-3-shaped workload's norm) with scale w (+ an
    optional constant offset): the forward is one gfx950 kernel that also
    keeps the row rstd; the backward uses it, dx = r*(g*w) - x * r^3/n *
    sum(g*w*x) and dw = sum_rows(g*x*r), in one kernel (mi355x_rms_norm_bwd;
    device ops in f32 for inputs it does not take)."""

    @staticmethod
    def forward(ctx, x, normalized_shape, weight, eps, weight_offset=0.0):
        y, rstd = aten_fast.rms_norm_forward(x, normalized_shape, weight, eps, weight_offset)
        ctx.save_for_backward(x, weight, rstd)
        ctx.n = len(normalized_shape)
        ctx.offset = weight_offset
        return y

    @staticmethod
    def backward(ctx, grad):
        x, weight, rstd = ctx.saved_tensors
        nd = ctx.n
        need_w = weight is not None and ctx.needs_input_grad[2]
        with torch._C._AutoDispatchBelowAutograd():
            res = aten_fast.rms_norm_backward(grad, x, tuple(x.shape[x.dim() - nd:]), weight, rstd, ctx.offset,
                                              ctx.needs_input_grad[0], need_w)
        if res is not aten_fast.NOT_HANDLED:
            return res[0], None, res[1], None, None
        # other inputs: device elementwise and reduction ops
        dims = tuple(range(x.dim() - nd, x.dim()))
        n = 1
        for d in dims:
            n *= x.shape[d]
        xf, gf = x.float(), grad.float()
        r = rstd.view(tuple(x.shape[: x.dim() - nd]) + (1,) * nd)
        gw = gf * (weight.float() + ctx.offset) if weight is not None else gf
        dot = (gw * xf).sum(dim=dims, keepdim=True)
        dx = (r * gw - xf * (r * r * r) * (dot / n)).to(x.dtype) if ctx.needs_input_grad[0] else None
        dw = None
        if weight is not None and ctx.needs_input_grad[2]:
            lead = tuple(range(x.dim() - nd))
            dw = (gf * xf * r).sum(dim=lead).to(weight.dtype) if lead else (gf * xf * r).to(weight.dtype)
        return dx, None, dw, None, None


def _rms_norm_autograd(input, normalized_shape, weight=None, eps=None):
    if eps is None:
        eps = torch.finfo(input.dtype).eps
    shape = tuple(int(v) for v in normalized_shape)
    if isinstance(input, TorchMojoTensor) and (weight is None or isinstance(weight, TorchMojoTensor)):
        with torch._C._AutoDispatchBelowAutograd():
            ok = aten_fast.rms_norm_inputs(input, shape, weight)
        if ok:
            return _FusedRMSNorm.apply(input, shape, weight, float(eps))
    # other inputs: the decomposition on the device
    dims = tuple(range(input.dim() - len(shape), input.dim()))
    xf = input.float()
    y = xf * torch.rsqrt(xf.pow(2).mean(dim=dims, keepdim=True) + eps)
    if weight is not None:
        y = y * weight.float()
    return y.to(input.dtype)
