"""The mojo device's host layer on the CPU (no GPU): dispatch, views,
autograd and autocast routing, argument packing, error behaviour.

The device runs over the host stand-in of the kernel library here
(tests/host_standin.py), so these tests check the Python side and the ABI
contract it relies on, not the gfx950 kernels (the `gpu` tests do that).
The reference's own device tests follow the same pattern: build on the
device, compare with stock PyTorch CPU (torch_mojo_backend/testing.py:
186-229).
"""

from __future__ import annotations

import subprocess
import sys

import pytest
import torch
import torch.nn.functional as F

from conftest import HAS_GPU, ROOT

pytestmark = pytest.mark.skipif(HAS_GPU, reason="host stand-in tests run where there is no GPU")


def test_device_identity_and_copies(mojo):
    x = torch.randn(4, 8)
    xm = x.to("mojo")
    assert xm.device.type == "mojo" and xm.device.index == 0
    assert torch.device("mojo:0") == xm.device
    assert torch.equal(xm.cpu(), x)
    assert torch.equal(torch.empty(3, device="mojo").fill_(2.5).cpu(), torch.full((3,), 2.5))
    assert torch.equal(torch.arange(7, device="mojo").cpu(), torch.arange(7))


def test_views_share_storage_and_strides(mojo):
    x = torch.randn(6, 10)
    xm = x.to("mojo")
    for f in (lambda t: t.t(), lambda t: t[1:5, ::3], lambda t: t.view(2, 3, 10).transpose(0, 2),
              lambda t: t.narrow(1, 2, 5), lambda t: t.unsqueeze(0).expand(3, 6, 10)):
        v = f(xm)
        assert v.shape == f(x).shape and v.stride() == f(x).stride()
        assert torch.equal(v.cpu(), f(x))
    v = xm[2]
    v.mul_(0)
    assert (xm.cpu()[2] == 0).all()


def test_elementwise_reduction_and_indexing(mojo):
    g = torch.Generator().manual_seed(1)
    a, b = torch.randn(5, 7, generator=g), torch.randn(5, 7, generator=g)
    am, bm = a.to("mojo"), b.to("mojo")
    assert torch.allclose((am * bm + am / (bm.abs() + 1)).cpu(), a * b + a / (b.abs() + 1))
    assert torch.allclose(am.sum(1).cpu(), a.sum(1), atol=1e-6)
    assert torch.equal(am.argmax(1).cpu(), a.argmax(1))
    idx = torch.tensor([4, 0, 4, 2])
    assert torch.equal(am.index_select(0, idx.to("mojo")).cpu(), a.index_select(0, idx))
    assert torch.equal(torch.cat([am, bm], 1).cpu(), torch.cat([a, b], 1))


def test_sdpa_autograd_routes_to_the_flash_pair(mojo):
    g = torch.Generator().manual_seed(2)
    q, k, v = (torch.randn(2, 2, 32, 64, generator=g).bfloat16() for _ in range(3))
    qm, km, vm = (t.to("mojo").requires_grad_() for t in (q, k, v))
    out = F.scaled_dot_product_attention(qm, km, vm, is_causal=True)
    assert type(out.grad_fn).__name__ == "ScaledDotProductFlashAttentionBackward0"
    out.float().sum().backward()
    qc, kc, vc = (t.float().requires_grad_() for t in (q, k, v))
    ref = F.scaled_dot_product_attention(qc, kc, vc, is_causal=True)
    ref.sum().backward()
    assert torch.allclose(out.float().cpu(), ref, atol=2e-2, rtol=2e-2)
    for a, b in ((qm, qc), (km, kc), (vm, vc)):
        assert torch.allclose(a.grad.float().cpu(), b.grad, atol=5e-2, rtol=5e-2)


def test_sdpa_with_mask_uses_the_math_route(mojo):
    q = torch.randn(1, 2, 8, 16).to("mojo").requires_grad_()
    mask = torch.ones(8, 8, dtype=torch.bool).tril().to("mojo")
    out = F.scaled_dot_product_attention(q, q, q, attn_mask=mask)
    assert "Flash" not in type(out.grad_fn).__name__
    ref = F.scaled_dot_product_attention(q.detach().cpu(), q.detach().cpu(), q.detach().cpu(),
                                         attn_mask=mask.cpu())
    assert torch.allclose(out.detach().cpu(), ref, atol=1e-5)


def test_autocast_policy(mojo):
    a, b = torch.randn(4, 8).to("mojo"), torch.randn(8, 3).to("mojo")
    x = torch.randn(4, 8).to("mojo")
    with torch.autocast("mojo", dtype=torch.bfloat16):
        assert (a @ b).dtype == torch.bfloat16
        assert F.layer_norm(x.bfloat16(), (8,)).dtype == torch.float32
        assert (a + 1).dtype == torch.float32  # everything else falls through


def test_fused_cross_entropy_matches_cpu(mojo):
    g = torch.Generator().manual_seed(3)
    logits, tgt = torch.randn(6, 37, generator=g), torch.tensor([1, 36, -100, 0, 5, 5])
    lm = logits.to("mojo").requires_grad_()
    loss = F.cross_entropy(lm, tgt.to("mojo"), ignore_index=-100)
    loss.backward()
    lc = logits.clone().requires_grad_()
    ref = F.cross_entropy(lc, tgt, ignore_index=-100)
    ref.backward()
    assert torch.allclose(loss.cpu(), ref, atol=1e-6)
    assert torch.allclose(lm.grad.cpu(), lc.grad, atol=1e-6)
    with pytest.raises(NotImplementedError):
        F.cross_entropy(lm, tgt.to("mojo"), label_smoothing=0.1)


def test_cross_entropy_forward_waits_for_the_backward(mojo):
    """Under autograd the fused cross-entropy forward is left pending: the
    backward computes loss, lse and dlogits in one pass
    (mi355x_cross_entropy_fwd_bwd) and the loss reads correctly afterwards;
    reading the loss first runs the forward (then the plain backward); an
    unread pending forward is run when the next one is deferred."""
    from torch_mojo_backend import eager_kernels as ek

    g = torch.Generator().manual_seed(8)
    logits, tgt = torch.randn(6, 40, generator=g), torch.tensor([1, 39, -100, 0, 5, 5])
    lc = logits.clone().requires_grad_()
    ref = F.cross_entropy(lc, tgt, ignore_index=-100)
    ref.backward()
    inner, counting, calls = _counting_library()
    ek.set_library_for_tests(counting)
    try:
        for read_first in (False, True):
            lm = logits.to("mojo").requires_grad_()
            loss = F.cross_entropy(lm, tgt.to("mojo"), ignore_index=-100)
            before = dict(calls)
            if read_first:
                assert torch.allclose(loss.cpu(), ref, atol=1e-6)
            loss.backward()
            assert torch.allclose(lm.grad.cpu(), lc.grad, atol=1e-6)
            assert torch.allclose(loss.cpu(), ref, atol=1e-6)
            fused = calls["mi355x_cross_entropy_fwd_bwd"] - before.get("mi355x_cross_entropy_fwd_bwd", 0)
            fwd = calls["mi355x_cross_entropy_fwd"] - before.get("mi355x_cross_entropy_fwd", 0)
            assert (fused, fwd) == ((0, 1) if read_first else (1, 0)), (read_first, fused, fwd)
        # a pending forward whose backward never comes runs at the next deferral
        lm = logits.to("mojo").requires_grad_()
        first = F.cross_entropy(lm, tgt.to("mojo"), ignore_index=-100)
        n0 = calls["mi355x_cross_entropy_fwd"]
        second = F.cross_entropy(lm, tgt.to("mojo"), ignore_index=-100)
        assert calls["mi355x_cross_entropy_fwd"] == n0 + 1
        second.backward()
        assert torch.allclose(first.cpu(), ref, atol=1e-6) and torch.allclose(second.cpu(), ref, atol=1e-6)
    finally:
        ek.set_library_for_tests(inner)


def test_gpt_step_matches_cpu(mojo):
    from torch_mojo_backend.gpt2 import BETAS, LEARNING_RATE, WEIGHT_DECAY, GPT, GPTConfig, make_batches, training_step

    cfg = GPTConfig(block_size=64, vocab_size=97, n_layer=2, n_head=2, n_embd=32)
    torch.manual_seed(0)
    ref = GPT(cfg)
    model = GPT(cfg)
    model.load_state_dict(ref.state_dict())
    model.to("mojo")
    assert model.lm_head.weight is model.transformer.wte.weight
    opt = model.configure_optimizers(WEIGHT_DECAY, LEARNING_RATE, BETAS, fused=True)
    ropt = ref.configure_optimizers(WEIGHT_DECAY, LEARNING_RATE, BETAS, fused=True)
    for x, y in make_batches(2, 64, cfg.vocab_size, 3, 5, "cpu"):
        lr_ = training_step(ref, ropt, x, y).item()
        lm = training_step(model, opt, x.to("mojo"), y.to("mojo")).item()
        assert abs(lm - lr_) <= 1e-4 * abs(lr_)
    for (name, p_ref), p in zip(ref.named_parameters(), model.parameters()):
        assert torch.allclose(p.detach().cpu(), p_ref.detach(), atol=1e-5, rtol=1e-4), name


def test_embedding_out_of_range_raises(mojo):
    w = torch.randn(10, 4).to("mojo")
    out = F.embedding(torch.tensor([1, 10]).to("mojo"), w)  # no host sync here
    with pytest.raises(IndexError, match="index out of range"):
        out.cpu()  # the flagged error surfaces at the next host read
    assert torch.equal(F.embedding(torch.tensor([1, 9]).to("mojo"), w).cpu(), w.cpu()[[1, 9]])
    lp = torch.randn(3, 5).log_softmax(1).to("mojo")
    loss = F.nll_loss(lp, torch.tensor([0, 5, 1]).to("mojo"))
    with pytest.raises(IndexError, match="Target is out of bounds"):
        loss.item()
    assert torch.isfinite(F.nll_loss(lp, torch.tensor([0, 4, 1]).to("mojo")).cpu())


def test_missing_library_fails_loudly(tmp_path):
    """No kernel library -> KernelLibraryError naming the build command; there
    is no CPU fallback."""
    code = (
        "import sys; sys.path.insert(0, %r)\n"
        "from torch_mojo_backend import eager_kernels as ek\n"
        "try:\n    ek.lib()\nexcept ek.KernelLibraryError as e:\n    print('RAISED', e)\n"
    ) % str(ROOT / "torch-mojo-backend_amd")
    env = {"MI355X_KERNELS_LIB": str(tmp_path / "absent.so"), "PATH": "/usr/bin:/bin"}
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, env=env, timeout=300)
    assert "RAISED" in r.stdout and "build" in r.stdout, r.stdout + r.stderr


def _linear_autocast_reference(x, w, b, dy):
    """torch CPU f32 restatement of autocast linear: operands rounded to
    bf16, f32 accumulation, output rounded to bf16; gradients computed from
    the rounded operands, rounded to bf16, then widened to f32."""
    xl, wl = x.bfloat16().float(), w.bfloat16().float()
    out = xl @ wl.t()
    if b is not None:
        out = out + b.bfloat16().float()
    out = out.bfloat16()
    dyf = dy.bfloat16().float()
    dx = (dyf @ wl).bfloat16().float()
    dw = (dyf.reshape(-1, dyf.shape[-1]).t() @ xl.reshape(-1, xl.shape[-1])).bfloat16().float()
    db = dyf.reshape(-1, dyf.shape[-1]).sum(0).bfloat16().float() if b is not None else None
    return out, dx, dw, db


@pytest.mark.parametrize("shape,bias,strided", [((6, 40), True, False), ((2, 5, 40), True, False),
                                                 ((2, 5, 40), False, True)])
def test_fused_linear_under_autocast(mojo, shape, bias, strided):
    g = torch.Generator().manual_seed(11)
    x = torch.randn(*shape, generator=g)
    if strided:  # a [.., 40] slice of a wider buffer
        x = torch.randn(*shape[:-1], 56, generator=g)[..., 8:48]
    w = torch.randn(24, 40, generator=g) * 0.2
    b = torch.randn(24, generator=g) if bias else None
    dy = torch.randn(*shape[:-1], 24, generator=g)
    xm = x.to("mojo").requires_grad_()
    wm = w.to("mojo").requires_grad_()
    bm = b.to("mojo").requires_grad_() if bias else None
    with torch.autocast("mojo", dtype=torch.bfloat16):
        out = F.linear(xm, wm, bm)
    assert out.dtype == torch.bfloat16 and tuple(out.shape) == tuple(shape[:-1]) + (24,)
    assert type(out.grad_fn).__name__ == "_FusedLinearBackward"
    out.backward(dy.bfloat16().to("mojo"))
    eo, edx, edw, edb = _linear_autocast_reference(x, w, b, dy)
    assert torch.allclose(out.float().cpu(), eo.float(), atol=2e-2, rtol=2e-2)
    assert xm.grad.dtype == torch.float32 and wm.grad.dtype == torch.float32
    assert torch.allclose(xm.grad.cpu(), edx, atol=2e-2, rtol=2e-2)
    assert torch.allclose(wm.grad.cpu(), edw, atol=2e-2, rtol=2e-2)
    if bias:
        assert torch.allclose(bm.grad.cpu(), edb, atol=2e-2, rtol=2e-2)


def _counting_library():
    """Wrap the active kernel library so calls are counted by entry point."""
    import collections

    from torch_mojo_backend import eager_kernels as ek

    inner = ek.lib()
    calls = collections.Counter()

    class Counting:
        def __getattr__(self, name):
            fn = getattr(inner, name)

            def wrapped(*a, **k):
                calls[name] += 1
                return fn(*a, **k)

            return wrapped

    return inner, Counting(), calls


def test_layer_norm_low_copy_feeds_autocast_linear(mojo):
    """Under autocast the f32 layer norm also writes its output in bf16 and
    the linear's cast takes that copy instead of a cast kernel; the copy is
    used once and never after the output is modified."""
    from torch_mojo_backend import eager_kernels as ek

    g = torch.Generator().manual_seed(5)
    x = torch.randn(6, 16, generator=g)
    w, b = torch.randn(8, 16, generator=g), torch.randn(8, generator=g)
    lw, lb = torch.randn(16, generator=g), torch.randn(16, generator=g)
    xm, wm, bm, lwm, lbm = (t.to("mojo") for t in (x, w, b, lw, lb))
    inner, counting, calls = _counting_library()
    ek.set_library_for_tests(counting)
    try:
        with torch.autocast("mojo", dtype=torch.bfloat16):
            y = F.layer_norm(xm, (16,), lwm, lbm)
            assert y.dtype == torch.float32
            casts = calls["mi355x_copy"]
            out = F.linear(y, wm, bm)
            assert calls["mi355x_layer_norm_fwd_ex"] == 1
            # only the weight and bias casts, not the activation's
            assert calls["mi355x_copy"] - casts == 2
            y2 = y.bfloat16()  # the copy went to the linear: this one is a fresh cast
            assert calls["mi355x_copy"] - casts == 3
            z = F.layer_norm(xm, (16,), lwm, lbm)
            z.mul_(2.0)  # modified: its copy is stale
            before = calls["mi355x_copy"]
            z2 = z.bfloat16()
            assert calls["mi355x_copy"] == before + 1
    finally:
        ek.set_library_for_tests(inner)
    yr = F.layer_norm(x, (16,), lw, lb)
    ref = yr.bfloat16().float() @ w.bfloat16().float().t() + b.bfloat16().float()
    assert torch.allclose(out.float().cpu(), ref, atol=2e-2, rtol=2e-2)
    assert torch.equal(y2.cpu(), yr.bfloat16()) or torch.allclose(y2.float().cpu(), yr, atol=1e-2)
    assert torch.allclose(z2.float().cpu(), 2 * yr, atol=3e-2)


def test_autocast_layer_norm_output_is_computed_on_first_use(mojo):
    """Under autocast the layer norm writes its bf16 copy and statistics; its
    f32 output is produced (mi355x_layer_norm_apply, from the saved x, mean
    and rstd) only when something touches it, never when the linear takes the
    copy and the output dies.  Writes into its inputs (x, the weight) or into
    the output itself wait for it."""
    from torch_mojo_backend import eager_kernels as ek

    g = torch.Generator().manual_seed(23)
    x = torch.randn(64, 768, generator=g)
    w, b = torch.randn(768, generator=g), torch.randn(768, generator=g)
    lw = torch.randn(32, 768, generator=g)
    xm, wm, bm, lwm = (t.to("mojo") for t in (x, w, b, lw))
    ref = F.layer_norm(x, (768,), w, b)
    inner, counting, calls = _counting_library()
    ek.set_library_for_tests(counting)

    def ln(t=xm):
        with torch.autocast("mojo", dtype=torch.bfloat16):
            return F.layer_norm(t, (768,), wm, bm)

    try:
        # only the copy is used: the f32 output is never computed
        with torch.autocast("mojo", dtype=torch.bfloat16):
            y = F.layer_norm(xm, (768,), wm, bm)
            assert ek._lazy
            z = F.linear(y, lwm)
        del y
        assert not ek._lazy and calls["mi355x_layer_norm_apply"] == 0
        zr = ref.bfloat16().float() @ lw.bfloat16().float().t()
        assert torch.allclose(z.float().cpu(), zr, atol=3e-2, rtol=2e-2)
        # a host read, a kernel, a view
        assert torch.allclose(ln().cpu(), ref, atol=1e-5, rtol=1e-5)
        assert torch.allclose((ln() * 2).cpu(), 2 * ref, atol=2e-5, rtol=1e-5)
        assert torch.allclose(ln()[5].cpu(), ref[5], atol=1e-5, rtol=1e-5)
        assert calls["mi355x_layer_norm_apply"] == 3 and not ek._lazy
        # writes into x, the weight and the output itself wait for it
        x2 = xm.clone()
        y = ln(x2)
        x2.mul_(0)
        assert torch.allclose(y.cpu(), ref, atol=1e-5, rtol=1e-5)
        y = ln()
        wm.add_(1.0)
        assert torch.allclose(y.cpu(), ref, atol=1e-5, rtol=1e-5)
        wm.sub_(1.0)
        y = ln()
        y.add_(1.0)
        assert torch.allclose(y.cpu(), ref + 1, atol=2e-5, rtol=1e-5)
        # the output of a fused residual add + norm: x is the add's result
        d = torch.randn(64, 768, generator=g).bfloat16()
        s = xm + d.to("mojo")
        y = ln(s)
        assert torch.allclose(y.cpu(), F.layer_norm(x + d.float(), (768,), w, b), atol=1e-5, rtol=1e-5)
    finally:
        ek.set_library_for_tests(inner)
    assert not ek._lazy


def test_clip_scale_is_applied_inside_the_fused_adamw_step(mojo):
    """clip_grad_norm_'s _foreach_mul_ of the gradients is held back and the
    fused AdamW step applies it as it reads them (grad_mul): no separate
    multiply runs, the update equals stock PyTorch's, and the gradients still
    read as scaled afterwards (the multiply then runs once)."""
    from torch_mojo_backend import eager_kernels as ek

    torch.manual_seed(3)
    ref = torch.nn.Sequential(torch.nn.Linear(16, 32), torch.nn.GELU(), torch.nn.Linear(32, 4))
    dev = torch.nn.Sequential(torch.nn.Linear(16, 32), torch.nn.GELU(), torch.nn.Linear(32, 4))
    dev.load_state_dict(ref.state_dict())
    dev.to("mojo")
    opts = [torch.optim.AdamW(m.parameters(), lr=1e-2, fused=(m is dev)) for m in (ref, dev)]
    x = torch.randn(8, 16)
    inner = ek.lib()
    muls = []

    class MulCounting:  # counts foreach multiplies (opcode 2; the step count's add is opcode 0)
        def __getattr__(self, name):
            fn = getattr(inner, name)
            if name != "mi355x_foreach_apply":
                return fn

            def wrapped(op, *a):
                if op == 2:
                    muls.append(1)
                return fn(op, *a)

            return wrapped

    calls = {}
    ek.set_library_for_tests(MulCounting())
    try:
        for m, opt, xx in ((ref, opts[0], x), (dev, opts[1], x.to("mojo"))):
            (m(xx) ** 2).sum().backward()
            n = torch.nn.utils.clip_grad_norm_(m.parameters(), 0.1)
            assert float(n.cpu()) > 0.1  # the clip scales
            opt.step()
        calls["mi355x_foreach_apply"] = len(muls)
        assert calls["mi355x_foreach_apply"] == 0 and ek._lazy
        for a, b in zip(ref.parameters(), dev.parameters()):
            assert torch.allclose(b.detach().cpu(), a.detach(), atol=1e-6, rtol=1e-5)
        for a, b in zip(ref.parameters(), dev.parameters()):
            assert torch.allclose(b.grad.cpu(), a.grad, atol=1e-7, rtol=1e-5)
        calls["mi355x_foreach_apply"] = len(muls)
        assert calls["mi355x_foreach_apply"] == 1 and not ek._lazy
        # a second step: the grads die at zero_grad, the multiply never runs
        for m, opt, xx in ((ref, opts[0], x), (dev, opts[1], x.to("mojo"))):
            opt.zero_grad()
            (m(xx) ** 2).sum().backward()
            torch.nn.utils.clip_grad_norm_(m.parameters(), 0.1)
            opt.step()
            opt.zero_grad()
        calls["mi355x_foreach_apply"] = len(muls)
        assert calls["mi355x_foreach_apply"] == 1 and not ek._lazy
        for a, b in zip(ref.parameters(), dev.parameters()):
            assert torch.allclose(b.detach().cpu(), a.detach(), atol=1e-6, rtol=1e-5)
    finally:
        ek.set_library_for_tests(inner)


def test_pending_scale_reaches_views_that_outlive_the_scaled_tensor(mojo):
    """A pending _foreach_mul_ holds the storages, not the tensor objects: a
    view taken before the scaled tensor itself is dropped still reads the
    scaled values."""
    from torch_mojo_backend import eager_kernels as ek

    g = torch.Generator().manual_seed(31)
    a, b = torch.randn(64, generator=g), torch.randn(8, 8, generator=g)
    am, bm = a.to("mojo"), b.to("mojo")
    coef = torch.tensor(0.25).to("mojo")
    torch._foreach_mul_([am, bm], coef)
    assert ek._lazy
    view = bm.detach()[2:5]
    del bm
    assert torch.allclose(view.cpu(), b[2:5] * 0.25)
    assert torch.allclose(am.cpu(), a * 0.25)
    assert not ek._lazy


def test_tied_embedding_gradient_is_added_in_place_of_a_dense_sum(mojo):
    """With tied input/output embeddings, autograd adds the embedding's dense
    gradient onto the projection's (`grad += g`); that add takes the lazy
    embedding gradient as a scatter-add of the named rows
    (mi355x_embedding_bwd_accumulate): no dense gradient is written and the
    result matches PyTorch.  An untied embedding's gradient stays lazy until
    read."""
    from torch_mojo_backend import eager_kernels as ek

    torch.manual_seed(4)
    V, D = 50, 16
    emb = torch.nn.Embedding(V, D)
    pos = torch.nn.Embedding(12, D)
    idx = torch.randint(0, V, (3, 12))
    idx[0, :4] = 7  # repeated rows
    demb = torch.nn.Embedding(V, D).to("mojo")
    dpos = torch.nn.Embedding(12, D).to("mojo")
    demb.load_state_dict({k: v.to("mojo") for k, v in emb.state_dict().items()})
    dpos.load_state_dict({k: v.to("mojo") for k, v in pos.state_dict().items()})

    tgt = torch.randint(0, V, (36,))

    def loss(e, p_, ids):
        h = e(ids) + p_(torch.arange(12, device=ids.device))
        return F.cross_entropy((h @ e.weight.t()).view(-1, V), tgt.to(ids.device))

    inner, counting, calls = _counting_library()
    ek.set_library_for_tests(counting)
    try:
        loss(emb, pos, idx).backward()
        loss(demb, dpos, idx.to("mojo")).backward()
        assert calls["mi355x_embedding_bwd_accumulate"] == 1 and calls["mi355x_embedding_bwd"] == 0
        assert torch.allclose(demb.weight.grad.cpu(), emb.weight.grad, atol=1e-5, rtol=1e-5)
        assert calls["mi355x_embedding_bwd"] == 0
        assert torch.allclose(dpos.weight.grad.cpu(), pos.weight.grad, atol=1e-5, rtol=1e-5)
        assert calls["mi355x_embedding_bwd"] == 1  # the position embedding's, on first read
    finally:
        ek.set_library_for_tests(inner)
    assert not ek._lazy


def test_adamw_parameter_copies_feed_next_autocast_forward(mojo):
    """The fused AdamW step writes the bf16 copy of every parameter the
    autocast forward casts; the next forward uses it with no cast kernel.  A
    write into a parameter (in place, or through .data) drops its copy."""
    from torch_mojo_backend import eager_kernels as ek

    torch.manual_seed(0)
    lin = torch.nn.Linear(16, 8).to("mojo")
    opt = torch.optim.AdamW(lin.parameters(), lr=1e-2, fused=True)
    x = torch.randn(4, 16).to("mojo")

    def step():
        with torch.autocast("mojo", dtype=torch.bfloat16):
            out = lin(x)
        out.float().sum().backward()
        opt.step()
        opt.zero_grad()

    def forward_counting():
        inner, counting, calls = _counting_library()
        ek.set_library_for_tests(counting)
        try:
            with torch.autocast("mojo", dtype=torch.bfloat16):
                out = lin(x)
        finally:
            ek.set_library_for_tests(inner)
        return out, calls["mi355x_copy"]

    def expected():
        w, b = lin.weight.detach().cpu(), lin.bias.detach().cpu()
        return x.cpu().bfloat16().float() @ w.bfloat16().float().t() + b.bfloat16().float()

    step()  # the first forward casts; this step writes the copies
    out, casts = forward_counting()
    assert casts == 1  # only the f32 input x; weight and bias come from the optimizer
    assert torch.allclose(out.float().cpu(), expected(), atol=2e-2, rtol=2e-2)
    step()
    with torch.no_grad():
        lin.weight.data.mul_(2.0)  # a write the version counter does not see
    out, casts = forward_counting()
    assert casts == 2  # x and the weight again; the bias copy is still current
    assert torch.allclose(out.float().cpu(), expected(), atol=2e-2, rtol=2e-2)
    step()
    with torch.no_grad():
        lin.bias.copy_(torch.randn(8).to("mojo"))  # an in-place op on the parameter itself
    out, casts = forward_counting()
    assert casts == 2
    assert torch.allclose(out.float().cpu(), expected(), atol=2e-2, rtol=2e-2)


def test_window_mask_tag_and_gqa_route(mojo):
    from torch_mojo_backend import eager_kernels as ek
    from torch_mojo_backend.masks import sliding_window_causal_mask, window_of

    g = torch.Generator().manual_seed(12)
    q = torch.randn(1, 4, 10, 64, generator=g).bfloat16()
    k, v = (torch.randn(1, 2, 10, 64, generator=g).bfloat16() for _ in range(2))
    mask = sliding_window_causal_mask(10, 3)
    assert window_of(mask) == 3
    inner, counting, calls = _counting_library()
    ek.set_library_for_tests(counting)
    try:
        with torch.no_grad():
            out = F.scaled_dot_product_attention(q.to("mojo"), k.to("mojo"), v.to("mojo"), attn_mask=mask,
                                                 enable_gqa=True)
        assert calls["mi355x_attn_fwd_ex"] == 1
        ref = F.scaled_dot_product_attention(q.float(), k.float(), v.float(), attn_mask=mask.cpu(), enable_gqa=True)
        assert torch.allclose(out.float().cpu(), ref, atol=2e-2, rtol=2e-2)
        mask[0, 0] = False  # an in-place edit voids the tag: the math path takes it
        assert window_of(mask) is None
        with torch.no_grad():
            F.scaled_dot_product_attention(q.to("mojo"), k.to("mojo"), v.to("mojo"), attn_mask=mask,
                                           enable_gqa=True)
        assert calls["mi355x_attn_fwd_ex"] == 1
    finally:
        ek.set_library_for_tests(inner)


def test_gemma_shaped_prefill_on_device(mojo):
    """A small Gemma-3-shaped model (GQA, sliding window, RMSNorm, GeGLU,
    RoPE) in bf16 on the device against the same weights in f32 on the CPU;
    the windowed/grouped attention and RMSNorm go through their kernels."""
    from torch_mojo_backend import eager_kernels as ek
    from torch_mojo_backend.gemma3 import Gemma3, Gemma3Config

    cfg = Gemma3Config(vocab_size=97, hidden=64, layers=3, heads=4, kv_heads=1, head_dim=64, d_ff=96,
                       window=5, global_every=3)
    torch.manual_seed(0)
    ref = Gemma3(cfg)
    for _, prm in ref.named_parameters():
        if prm.dim() == 1:
            torch.nn.init.normal_(prm, std=0.1)
    ref = ref.to(torch.bfloat16).float()  # the bf16-rounded weights, in f32
    model = Gemma3(cfg)
    model.load_state_dict(ref.state_dict())
    model = model.to(torch.bfloat16).to("mojo")
    idx = torch.randint(0, 97, (2, 12), generator=torch.Generator().manual_seed(1))
    inner, counting, calls = _counting_library()
    ek.set_library_for_tests(counting)
    try:
        with torch.no_grad():
            got = model(idx.to("mojo")).float().cpu()
    finally:
        ek.set_library_for_tests(inner)
    with torch.no_grad():
        want = ref(idx)
    assert calls["mi355x_attn_fwd_ex"] == 3 and calls["mi355x_rms_norm_fwd"] >= 3 * 6 + 1
    assert torch.allclose(got, want, atol=5e-2, rtol=5e-2), (got - want).abs().max()


def test_fused_gemma_ops_gradients(mojo):
    """rotary_embedding, geglu and rms_norm(weight_offset) on the device
    against autograd of their formulas on the CPU."""
    from torch_mojo_backend import ops

    g = torch.Generator().manual_seed(13)
    x = torch.randn(2, 3, 7, 16, generator=g)
    ang = torch.randn(7, 8, generator=g)
    cos, sin = torch.cat([ang.cos()] * 2, -1), torch.cat([ang.sin()] * 2, -1)
    gate, up = torch.randn(5, 24, generator=g), torch.randn(5, 24, generator=g)
    h, w = torch.randn(5, 24, generator=g), torch.randn(24, generator=g) * 0.1
    dy1, dy2, dy3 = torch.randn(2, 3, 7, 16, generator=g), torch.randn(5, 24, generator=g), torch.randn(5, 24, generator=g)

    def run(dev):
        ts = [t.to(dev).requires_grad_() for t in (x, gate, up, h, w)]
        xm, gm, um, hm, wm = ts
        y1 = ops.rotary_embedding(xm, cos.to(dev), sin.to(dev))
        y2 = ops.geglu(gm, um)
        y3 = ops.rms_norm(hm, wm, 1e-6, weight_offset=1.0)
        torch.autograd.backward([y1, y2, y3], [dy1.to(dev), dy2.to(dev), dy3.to(dev)])
        return [y.detach().cpu() for y in (y1, y2, y3)] + [t.grad.cpu() for t in ts]

    for a, b in zip(run("mojo"), run("cpu")):
        assert torch.allclose(a, b, atol=1e-5, rtol=1e-5), (a - b).abs().max()


def test_allocation_retries_once_after_out_of_memory(mojo, monkeypatch):
    """An allocation the allocator refuses is retried once after releasing
    cached blocks (the reference's drain-and-retry,
    torch_mojo_tensor.py:213-244); a second refusal propagates."""
    from torch_mojo_backend.mojo_device import torch_mojo_tensor as tm

    real = torch.empty
    fails = {"n": 1}

    def flaky(*a, **k):
        if fails["n"] > 0:
            fails["n"] -= 1
            raise torch.OutOfMemoryError("out of memory (test)")
        return real(*a, **k)

    monkeypatch.setattr(tm.torch, "empty", flaky)
    x = torch.ones(5).to("mojo")
    assert torch.equal(x.cpu(), torch.ones(5))
    fails["n"] = 2
    with pytest.raises(torch.OutOfMemoryError):
        torch.ones(7).to("mojo")


def test_checkpoints_pickle_as_cpu_tensors(mojo, tmp_path):
    """torch.save of device tensors and state_dicts writes plain CPU tensors
    (torch_mojo_tensor.py:572-583), so the file loads without the backend."""
    lin = torch.nn.Linear(4, 3)
    ref = {k: v.clone() for k, v in lin.state_dict().items()}
    lin.to("mojo")
    path = tmp_path / "ckpt.pt"
    torch.save({"model": lin.state_dict(), "t": torch.arange(6.0).to("mojo")}, path)
    loaded = torch.load(path, weights_only=True)
    assert loaded["t"].device.type == "cpu" and torch.equal(loaded["t"], torch.arange(6.0))
    for k, v in ref.items():
        assert loaded["model"][k].device.type == "cpu" and torch.equal(loaded["model"][k], v)


@pytest.mark.parametrize("dtype,bits", [(torch.float32, torch.int32), (torch.bfloat16, torch.int16)])
def test_stack_and_cat_of_many_pieces_are_bit_exact(mojo, dtype, bits):
    """The multi-tensor path of stack/cat (8 or more contiguous pieces)
    keeps signed zeros and infinities bit for bit.  (The host stand-in's
    x86 arithmetic may return a different NaN payload; the GPU test checks
    NaN bits too.)"""
    vals = torch.tensor([0.0, -0.0, float("nan"), float("inf"), -float("inf"), 1e-40, -3.5, 2.0 ** 100] * 3)
    pieces = [v.clone().to(dtype) for v in vals]
    got = torch.stack([x.to("mojo") for x in pieces]).cpu()
    exp = torch.stack(pieces)
    nan = torch.isnan(exp)
    assert torch.equal(torch.isnan(got), nan)
    assert torch.equal(got[~nan].view(bits), exp[~nan].view(bits))
    rows = [torch.randn(5 + i).to(dtype) for i in range(10)]
    rows[3][2] = -0.0
    got = torch.cat([r.to("mojo") for r in rows]).cpu()
    assert torch.equal(got.view(bits), torch.cat(rows).view(bits))


@pytest.mark.parametrize("n_pieces", [3, 9])
def test_cat_rejects_mismatched_shapes(mojo, n_pieces):
    """torch.cat's shape checks on the device (both the per-piece path and
    the multi-tensor path of 8 or more pieces): a piece whose size differs
    outside the cat dim, or whose rank differs, raises instead of writing
    past the output."""
    pieces = [torch.randn(2, 3).to("mojo") for _ in range(n_pieces - 1)]
    with pytest.raises(RuntimeError, match="Sizes of tensors must match"):
        torch.cat(pieces + [torch.randn(2, 5).to("mojo")])
    with pytest.raises(RuntimeError, match="same number of dimensions"):
        torch.cat(pieces + [torch.randn(2, 3, 1).to("mojo")])
    ok = [torch.randn(2, 3) for _ in range(n_pieces)]
    assert torch.equal(torch.cat([x.to("mojo") for x in ok], 1).cpu(), torch.cat(ok, 1))


@pytest.mark.parametrize("case", ["noncontig", "mixed_dtype", "dim1"])
def test_cat_of_many_pieces_off_the_fast_path(mojo, case):
    """Conditions that keep cat off its multi-tensor path (a non-contiguous
    piece, mixed dtypes, a cat dim with leading extent > 1) still give
    torch.cat's result."""
    g = torch.Generator().manual_seed(5)
    pieces = [torch.randn(4, 6, generator=g) for _ in range(9)]
    dim = 0
    if case == "noncontig":
        pieces[4] = torch.randn(6, 4, generator=g).t()
    elif case == "mixed_dtype":
        pieces[2] = pieces[2].bfloat16()
    else:
        dim = 1
    got = torch.cat([x.to("mojo") for x in pieces], dim).cpu()
    exp = torch.cat(pieces, dim)
    assert got.dtype == exp.dtype and torch.equal(got, exp)


def test_fused_adamw_checks_the_amsgrad_state(mojo):
    """max_exp_avg_sqs gets the same numel check as the other state lists
    (a short buffer would be read and written past its end)."""
    p = torch.randn(10).to("mojo")
    g, m, v = (torch.randn(10).to("mojo") for _ in range(3))
    step = torch.zeros(()).to("mojo")
    short = torch.zeros(7).to("mojo")
    with pytest.raises(RuntimeError, match="max_exp_avg_sq 0 has 7 elements"):
        torch._fused_adamw_([p], [g], [m], [v.abs()], [short], [step], lr=1e-3, beta1=0.9, beta2=0.99,
                            weight_decay=0.0, eps=1e-8, amsgrad=True, maximize=False)


def test_cat_of_attention_gradient_slices_is_a_view(mojo):
    """The attention backward hands out dQ, dK, dV as adjacent slices of one
    buffer; the cat of the fused-qkv split's backward returns that buffer as
    a view (no copy) and matches torch.  A cat of adjacent slices of an
    unmarked buffer still copies (cat never aliases its inputs otherwise)."""
    from torch_mojo_backend.eager_kernels import aten_fast

    g = torch.Generator().manual_seed(4)
    B, T, H, D = 2, 16, 2, 8
    qkv = torch.randn(B, T, 3 * H * D, generator=g)
    qkv_m = qkv.to("mojo").requires_grad_()
    q, k, v = (t.view(B, T, H, D).transpose(1, 2) for t in qkv_m.split(H * D, dim=2))
    out = F.scaled_dot_product_attention(q, k, v, is_causal=True)
    dout = torch.randn(out.shape, generator=g)
    out.backward(dout.to("mojo"))
    qc = qkv.clone().requires_grad_()
    qq, kk, vv = (t.view(B, T, H, D).transpose(1, 2) for t in qc.split(H * D, dim=2))
    F.scaled_dot_product_attention(qq, kk, vv, is_causal=True).backward(dout)
    assert torch.allclose(qkv_m.grad.cpu(), qc.grad, atol=1e-5, rtol=1e-4)
    # unmarked storage: a copy, so writing the result leaves the pieces alone
    base = torch.randn(4, 6).to("mojo")
    a, b = base[:, :3], base[:, 3:]
    c = torch.cat([a, b], 1)
    c.zero_()
    assert not torch.equal(base.cpu(), torch.zeros(4, 6))
    assert aten_fast._CAT_READY


def test_residual_add_is_fused_into_the_next_layer_norm(mojo):
    """A large f32 + bf16 add whose result feeds a LayerNorm runs inside the
    norm (one pass); the sum is still materialised for its other users, and
    any other consumer (a host read, another kernel) gets the add first."""
    from torch_mojo_backend import eager_kernels as ek

    g = torch.Generator().manual_seed(9)
    x = torch.randn(128, 768, generator=g)
    d = torch.randn(128, 768, generator=g).bfloat16()
    w, b = torch.randn(768, generator=g), torch.randn(768, generator=g)
    xm, dm, wm, bm = (t.to("mojo") for t in (x, d, w, b))
    s = xm + dm
    assert ek._pending  # held back
    y = F.layer_norm(s, (768,), wm, bm)
    assert not ek._pending
    ref_s = x + d.float()
    assert torch.equal(s.cpu(), ref_s)
    assert torch.allclose(y.cpu(), F.layer_norm(ref_s, (768,), w, b), atol=1e-5, rtol=1e-5)
    # other consumers see the sum: another kernel, then a host read
    s2 = xm + dm
    assert torch.equal((s2 * 2).cpu(), ref_s * 2)
    s3 = xm + dm
    assert torch.equal(s3.cpu(), ref_s)
    # the inputs may change after the add is taken: it was computed first
    s4 = xm + dm
    xm.mul_(0)
    assert torch.equal(s4.cpu(), ref_s)


def test_chained_held_back_adds_keep_their_order(mojo):
    """h = x + a and h2 = h + b are both held back; a LayerNorm (or a cast)
    of h must not take h's add out of the queue ahead of h2's, which reads
    h: h2 would then be computed from h before h exists."""
    from torch_mojo_backend import eager_kernels as ek

    g = torch.Generator().manual_seed(19)
    x = torch.randn(128, 768, generator=g)
    a = torch.randn(128, 768, generator=g).bfloat16()
    b = torch.randn(128, 768, generator=g).bfloat16()
    w, bias = torch.randn(768, generator=g), torch.randn(768, generator=g)
    xm, am, bm, wm, biasm = (t.to("mojo") for t in (x, a, b, w, bias))
    ref_h = x + a.float()
    ref_h2 = ref_h + b.float()
    for consume in (lambda h: F.layer_norm(h, (768,), wm, biasm), lambda h: h.to(torch.bfloat16)):
        h = xm + am
        h2 = h + bm
        assert len(ek._pending) == 2
        y = consume(h)
        assert not ek._pending
        assert torch.equal(h.cpu(), ref_h)
        assert torch.equal(h2.cpu(), ref_h2)
        assert y.cpu().shape == (128, 768)
    assert torch.allclose(F.layer_norm(xm + am, (768,), wm, biasm).cpu(),
                          F.layer_norm(ref_h, (768,), w, bias), atol=1e-5, rtol=1e-5)


def test_held_back_sum_and_its_autocast_copy_in_one_pass(mojo):
    """cast_to of a held-back f32 sum (the residual gradient the autograd
    engine adds up, then cast for the next linear's backward) computes the
    sum and the bf16 copy together; both match the separate ops."""
    from torch_mojo_backend import eager_kernels as ek
    from torch_mojo_backend.eager_kernels import aten_fast

    g = torch.Generator().manual_seed(10)
    a, r = torch.randn(256, 768, generator=g), torch.randn(256, 768, generator=g)
    am, rm = a.to("mojo"), r.to("mojo")
    s = am + rm
    assert ek._pending
    low = aten_fast.cast_to(s, torch.bfloat16)
    assert not ek._pending
    assert torch.equal(s.cpu(), a + r)
    assert torch.equal(low.cpu(), (a + r).bfloat16())


def test_clip_grad_norm_stacks_the_norms_as_a_view(mojo):
    """_foreach_norm writes its per-tensor norms into one buffer; the stack
    that clip_grad_norm_ takes of them is a view of it (no copy).  Norms and
    clipped gradients match torch; a second stack of the same norms copies."""
    g = torch.Generator().manual_seed(5)
    shapes = [(7, 3), (5,), (2, 4, 3), (1,)]
    grads = [torch.randn(s, generator=g) for s in shapes]
    ps = [torch.zeros(s).to("mojo").requires_grad_() for s in shapes]
    for p, gr in zip(ps, grads):
        p.grad = gr.to("mojo")
    norms = torch._foreach_norm([p.grad for p in ps])
    stacked = torch.stack(norms)
    assert stacked._ptr == norms[0]._ptr and stacked._holder is norms[0]._holder
    assert torch.allclose(stacked.cpu(), torch.stack([gr.norm() for gr in grads]), rtol=1e-6)
    again = torch.stack(norms)  # the mark is spent: a copy
    assert again._holder is not stacked._holder
    assert torch.equal(again.cpu(), stacked.cpu())
    total = torch.nn.utils.clip_grad_norm_(ps, 1.0)
    ref = [gr.clone().requires_grad_() for gr in grads]
    cpu_ps = [torch.zeros(s, requires_grad=True) for s in shapes]
    for p, gr in zip(cpu_ps, ref):
        p.grad = gr.detach().clone()
    ref_total = torch.nn.utils.clip_grad_norm_(cpu_ps, 1.0)
    assert torch.allclose(total.cpu(), ref_total, rtol=1e-6)
    for p, q in zip(ps, cpu_ps):
        assert torch.allclose(p.grad.cpu(), q.grad, rtol=1e-5, atol=1e-7)


def test_adamw_parameter_copies_are_aligned_slices(mojo):
    """The bf16 parameter copies that one fused AdamW call writes are slices
    of one allocation, each 256-byte aligned, and equal to the cast of the
    updated parameter."""
    from torch_mojo_backend.eager_kernels import aten_fast

    torch.manual_seed(1)
    model = torch.nn.Sequential(torch.nn.Linear(16, 33), torch.nn.Linear(33, 8)).to("mojo")
    opt = torch.optim.AdamW(model.parameters(), lr=1e-2, fused=True)
    x = torch.randn(4, 16).to("mojo")
    with torch.autocast("mojo", dtype=torch.bfloat16):
        out = model(x)
    out.float().sum().backward()
    opt.step()
    copies = [p.__dict__.get(aten_fast._PARAM_LOW_ATTR) for p in model.parameters()]
    assert all(c is not None for c in copies)
    holders = {id(c[0]._holder) for c in copies}
    assert len(holders) == 1
    for p, c in zip(model.parameters(), copies):
        # 256-byte aligned within the allocation (whose base the device
        # allocator aligns; the host stand-in's may not be)
        assert (c[0]._ptr - c[0]._holder.data_ptr()) % 256 == 0
        assert torch.equal(c[0].cpu(), p.detach().cpu().bfloat16())


def test_held_back_gradient_sum_becomes_the_leaf_grad_without_a_copy(mojo):
    """A parameter used twice gets the sum of its two gradients; that sum is
    a held-back add (large f32, same shape).  The record keeps only the
    storages, so autograd takes the sum as .grad as is (no clone) and the
    value matches torch."""
    from torch_mojo_backend.mojo_device import dispatch as D

    g = torch.Generator().manual_seed(6)
    w = torch.randn(512, 256, generator=g)
    x, z = torch.randn(8, 256, generator=g), torch.randn(8, 256, generator=g)
    wm = w.to("mojo").requires_grad_()
    seen = []
    orig = D.dispatch

    def spy(func, args, kwargs):
        seen.append(str(func))
        return orig(func, args, kwargs)

    D.dispatch = spy
    try:
        ((x.to("mojo") @ wm.t()).sum() + (z.to("mojo") @ wm.t() * 2.0).sum()).backward()
    finally:
        D.dispatch = orig
    wc = w.clone().requires_grad_()
    ((x @ wc.t()).sum() + (z @ wc.t() * 2.0).sum()).backward()
    assert torch.allclose(wm.grad.cpu(), wc.grad, atol=1e-5, rtol=1e-5)
    assert "aten.copy_.default" not in seen, seen
