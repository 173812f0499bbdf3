"""The mojo device end to end on the GPU: ops through `model.to("mojo")`,
compared with stock PyTorch CPU f32 (the reference's oracle)."""

import math

import pytest
import torch
import torch.nn.functional as F

from torch_mojo_backend.eager_kernels import aten_fast
from torch_mojo_backend.gpt2 import BETAS, LEARNING_RATE, WEIGHT_DECAY, GPT, GPTConfig, make_batches, training_step

pytestmark = pytest.mark.gpu


def test_device_basics(mojo):
    x = torch.randn(4, 8)
    xm = x.to("mojo")
    assert xm.device.type == "mojo"
    assert torch.equal((xm * 2 + 1).cpu(), x * 2 + 1)
    assert torch.equal(xm.t().contiguous().cpu(), x.t().contiguous())
    assert torch.allclose(xm.sum(0).cpu(), x.sum(0))
    assert xm[1, 2].item() == x[1, 2].item()
    assert torch.equal(torch.arange(10, device="mojo").cpu(), torch.arange(10))


def test_sdpa_autograd_uses_fused_kernels(mojo):
    B, H, T, D = 2, 4, 256, 64
    g = torch.Generator().manual_seed(0)
    q, k, v = (torch.randn(B, H, T, D, generator=g) for _ in range(3))
    qm, km, vm = (t.to("mojo").bfloat16().requires_grad_() for t in (q, k, v))
    out = F.scaled_dot_product_attention(qm, km, vm, is_causal=True)
    out.float().sum().backward()
    qc, kc, vc = (t.bfloat16().float().requires_grad_() for t in (q, k, v))
    ref = F.scaled_dot_product_attention(qc, kc, vc, is_causal=True)
    ref.sum().backward()
    assert torch.allclose(out.float().cpu(), ref, atol=2e-2, rtol=2e-2)
    for a, b in ((qm, qc), (km, kc), (vm, vc)):
        assert torch.allclose(a.grad.float().cpu(), b.grad, atol=5e-2, rtol=5e-2)


def _small_cfg():
    return GPTConfig(block_size=256, vocab_size=1000, n_layer=2, n_head=4, n_embd=256)


@pytest.mark.parametrize("amp", [False, True])
def test_gpt_training_steps_match_cpu(mojo, amp):
    cfg = _small_cfg()
    torch.manual_seed(0)
    ref = GPT(cfg)
    torch.manual_seed(0)
    model = GPT(cfg)
    model.load_state_dict(ref.state_dict())
    model.to("mojo")
    assert model.lm_head.weight is model.transformer.wte.weight
    opt = model.configure_optimizers(WEIGHT_DECAY, LEARNING_RATE, BETAS, fused=True)
    ropt = ref.configure_optimizers(WEIGHT_DECAY, LEARNING_RATE, BETAS, fused=True)
    batches = make_batches(4, 256, cfg.vocab_size, 2, 7, "cpu")
    for step in range(4):
        x, y = batches[step % 2]
        lr_ = training_step(ref, ropt, x, y).item()
        lm = training_step(model, opt, x.to("mojo"), y.to("mojo"),
                           autocast_dtype=torch.bfloat16 if amp else None).item()
        tol = 1e-2 if amp else 1e-4
        assert math.isfinite(lm)
        assert abs(lm - lr_) <= tol * abs(lr_), (step, lm, lr_)
    for (name, p_ref), p_m in zip(ref.named_parameters(), model.parameters()):
        tol = 2e-2 if amp else 1e-4
        assert torch.allclose(p_m.detach().cpu(), p_ref.detach(), atol=tol, rtol=tol), name


def test_bounds_errors_surface(mojo):
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
    assert aten_fast is not None



def _loss_curve(amp):
    """The headline run (GPT-2 124M, batch 16 x 1024 uniform ids, fused AdamW,
    clip 1.0, 2 batches cycled) on the mojo device, from the same seed as the
    f32 CPU fixture in tests/golden; returns (mojo losses, fixture losses)."""
    import json
    from pathlib import Path

    fx = json.loads((Path(__file__).parent / "golden" / "loss_curve_b16_t1024_f32cpu.json").read_text())
    c = fx["config"]
    torch.manual_seed(c["seed"])
    model = GPT(GPTConfig()).to("mojo")
    opt = model.configure_optimizers(WEIGHT_DECAY, LEARNING_RATE, BETAS, fused=True)
    batches = [(x.to("mojo"), y.to("mojo"))
               for x, y in make_batches(c["batch"], c["block"], c["vocab"], c["batches_cycled"],
                                        c["data_seed"], "cpu")]
    losses = []
    for step in range(len(fx["losses"])):
        x, y = batches[step % len(batches)]
        losses.append(training_step(model, opt, x, y,
                                    autocast_dtype=torch.bfloat16 if amp else None).item())
    return losses, fx["losses"]


def test_nanogpt_loss_curve_f32_matches_cpu_fixture(mojo):
    """f32 on the device: every one of the 50 steps within 1% relative of the
    f32 CPU curve (measured: within 0.2%)."""
    got, ref = _loss_curve(amp=False)
    rel = [abs(a - b) / abs(b) for a, b in zip(got, ref)]
    assert max(rel) <= 1e-2, max(enumerate(rel), key=lambda t: t[1])


def test_nanogpt_loss_curve_bf16_autocast_tracks_cpu_fixture(mojo):
    """bf16 autocast: within 0.1% relative of the f32 curve on every step
    before the run's first loss spike (steps 0-4), and within 5% on every
    one of the 50 steps (no divergence, no NaN).

    From the spike at step 5 on, this 2-batch memorisation run amplifies
    rounding noise: with the initial weights scaled by (1 + 1e-6 N(0,1))
    under six seeds, stock torch-ROCm bf16 autocast lands up to 3.4% from
    the f32 curve and the device up to 4.6%, in either direction; which
    realisation a run follows depends on last-bit differences (summation
    order, exp rounding), so a tighter per-step bound there would test the
    seed.  Kernel parity is pinned by the f32 curve test above and by the
    per-op parity tests; the device's per-parameter gradient error against
    f32 equals torch's bf16 error at init and at step 7."""
    got, ref = _loss_curve(amp=True)
    rel = [abs(a - b) / abs(b) for a, b in zip(got, ref)]
    assert all(math.isfinite(v) for v in got)
    assert max(rel[:5]) <= 1e-3, max(enumerate(rel[:5]), key=lambda t: t[1])
    assert max(rel) <= 5e-2, max(enumerate(rel), key=lambda t: t[1])


@pytest.mark.parametrize("shape,bias,strided", [((96, 200), True, False), ((3, 70, 200), True, False),
                                                 ((3, 70, 200), False, True)])
def test_fused_linear_under_autocast_gpu(mojo, shape, bias, strided):
    """Autocast linear on the device (one fused autograd Function) against
    torch CPU with autocast's rounding points (bf16 operands, f32
    accumulation, bf16 results widened to f32 gradients)."""
    from test_host_device import _linear_autocast_reference

    g = torch.Generator().manual_seed(12)
    x = torch.randn(*shape, generator=g)
    if strided:
        x = torch.randn(*shape[:-1], 232, generator=g)[..., 16:216]
    w = torch.randn(136, 200, generator=g) * 0.1
    b = torch.randn(136, generator=g) if bias else None
    dy = torch.randn(*shape[:-1], 136, generator=g)
    xm = x.to("mojo").requires_grad_()
    wm = w.to("mojo").requires_grad_()
    bm = b.to("mojo").requires_grad_() if bias else None
    with torch.autocast("mojo", dtype=torch.bfloat16):
        out = F.linear(xm, wm, bm)
    assert type(out.grad_fn).__name__ == "_FusedLinearBackward"
    out.backward(dy.bfloat16().to("mojo"))
    eo, edx, edw, edb = _linear_autocast_reference(x, w, b, dy)
    assert torch.allclose(out.float().cpu(), eo.float(), atol=2e-2, rtol=2e-2)
    assert torch.allclose(xm.grad.cpu(), edx, atol=2e-2, rtol=2e-2)
    assert torch.allclose(wm.grad.cpu(), edw, atol=5e-2, rtol=2e-2)
    if bias:
        assert torch.allclose(bm.grad.cpu(), edb, atol=5e-2, rtol=2e-2)


def test_gemma_shaped_prefill_matches_cpu(mojo):
    """Gemma-3-shaped prefill (grouped-query windowed and global attention at
    head_dim 256, RMSNorm, GeGLU, RoPE) in bf16 on the device against the same
    bf16-rounded weights in f32 on the CPU."""
    from torch_mojo_backend.gemma3 import Gemma3, Gemma3Config

    cfg = Gemma3Config(vocab_size=512, hidden=256, layers=4, heads=4, kv_heads=1, head_dim=256, d_ff=512,
                       window=40, global_every=2)
    torch.manual_seed(0)
    ref = Gemma3(cfg)
    for _, prm in ref.named_parameters():
        if prm.dim() == 1:
            torch.nn.init.normal_(prm, std=0.1)
    ref = ref.to(torch.bfloat16).float()
    model = Gemma3(cfg)
    model.load_state_dict(ref.state_dict())
    model = model.to(torch.bfloat16).to("mojo")
    idx = torch.randint(0, cfg.vocab_size, (1, 200), generator=torch.Generator().manual_seed(2))
    with torch.no_grad():
        got = model(idx.to("mojo")).float().cpu()
        want = ref(idx)
    err = (got - want).abs().max().item()
    assert err <= 5e-2 * want.abs().max().item() + 5e-2, err


@pytest.mark.parametrize("dtype,bits", [(torch.float32, torch.int32), (torch.bfloat16, torch.int16)])
def test_stack_and_cat_of_many_pieces_are_bit_exact(mojo, dtype, bits):
    """stack/cat of many contiguous pieces (clip_grad_norm_ stacks one norm
    per parameter) run as one multi-tensor launch; signed zeros, NaN,
    infinities and subnormals must come through bit for bit."""
    vals = torch.tensor([0.0, -0.0, float("nan"), float("inf"), -float("inf"), 1e-40, -3.5, 2.0 ** 100] * 3)
    pieces = [v.clone().to(dtype) for v in vals]
    got = torch.stack([x.to("mojo") for x in pieces]).cpu()
    assert torch.equal(got.view(bits), torch.stack(pieces).view(bits))
    rows = [torch.randn(5 + i).to(dtype) for i in range(10)]
    rows[3][2] = -0.0
    got = torch.cat([r.to("mojo") for r in rows]).cpu()
    assert torch.equal(got.view(bits), torch.cat(rows).view(bits))
