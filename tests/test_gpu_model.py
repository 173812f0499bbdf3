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
        assert torch.allclose(a.grad.float().cpu(), b.grad, atol=2e-2, rtol=2e-2), (a.grad.float().cpu() - b.grad).abs().max()


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
    """bf16 autocast on the device against the f32 CPU
    curve.

    tests/golden/loss_envelope_b16_t1024_bf16_torch.json holds stock
    PyTorch-ROCm bf16-autocast runs of the same seed: unperturbed, and with
    the initial weights scaled by 1 + 1e-6 N(0,1) under twelve seeds.  All
    thirteen stay within 1% of the f32 curve up to step 31; from step 32 on
    the two-batch memorisation run amplifies bf16 rounding noise and the
    realisations spread to 1-3.8% (the unperturbed one happens to stay
    within 0.93%).  Which realisation a run follows is set by last-bit
    differences (summation order, exp rounding), so the device is held to:
      - within 0.1% of f32 on steps 0-4 (before the first loss spike);
      - within 1% of f32 on steps 0-31, where every stock realisation is;
      - on steps 32-49, within 1% (of the f32 loss) of the stock
        realisations' range joined with the f32 loss."""
    import json
    from pathlib import Path

    env = json.loads((Path(__file__).parent / "golden" / "loss_envelope_b16_t1024_bf16_torch.json").read_text())
    got, ref = _loss_curve(amp=True)
    assert all(math.isfinite(v) for v in got)
    rel = [abs(a - b) / abs(b) for a, b in zip(got, ref)]
    per_step = [round(r, 5) for r in rel]
    curves = list(env["curves"].values())
    stock_max = [max(abs(c[i] - ref[i]) / ref[i] for c in curves) for i in range(len(ref))]
    tight = [i for i in range(len(ref)) if max(stock_max[:i + 1]) <= 1e-2]
    assert tight == list(range(32)), tight
    assert max(rel[:5]) <= 1e-3, per_step
    bad = [(i, round(got[i], 4), round(ref[i], 4)) for i in tight if rel[i] > 1e-2]
    assert not bad, f"steps more than 1% from the f32 CPU curve (step, device, f32): {bad}; per step {per_step}"
    bad = []
    for i in range(len(tight), len(ref)):
        g, f, lo, hi = got[i], ref[i], env["lo"][i], env["hi"][i]
        if not (min(lo, f) - 0.01 * f <= g <= max(hi, f) + 0.01 * f):
            bad.append((i, round(g, 4), round(f, 4), round(lo, 4), round(hi, 4)))
    assert not bad, f"steps more than 1% outside the stock-torch bf16 range (step, dev, f32, lo, hi): {bad}"


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


def test_gemma_full_width_prefill_matches_cpu(mojo):
    """Gemma-3-1B's real layer shapes at its benchmarked length: hidden 1152,
    4 query heads on 1 K/V head of head_dim 256, GeGLU 6912, window 512,
    T = 4096, with six layers (five sliding-window, one global) and a 4096
    vocabulary so the f32 CPU reference stays cheap.  Device bf16 against
    the same bf16-rounded weights in f32 on the CPU."""
    from torch_mojo_backend.gemma3 import Gemma3, Gemma3Config

    cfg = Gemma3Config(vocab_size=4096, layers=6)
    torch.manual_seed(0)
    ref = Gemma3(cfg)
    for _, prm in ref.named_parameters():
        if prm.dim() == 1:
            torch.nn.init.normal_(prm, std=0.1)
    ref = ref.to(torch.bfloat16).float()
    model = Gemma3(cfg)
    model.load_state_dict(ref.state_dict())
    model = model.to(torch.bfloat16).to("mojo")
    idx = torch.randint(0, cfg.vocab_size, (1, 4096), generator=torch.Generator().manual_seed(3))
    with torch.no_grad():
        got = model(idx.to("mojo")).float().cpu()
        want = ref(idx)
    err = (got - want).abs().max().item()
    assert err <= 5e-2 * want.abs().max().item() + 5e-2, (err, want.abs().max().item())


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


@pytest.mark.parametrize("dtype,d", [(torch.float32, 64), (torch.bfloat16, 256), (torch.float32, 80)])
def test_sdpa_autograd_f32_and_wide_heads_use_the_flash_pair(mojo, dtype, d):
    """f32 inputs and head_dims beyond the MFMA backward's (the fused gate
    takes f32 and head_dim up to 256, aten_fast.py:7462-7530) go through the
    flash pair, not the decomposition, and match torch CPU autograd."""
    g = torch.Generator().manual_seed(d)
    q, k, v = (torch.randn(2, 3, 77, d, generator=g).to(dtype) for _ in range(3))
    qm, km, vm = (t.to("mojo").requires_grad_() for t in (q, k, v))
    out = F.scaled_dot_product_attention(qm, km, vm, is_causal=True)
    assert type(out.grad_fn).__name__ == "ScaledDotProductFlashAttentionBackward0"
    dout = torch.randn(out.shape, generator=g).to(dtype)
    out.backward(dout.to("mojo"))
    qc, kc, vc = (t.double().requires_grad_() for t in (q, k, v))
    ref = F.scaled_dot_product_attention(qc, kc, vc, is_causal=True)
    ref.backward(dout.double())
    tol = 1e-4 if dtype == torch.float32 else 2e-2
    assert torch.allclose(out.detach().double().cpu(), ref.detach(), atol=tol, rtol=tol)
    for a, b in ((qm, qc), (km, kc), (vm, vc)):
        assert torch.allclose(a.grad.double().cpu(), b.grad, atol=tol, rtol=tol), (a.grad.double().cpu() - b.grad).abs().max()


@pytest.mark.parametrize("window", [0, 40])
def test_gqa_window_attention_backward_is_fused(mojo, window):
    """Gemma-3-shaped attention under autograd (4 query heads on 1 K/V head,
    head_dim 256, sliding window from torch_mojo_backend.masks): the fused
    backward (dK/dV summed over the group) matches torch CPU autograd of the
    same masked SDPA."""
    from torch_mojo_backend.masks import sliding_window_causal_mask

    g = torch.Generator().manual_seed(window + 1)
    T = 150
    q = torch.randn(1, 4, T, 256, generator=g).bfloat16()
    k, v = (torch.randn(1, 1, T, 256, generator=g).bfloat16() for _ in range(2))
    qm, km, vm = (t.to("mojo").requires_grad_() for t in (q, k, v))
    if window:
        mask = sliding_window_causal_mask(T, window, device="mojo")
        out = F.scaled_dot_product_attention(qm, km, vm, attn_mask=mask, enable_gqa=True)
    else:
        out = F.scaled_dot_product_attention(qm, km, vm, is_causal=True, enable_gqa=True)
    assert type(out.grad_fn).__name__ == "_FusedAttentionBackward"
    dout = torch.randn(out.shape, generator=g).bfloat16()
    out.backward(dout.to("mojo"))
    qc, kc, vc = (t.double().requires_grad_() for t in (q, k, v))
    i, j = torch.arange(T)[:, None], torch.arange(T)[None, :]
    keep = (j <= i) & ((i - j < window) if window else True)
    ref = F.scaled_dot_product_attention(qc, kc, vc, attn_mask=keep, enable_gqa=True)
    ref.backward(dout.double())
    assert torch.allclose(out.detach().double().cpu(), ref.detach(), atol=2e-2, rtol=2e-2)
    for a, b in ((qm, qc), (km, kc), (vm, vc)):
        assert a.grad.shape == b.grad.shape
        assert torch.allclose(a.grad.double().cpu(), b.grad, atol=2e-2, rtol=2e-2), (a.grad.double().cpu() - b.grad).abs().max()


@pytest.mark.parametrize("causal", [False, True])
def test_flash_attention_pair_return_contract(mojo, causal):
    """The ATen flash pair called directly on mojo tensors: the forward's
    9-tuple (out, lse f32 [B,H,Sq], None, None, Sq, Sk, rng_state, unused,
    debug mask), its lse against the log-sum-exp of the scaled scores, and
    the backward's (dq, dk, dv) against torch CPU autograd
    (reference aten_fast.py:7726-7734)."""
    g = torch.Generator().manual_seed(7 + causal)
    B, H, S, D = 2, 3, 70, 64
    q, k, v = (torch.randn(B, H, S, D, generator=g).bfloat16() for _ in range(3))
    qm, km, vm = (t.to("mojo") for t in (q, k, v))
    res = torch.ops.aten._scaled_dot_product_flash_attention(qm, km, vm, 0.0, causal)
    assert len(res) == 9
    out, lse, cq, ck, mq, mk, seed, offset, dbg = res
    assert cq is None and ck is None
    assert int(mq) == S and int(mk) == S
    assert out.shape == (B, H, S, D) and out.dtype == torch.bfloat16
    assert lse.shape == (B, H, S) and lse.dtype == torch.float32
    assert seed.numel() == 2 and offset.numel() == 0
    assert dbg.numel() == 0

    qd, kd, vd = (t.double() for t in (q, k, v))
    scores = qd @ kd.transpose(-1, -2) / math.sqrt(D)
    if causal:
        scores = scores.masked_fill(torch.ones(S, S, dtype=torch.bool).triu(1), float("-inf"))
    ref_lse = torch.logsumexp(scores, dim=-1)
    ref_out = torch.softmax(scores, dim=-1) @ vd
    assert torch.allclose(lse.double().cpu(), ref_lse, atol=2e-3, rtol=1e-3)
    assert torch.allclose(out.double().cpu(), ref_out, atol=2e-2, rtol=2e-2)

    dout = torch.randn(B, H, S, D, generator=g).bfloat16()
    dq, dk, dv = torch.ops.aten._scaled_dot_product_flash_attention_backward(
        dout.to("mojo"), qm, km, vm, out, lse, cq, ck, S, S, 0.0, causal, seed, offset)
    qc, kc, vc = (t.double().requires_grad_() for t in (q, k, v))
    ref = F.scaled_dot_product_attention(qc, kc, vc, is_causal=causal)
    ref.backward(dout.double())
    for a, b in ((dq, qc), (dk, kc), (dv, vc)):
        assert a.shape == b.shape and a.dtype == torch.bfloat16
        assert torch.allclose(a.double().cpu(), b.grad, atol=2e-2, rtol=2e-2), (a.double().cpu() - b.grad).abs().max()
