"""Pins for oracle/ops.py (CPU only).

Every oracle function is checked three ways, chosen so a plausible slip (a
dropped term, a flipped sign, a wrong axis or index, transposed operands)
fails at least one of them:
  golden  - the committed outputs of stock PyTorch CPU (the reference's own
            oracle) in tests/golden/golden_ops.npz;
  live    - PyTorch CPU recomputed here on other seeded inputs;
  maths   - closed forms, invariants, special cases and central finite
            differences of the oracle's own forward (for each backward).
"""

from __future__ import annotations

import math
from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import ops

G = np.load(Path(__file__).parent / "golden" / "golden_ops.npz")
F32 = dict(rtol=2e-5, atol=2e-6)  # f64 oracle vs f32 torch


def close(a, b, **kw):
    np.testing.assert_allclose(np.asarray(a, dtype=np.float64), np.asarray(b, dtype=np.float64), **(kw or F32))


def fd_grad(f, x, dy, h=1e-6):
    """Central-difference vector-Jacobian product dy . d f(x) / dx."""
    x = np.array(x, dtype=np.float64)
    g = np.zeros_like(x)
    it = np.nditer(x, flags=["multi_index"])
    for _ in it:
        i = it.multi_index
        xp, xm = x.copy(), x.copy()
        xp[i] += h
        xm[i] -= h
        g[i] = ((np.asarray(f(xp)) - np.asarray(f(xm))) * dy).sum() / (2 * h)
    return g


# ---------------------------------------------------------------- layer norm
def test_layer_norm_golden():
    y, mean, rstd = ops.layer_norm(G["ln_x"], G["ln_w"], G["ln_b"], 1e-5)
    close(y, G["ln_y"])
    close(mean.reshape(-1), G["ln_mean"].reshape(-1))
    close(rstd.reshape(-1), G["ln_rstd"].reshape(-1))
    dx, dw, db = ops.layer_norm_backward(G["ln_dy"], G["ln_x"], mean, rstd, G["ln_w"])
    close(dx, G["ln_dx"], rtol=1e-4, atol=1e-5)
    close(dw, G["ln_dw"], rtol=1e-4, atol=1e-5)
    close(db, G["ln_db"], rtol=1e-4, atol=1e-5)


def test_layer_norm_maths():
    rng = np.random.default_rng(0)
    x = rng.normal(3.0, 2.0, (4, 10))
    y, _, _ = ops.layer_norm(x, eps=0.0)
    close(y.mean(-1), 0, atol=1e-12, rtol=0)
    close((y**2).mean(-1), 1, atol=1e-12, rtol=0)  # biased variance
    g, b, dy = rng.normal(size=10), rng.normal(size=10), rng.normal(size=(4, 10))
    _, mean, rstd = ops.layer_norm(x, g, b, 1e-5)
    dx, dg, db = ops.layer_norm_backward(dy, x, mean, rstd, g)
    close(dx, fd_grad(lambda t: ops.layer_norm(t, g, b, 1e-5)[0], x, dy), rtol=1e-5, atol=1e-7)
    close(dg, fd_grad(lambda t: ops.layer_norm(x, t, b, 1e-5)[0], g, dy), rtol=1e-5, atol=1e-7)
    close(db, dy.sum(0), rtol=1e-12, atol=0)


# ---------------------------------------------------------------- GELU
@pytest.mark.parametrize("approx", ["none", "tanh"])
def test_gelu_golden(approx):
    close(ops.gelu(G[f"gelu_{approx}_x"], approx), G[f"gelu_{approx}_y"], rtol=1e-5, atol=1e-6)
    dx = ops.gelu_backward(G[f"gelu_{approx}_dy"], G[f"gelu_{approx}_x"], approx)
    close(dx, G[f"gelu_{approx}_dx"], rtol=1e-5, atol=1e-6)


def test_gelu_maths():
    # closed forms: 0.5*x*(1+erf(x/sqrt2)); Phi(1) = 0.8413447460685429
    close(ops.gelu(np.array([0.0, 1.0, -1.0])), [0.0, 0.8413447460685429, -0.15865525393145707],
          rtol=1e-15, atol=1e-15)
    close(ops.gelu(np.array([40.0, -40.0])), [40.0, 0.0], rtol=0, atol=1e-300)
    rng = np.random.default_rng(1)
    x, dy = rng.normal(0, 2, 30), rng.normal(size=30)
    for approx in ("none", "tanh"):
        close(ops.gelu_backward(dy, x, approx), fd_grad(lambda t: ops.gelu(t, approx), x, dy),
              rtol=1e-6, atol=1e-8)
    # tanh form approximates the exact one to ~1e-3
    assert np.abs(ops.gelu(x, "tanh") - ops.gelu(x)).max() < 2e-3


# ---------------------------------------------------------------- softmax
@pytest.mark.parametrize("name", ["softmax", "log_softmax"])
def test_softmax_golden(name):
    fwd = getattr(ops, name)
    bwd = getattr(ops, name + "_backward")
    y = fwd(G[f"{name}_x"])
    close(y, G[f"{name}_y"], rtol=1e-5, atol=1e-6)
    close(bwd(G[f"{name}_dy"], y), G[f"{name}_dx"], rtol=1e-5, atol=1e-6)


def test_softmax_maths():
    rng = np.random.default_rng(2)
    x = rng.normal(0, 3, (3, 7))
    close(ops.softmax(x).sum(-1), 1.0, rtol=1e-14, atol=0)
    close(ops.softmax(x + 1000.0), ops.softmax(x), rtol=1e-12, atol=0)  # shift invariance, no overflow
    close(ops.log_softmax(x), np.log(ops.softmax(x)), rtol=1e-12, atol=1e-12)
    close(ops.softmax(x, axis=0).sum(0), 1.0, rtol=1e-14, atol=0)
    dy = rng.normal(size=x.shape)
    close(ops.softmax_backward(dy, ops.softmax(x)), fd_grad(ops.softmax, x, dy), rtol=1e-6, atol=1e-8)
    close(ops.log_softmax_backward(dy, ops.log_softmax(x)), fd_grad(ops.log_softmax, x, dy),
          rtol=1e-6, atol=1e-8)


# ---------------------------------------------------------------- NLL
@pytest.mark.parametrize("red", ["mean", "sum", "none"])
@pytest.mark.parametrize("use_w", [False, True])
def test_nll_golden(red, use_w):
    tag = f"nll_{red}_{'w' if use_w else 'nw'}"
    w = G["nll_weight"] if use_w else None
    out, total = ops.nll_loss(G["nll_logp"], G["nll_target"], w, red)
    close(out, G[tag + "_out"], rtol=1e-5, atol=1e-6)
    d = ops.nll_loss_backward(G[tag + "_gout"], G["nll_logp"].shape, G["nll_target"], w, red,
                              total_weight=total)
    close(d, G[tag + "_dlogp"], rtol=1e-5, atol=1e-7)


def test_nll_maths():
    rng = np.random.default_rng(3)
    logp = ops.log_softmax(rng.normal(size=(6, 5)))
    t = np.array([0, 4, -100, 2, 2, 1])
    w = rng.uniform(0.5, 2.0, 5)
    out, total = ops.nll_loss(logp, t, w, "mean")
    num = sum(-w[c] * logp[i, c] for i, c in enumerate(t) if c != -100)
    den = sum(w[c] for c in t if c != -100)
    close(out, num / den, rtol=1e-14, atol=0)
    close(total, den, rtol=1e-14, atol=0)
    d = ops.nll_loss_backward(np.array(1.0), logp.shape, t, w, "mean", total_weight=total)
    close(d, fd_grad(lambda z: ops.nll_loss(z, t, w, "mean")[0], logp, np.array(1.0)), rtol=1e-6, atol=1e-9)
    assert (d[2] == 0).all()  # ignored row


# ---------------------------------------------------------------- embedding
def test_embedding_golden_bit_exact():
    out = ops.embedding(G["emb_weight"], G["emb_ids"])
    assert np.array_equal(out, G["emb_out"])
    dw = ops.embedding_backward_f32(G["emb_dout"], G["emb_ids"], G["emb_weight"].shape[0])
    assert dw.dtype == np.float32
    assert np.array_equal(dw, G["emb_dweight"])


def test_embedding_backward_matches_index_add_and_padding():
    rng = np.random.default_rng(4)
    ids = rng.integers(0, 9, 200)
    g = rng.normal(size=(200, 5)).astype(np.float32)
    ref = torch.zeros(9, 5).index_add_(0, torch.from_numpy(ids), torch.from_numpy(g))
    assert np.array_equal(ops.embedding_backward_f32(g, ids, 9), ref.numpy())
    dw = ops.embedding_backward_f32(g, ids, 9, padding_idx=3)
    assert (dw[3] == 0).all()
    counts = np.bincount(ids, minlength=9)
    close(ops.embedding_backward_f32(np.ones((200, 5), np.float32), ids, 9)[:, 0], counts, rtol=0, atol=0)


# ---------------------------------------------------------------- attention
@pytest.mark.parametrize("tag,causal", [("causal", True), ("full", False), ("rect", True)])
def test_sdpa_golden(tag, causal):
    q, k, v = (G[f"sdpa_{tag}_{n}"] for n in "qkv")
    o, lse = ops.sdpa_forward(q, k, v, causal=causal)
    close(o, G[f"sdpa_{tag}_o"], rtol=1e-5, atol=2e-6)
    close(lse, G[f"sdpa_{tag}_lse"], rtol=1e-5, atol=2e-6)
    dq, dk, dv = ops.sdpa_backward(G[f"sdpa_{tag}_do"], q, k, v, o, lse, causal=causal)
    for name, got in (("dq", dq), ("dk", dk), ("dv", dv)):
        close(got, G[f"sdpa_{tag}_{name}"], rtol=1e-4, atol=1e-5)


def test_sdpa_special_cases_and_brute_force():
    rng = np.random.default_rng(5)
    q, k, v = rng.normal(size=(1, 2, 6, 4)), rng.normal(size=(1, 2, 6, 4)), rng.normal(size=(1, 2, 6, 4))
    # S = 1: O = V
    o1, lse1 = ops.sdpa_forward(q[:, :, :1], k[:, :, :1], v[:, :, :1])
    close(o1, v[:, :, :1], rtol=1e-15, atol=0)
    # causal row 0 attends to key 0 only
    oc, _ = ops.sdpa_forward(q, k, v, causal=True)
    close(oc[:, :, 0], v[:, :, 0], rtol=1e-15, atol=0)
    # brute force: explicit loops, top-left causal mask, natural-log LSE
    o_bf = np.zeros_like(oc)
    lse_bf = np.zeros(oc.shape[:-1])
    for b in range(1):
        for h in range(2):
            for i in range(6):
                s = [sum(q[b, h, i, d] * k[b, h, j, d] for d in range(4)) / 2.0 for j in range(i + 1)]
                m = max(s)
                z = sum(math.exp(x - m) for x in s)
                lse_bf[b, h, i] = m + math.log(z)
                for j in range(i + 1):
                    o_bf[b, h, i] += math.exp(s[j] - m) / z * v[b, h, j]
    oc, lsec = ops.sdpa_forward(q, k, v, causal=True)
    close(oc, o_bf, rtol=1e-12, atol=1e-14)
    close(lsec, lse_bf, rtol=1e-12, atol=1e-14)


def test_sdpa_window_and_gqa_brute_force():
    """Sliding-window causal attention with grouped-query heads (the
    Gemma-3-shaped workload) against explicit loops: query head h reads K/V
    head h // g; query i sees keys max(0, i-w+1) .. i."""
    rng = np.random.default_rng(9)
    hq, hk, t, d, w = 4, 2, 9, 4, 3
    q = rng.normal(size=(1, hq, t, d))
    k, v = rng.normal(size=(1, hk, t, d)), rng.normal(size=(1, hk, t, d))
    o, lse = ops.sdpa_forward(q, k, v, causal=True, window=w)
    g = hq // hk
    for h in range(hq):
        for i in range(t):
            js = range(max(0, i - w + 1), i + 1)
            sc = [sum(q[0, h, i, x] * k[0, h // g, j, x] for x in range(d)) / 2.0 for j in js]
            m = max(sc)
            z = sum(math.exp(x - m) for x in sc)
            assert abs(lse[0, h, i] - (m + math.log(z))) < 1e-12
            want = sum(math.exp(sv - m) / z * v[0, h // g, j] for sv, j in zip(sc, js))
            close(o[0, h, i], want, rtol=1e-12, atol=1e-14)
    # window >= T is plain causal attention; window 1 leaves only the diagonal: O = V
    oc, lc = ops.sdpa_forward(q, k, v, causal=True)
    ow, lw = ops.sdpa_forward(q, k, v, causal=True, window=t)
    close(ow, oc, rtol=0, atol=0)
    o1, _ = ops.sdpa_forward(q, k, v, causal=True, window=1)
    close(o1, np.repeat(v, g, axis=1), rtol=1e-15, atol=0)


def test_rms_norm_matches_torch_and_invariants():
    import torch

    rng = np.random.default_rng(10)
    x, w = rng.normal(size=(5, 48)) * 3.0, rng.normal(size=48)
    y, rstd = ops.rms_norm(x, w, eps=1e-6)
    ref = torch.nn.functional.rms_norm(torch.from_numpy(x), (48,), torch.from_numpy(w), eps=1e-6).numpy()
    close(y, ref, rtol=1e-12, atol=1e-12)
    # unit weight: every row has root-mean-square sqrt(ms/(ms+eps)); scale invariance up to eps
    y1, _ = ops.rms_norm(x, None, eps=1e-6)
    ms = (x * x).mean(-1)
    close(np.sqrt((y1 * y1).mean(-1)), np.sqrt(ms / (ms + 1e-6)), rtol=1e-12, atol=0)
    y2, _ = ops.rms_norm(x * 7.0, None, eps=0.0)
    y3, _ = ops.rms_norm(x, None, eps=0.0)
    close(y2, y3, rtol=1e-12, atol=1e-14)
    close(rstd, 1.0 / np.sqrt(ms + 1e-6), rtol=1e-14, atol=0)


def test_rms_norm_backward_finite_differences_and_invariants():
    """dx and dweight of rms_norm (scale weight + offset) against central
    finite differences of the oracle forward; with eps = 0 the forward is
    invariant to scaling x, so dx is orthogonal to x in every row."""
    rng = np.random.default_rng(11)
    x, w, dy = rng.normal(size=(4, 12)) * 2.0, rng.normal(size=12) * 0.3, rng.normal(size=(4, 12))
    dx, dw = ops.rms_norm_backward(dy, x, w, eps=1e-6, weight_offset=1.0)
    close(dx, fd_grad(lambda t: ops.rms_norm(t, w + 1.0, eps=1e-6)[0], x, dy), rtol=1e-6, atol=1e-8)
    close(dw, fd_grad(lambda t: ops.rms_norm(x, t + 1.0, eps=1e-6)[0], w, dy), rtol=1e-6, atol=1e-8)
    dx0, _ = ops.rms_norm_backward(dy, x, w, eps=0.0)
    close((dx0 * x).sum(-1), np.zeros(4), rtol=0, atol=1e-12)


def test_sdpa_backward_finite_differences():
    rng = np.random.default_rng(6)
    shp = (1, 1, 4, 3)
    q, k, v, do = (rng.normal(size=shp) for _ in range(4))
    for causal in (False, True):
        o, lse = ops.sdpa_forward(q, k, v, causal=causal)
        dq, dk, dv = ops.sdpa_backward(do, q, k, v, o, lse, causal=causal)
        close(dq, fd_grad(lambda t: ops.sdpa_forward(t, k, v, causal=causal)[0], q, do), rtol=1e-6, atol=1e-8)
        close(dk, fd_grad(lambda t: ops.sdpa_forward(q, t, v, causal=causal)[0], k, do), rtol=1e-6, atol=1e-8)
        close(dv, fd_grad(lambda t: ops.sdpa_forward(q, k, t, causal=causal)[0], v, do), rtol=1e-6, atol=1e-8)


def test_sdpa_backward_window_and_grouped_heads():
    """Backward with a sliding window and grouped K/V heads: finite
    differences of the forward (so dK/dV must sum each group's query heads
    and the window must mask the same keys as the forward), plus torch CPU
    autograd through SDPA with the equivalent boolean mask and enable_gqa."""
    rng = np.random.default_rng(8)
    q, do = rng.normal(size=(1, 4, 6, 3)), rng.normal(size=(1, 4, 6, 3))
    k, v = rng.normal(size=(1, 2, 6, 3)), rng.normal(size=(1, 2, 6, 3))
    for w in (0, 2, 4):
        f = lambda qq, kk, vv: ops.sdpa_forward(qq, kk, vv, causal=True, window=w)[0]  # noqa: E731
        o, lse = ops.sdpa_forward(q, k, v, causal=True, window=w)
        dq, dk, dv = ops.sdpa_backward(do, q, k, v, o, lse, causal=True, window=w)
        assert dk.shape == k.shape and dv.shape == v.shape
        close(dq, fd_grad(lambda t: f(t, k, v), q, do), rtol=1e-6, atol=1e-8)
        close(dk, fd_grad(lambda t: f(q, t, v), k, do), rtol=1e-6, atol=1e-8)
        close(dv, fd_grad(lambda t: f(q, k, t), v, do), rtol=1e-6, atol=1e-8)
        tq, tk, tv = (torch.tensor(a, requires_grad=True) for a in (q, k, v))
        i, j = torch.arange(6)[:, None], torch.arange(6)[None, :]
        keep = (j <= i) & ((i - j < w) if w else True)
        out = F.scaled_dot_product_attention(tq, tk, tv, attn_mask=keep, enable_gqa=True)
        out.backward(torch.tensor(do))
        close(dq, tq.grad.numpy(), rtol=1e-10, atol=1e-12)
        close(dk, tk.grad.numpy(), rtol=1e-10, atol=1e-12)
        close(dv, tv.grad.numpy(), rtol=1e-10, atol=1e-12)


def test_sdpa_live_torch_rect_top_left():
    g = torch.Generator().manual_seed(7)
    q, k, v = torch.randn(2, 2, 5, 3, generator=g), torch.randn(2, 2, 7, 3, generator=g), torch.randn(2, 2, 7, 3, generator=g)
    ref = F.scaled_dot_product_attention(q.double(), k.double(), v.double(), is_causal=True)
    o, _ = ops.sdpa_forward(q.numpy(), k.numpy(), v.numpy(), causal=True)
    close(o, ref.numpy(), rtol=1e-12, atol=1e-13)


# ---------------------------------------------------------------- GEMM
def test_addmm_golden_and_exact_integers():
    close(ops.addmm(G["addmm_a"], G["addmm_b"], G["addmm_bias"]), G["addmm_out"], rtol=1e-5, atol=2e-6)
    a = np.arange(6).reshape(2, 3)
    b = np.arange(12).reshape(3, 4) - 5
    exp = np.array([[sum(a[i, t] * b[t, j] for t in range(3)) + j for j in range(4)] for i in range(2)])
    assert np.array_equal(ops.addmm(a, b, np.arange(4)), exp)  # rows x cols, not transposed


# ---------------------------------------------------------------- AdamW
def test_adamw_golden_two_steps():
    p, m, v = G["adamw_p0"], np.zeros(40), np.zeros(40)
    for i in range(2):
        p, m, v = ops.adamw_step(p, G[f"adamw_g{i}"], m, v, i + 1, 6e-4, 0.9, 0.95, 0.1, 1e-8)
        close(p, G[f"adamw_p{i + 1}"], rtol=1e-6, atol=1e-7)
    close(m, G["adamw_m2"], rtol=1e-6, atol=1e-9)
    close(v, G["adamw_v2"], rtol=1e-6, atol=1e-10)


def test_adamw_maths_and_torch_variants():
    # step 1 from zero state: p <- p(1 - lr wd) - lr g / (|g| + eps)
    p, g = np.array([1.0, -2.0, 0.5]), np.array([0.3, -0.01, 2.0])
    got, _, _ = ops.adamw_step(p, g, np.zeros(3), np.zeros(3), 1, 1e-2, 0.9, 0.999, 0.1, 1e-8)
    close(got, p * (1 - 1e-3) - 1e-2 * g / (np.abs(g) + 1e-8), rtol=1e-12, atol=1e-15)
    # amsgrad + maximize against torch CPU (foreach=False), three steps
    rng = np.random.default_rng(8)
    p0 = rng.normal(size=16)
    tp = torch.tensor(p0, requires_grad=True)
    opt = torch.optim.AdamW([tp], lr=1e-3, betas=(0.8, 0.9), weight_decay=0.05, eps=1e-6, amsgrad=True,
                            maximize=True, foreach=False)
    p, m, v, vmax = p0, np.zeros(16), np.zeros(16), np.zeros(16)
    for s in range(1, 4):
        g = rng.normal(size=16)
        tp.grad = torch.tensor(g)
        opt.step()
        p, m, v, vmax = ops.adamw_step(p, g, m, v, s, 1e-3, 0.8, 0.9, 0.05, 1e-6, maximize=True, amsgrad=True,
                                       vmax=vmax)
    close(p, tp.detach().numpy(), rtol=1e-12, atol=1e-14)
    # weight decay off with a non-finite param stays non-finite without NaN from 0*inf
    q, _, _ = ops.adamw_step(np.array([np.inf]), np.array([1.0]), np.zeros(1), np.zeros(1), 1, 1e-3, 0.9, 0.99,
                             0.0, 1e-8)
    assert np.isinf(q[0])


# ---------------------------------------------------------------- norm
def test_l2_norm_golden_and_closed_form():
    tot = math.sqrt(ops.l2_norm(G["norm_t1"]) ** 2 + ops.l2_norm(G["norm_t2"]) ** 2)
    close(tot, G["norm_total"], rtol=1e-6, atol=0)
    assert ops.l2_norm(np.array([3.0, 4.0])) == 5.0
