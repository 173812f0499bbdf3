"""Parity at the BASELINE configs' real sizes, through the C ABI.

Config 1 (causal SDPA [8,12,1024,64] bf16): O, LSE, dQ, dK and dV of three
(batch, head) slices against the f64 oracle.  The slices sit on different
XCDs of the XCD-aware block map (each XCD owns 12 consecutive (b, h) pairs
at this shape) and take different places in its heaviest-first tile order,
so the one-launch dK/dV + dQ grid is pinned where it is timed.

Config 3's HBM-bound kernels at the step's sizes: the fused cross-entropy
and the stand-alone log_softmax on bf16 logits [16384, 50257], GELU on the
fc activation [16384, 3072]; and config 4's tied lm_head GEMM (M = 4096,
N = 262144, K = 1152).

Config 2 (GEMMs at M = 16384): every (K, N) of the sweep, in the three
launches of a linear layer as the autocast model issues them -- forward
x W^T + b (bf16 out), dX = dY W (f32 out rounded to bf16), dW = dY^T X (f32
out rounded to bf16) with the bias gradient as the row sums of dY^T -- each
against the f64 oracle on sampled rows that cross every row tile and every
column of the output, so each tile plan (tile size, split-K count) the
planner picks at these shapes is checked.
"""

import math

import numpy as np
import pytest
import torch

from abi import CODE, bhs, call, dev, host, lib, np64, p, tol_close, workspace  # noqa: F401
from oracle import ops as O
from test_gpu_gemm_attention import _attn_bwd, _attn_fwd

pytestmark = pytest.mark.gpu


def test_attention_cfg1_slices_match_oracle(kernels):
    B, H, S, D = 8, 12, 1024, 64
    g = torch.Generator().manual_seed(101)
    q, k, v, do = (torch.randn(B, H, S, D, generator=g).bfloat16() for _ in range(4))
    tq, tk, tv, tdo = dev(q), dev(k), dev(v), dev(do)
    o, lse = _attn_fwd(tq, tk, tv, True)
    dq, dk, dv = _attn_bwd(tdo, tq, tk, tv, o, lse, True)
    got = {name: host(t) for name, t in (("o", o), ("lse", lse), ("dq", dq), ("dk", dk), ("dv", dv))}
    for b, h in ((0, 0), (4, 5), (7, 11)):  # pairs 0, 53, 95: XCDs 0, 4, 7
        sl = (slice(b, b + 1), slice(h, h + 1))
        qs, ks, vs, dos = (t[sl].double().numpy() for t in (q, k, v, do))
        eo, el = O.sdpa_forward(qs, ks, vs, causal=True)
        what = f"cfg1 b{b} h{h}"
        tol_close(got["o"][sl].double().numpy(), eo, atol=2e-2, rtol=2e-2, what=f"O {what}")
        tol_close(got["lse"][sl].double().numpy(), el, atol=1e-3, rtol=1e-3, what=f"LSE {what}")
        # backward from the device's own O and LSE, as the autograd pair runs it
        edq, edk, edv = O.sdpa_backward(dos, qs, ks, vs, got["o"][sl].double().numpy(),
                                        got["lse"][sl].double().numpy(), causal=True)
        tol_close(got["dv"][sl].double().numpy(), edv, atol=2e-2, rtol=2e-2, what=f"dV {what}")
        tol_close(got["dk"][sl].double().numpy(), edk, atol=2e-2, rtol=2e-2, what=f"dK {what}")
        tol_close(got["dq"][sl].double().numpy(), edq, atol=2e-2, rtol=2e-2, what=f"dQ {what}")


def _gemm_ex(c, c_rs, a, ars, acs, b, brs, bcs, m, n, k, bias=None, flags=0, rowsum=None):
    ws_n = lib().mi355x_gemm_workspace_bytes(p(a), ars, acs, 0, p(b), brs, bcs, 0, CODE[torch.bfloat16], 1, m, n, k)
    ws = workspace(ws_n) if ws_n else None
    call("mi355x_gemm_ex", p(c), CODE[c.dtype], c_rs, 0, p(a), ars, acs, 0, p(b), brs, bcs, 0,
         CODE[torch.bfloat16], p(bias), CODE[bias.dtype] if bias is not None else 0, flags,
         p(rowsum), CODE[torch.float32] if rowsum is not None else 0, 1, m, n, k, p(ws), ws_n, None)


def _rows(total, step):
    r = np.arange(0, total, step)
    return np.unique(np.concatenate([r, [total - 1]]))


@pytest.mark.parametrize("K,N", [(768, 2304), (768, 768), (768, 3072), (3072, 768), (768, 50304)])
def test_gemm_cfg2_linear_launches_match_oracle(kernels, K, N):
    M = 16384
    g = torch.Generator().manual_seed(K * 7 + N)
    X = torch.randn(M, K, generator=g).bfloat16()
    W = (torch.randn(N, K, generator=g) * 0.02).bfloat16()
    bias = (torch.randn(N, generator=g) * 0.02).bfloat16()
    dY = torch.randn(M, N, generator=g).bfloat16()
    tx, tw, tb, tdy = dev(X), dev(W), dev(bias), dev(dY)
    rows = _rows(M, 41)  # 401 rows: every 128- and 256-row tile, at varying offsets
    Xr, Wd, dYr = X[rows].double().numpy(), W.double().numpy(), dY[rows].double().numpy()

    # forward: y = x W^T + b, B = W^T read in place (k-contiguous)
    y = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    _gemm_ex(y, N, tx, K, 1, tw, 1, K, M, N, K, bias=tb)
    tol_close(host(y[rows]).double().numpy(), O.addmm(Xr, Wd.T, bias.double().numpy()),
              atol=2e-2, rtol=2e-2, what=f"fwd {K}->{N}")
    del y

    # dX = dY W, f32 out holding bf16-rounded values
    dx = torch.empty(M, K, dtype=torch.float32, device="cuda")
    _gemm_ex(dx, K, tdy, N, 1, tw, K, 1, M, K, N, flags=2)
    got = host(dx[rows])
    assert torch.equal(got, got.bfloat16().float())
    tol_close(got.double().numpy(), O.addmm(dYr, Wd), atol=2e-2, rtol=2e-2, what=f"dX {K}->{N}")
    del dx

    # dW = dY^T X (A = dY^T: m-contiguous), db = row sums of dY^T
    dw = torch.empty(N, K, dtype=torch.float32, device="cuda")
    db = torch.empty(N, dtype=torch.float32, device="cuda")
    _gemm_ex(dw, K, tdy, 1, N, tx, K, 1, N, K, M, flags=2, rowsum=db)
    wrows = _rows(N, max(1, N // 256))
    got = host(dw[wrows])
    assert torch.equal(got, got.bfloat16().float())
    dyc = dY[:, wrows].double().numpy()
    tol_close(got.double().numpy(), O.addmm(dyc.T, X.double().numpy()), atol=5e-2, rtol=1e-2,
              what=f"dW {K}->{N}")
    tol_close(host(db).double().numpy(), dY.sum(0, dtype=torch.float64).numpy(), atol=5e-2, rtol=1e-2, what=f"db {K}->{N}")


def test_attention_gemma_shape_window_slices_match_oracle(kernels):
    """Gemma-3-1B-shaped attention at its real size: 4 query heads on one K/V
    head, head_dim 256, causal sliding window 512, T = 4096, bf16; forward
    through mi355x_attn_fwd_ex (the MFMA kernel) and backward through
    mi355x_attn_bwd_gen, as the fused autograd Function runs them.

    The f64 oracle runs on two 1024-row sub-problems that the window makes
    exact.  The prefix (rows 0..1023): top-left causal masking is the same
    there, so O, LSE and dQ of every row and dK/dV of keys 0..512 (all
    their queries are below 1024) must match.  The tail (rows 3072..4095):
    a query at local row >= 511 sees only keys inside the sub-problem, so
    O, LSE and dQ of rows 3583..4095 must match; with the device's O and
    LSE as the backward's inputs every P in the sub-problem is the full
    problem's, and every query of keys 3072..4095 lies inside, so their
    dK/dV must match too."""
    B, H, Hk, T, D, W = 1, 4, 1, 4096, 256, 512
    g = torch.Generator().manual_seed(4096)
    q, do = (torch.randn(B, H, T, D, generator=g).bfloat16() for _ in range(2))
    k, v = (torch.randn(B, Hk, T, D, generator=g).bfloat16() for _ in range(2))
    tq, tk, tv, tdo = dev(q), dev(k), dev(v), dev(do)
    scale = 1.0 / math.sqrt(D)
    o = torch.empty(B, T, H, D, dtype=torch.bfloat16, device="cuda").transpose(1, 2)
    lse = torch.empty(B, H, T, device="cuda")
    call("mi355x_attn_fwd_ex", p(o), bhs(o), p(lse), p(tq), bhs(tq), p(tk), bhs(tk), p(tv), bhs(tv),
         B, H, Hk, T, T, D, scale, 1, W, CODE[torch.bfloat16], None)
    dq = torch.empty(B, T, H, D, dtype=torch.bfloat16, device="cuda").transpose(1, 2)
    dk = torch.empty(B, T, Hk, D, dtype=torch.bfloat16, device="cuda").transpose(1, 2)
    dv = torch.empty(B, T, Hk, D, dtype=torch.bfloat16, device="cuda").transpose(1, 2)
    ws_n = lib().mi355x_attn_bwd_gen_workspace_bytes(B, H, Hk, T, T, D)
    ws = workspace(ws_n)
    call("mi355x_attn_bwd_gen", p(dq), bhs(dq), p(dk), bhs(dk), p(dv), bhs(dv), p(tdo), bhs(tdo),
         p(tq), bhs(tq), p(tk), bhs(tk), p(tv), bhs(tv), p(o), bhs(o), p(lse),
         B, H, Hk, T, T, D, scale, 1, W, CODE[torch.bfloat16], p(ws), ws_n, None)
    got = {name: host(t).double().numpy() for name, t in
           (("o", o), ("lse", lse), ("dq", dq), ("dk", dk), ("dv", dv))}
    n = lambda t: t.double().numpy()  # noqa: E731
    for s0, rows, keys in ((0, slice(0, 1024), slice(0, 513)), (3072, slice(511, 1024), slice(0, 1024))):
        sl = slice(s0, s0 + 1024)
        qs, ks, vs, dos = n(q[:, :, sl]), n(k[:, :, sl]), n(v[:, :, sl]), n(do[:, :, sl])
        eo, el = O.sdpa_forward(qs, ks, vs, causal=True, window=W)
        what = f"gemma T4096 rows {s0 + rows.start}..{s0 + rows.stop - 1}"
        tol_close(got["o"][:, :, sl][:, :, rows], eo[:, :, rows], atol=2e-2, rtol=2e-2, what=f"O {what}")
        tol_close(got["lse"][:, :, sl][:, :, rows], el[:, :, rows], atol=1e-2, rtol=1e-3, what=f"LSE {what}")
        edq, edk, edv = O.sdpa_backward(dos, qs, ks, vs, got["o"][:, :, sl], got["lse"][:, :, sl],
                                        causal=True, window=W)
        tol_close(got["dq"][:, :, sl][:, :, rows], edq[:, :, rows], atol=2e-2, rtol=2e-2, what=f"dQ {what}")
        kw = f"gemma T4096 keys {s0 + keys.start}..{s0 + keys.stop - 1}"
        tol_close(got["dk"][:, :, sl][:, :, keys], edk[:, :, keys], atol=2e-2, rtol=2e-2, what=f"dK {kw}")
        tol_close(got["dv"][:, :, sl][:, :, keys], edv[:, :, keys], atol=2e-2, rtol=2e-2, what=f"dV {kw}")


def test_cross_entropy_cfg3_logits_match_oracle(kernels):
    """Fused cross-entropy at config 3's real logits: bf16 [16384, 50257]
    (rows contiguous, 50257 columns: every row starts at another 2-byte
    phase), mean reduction, gradient rows padded to 50264 as the model
    allocates them.  The loss and every row's log-sum-exp against f64 over
    all rows; dlogits on sampled rows (every 64-row span, both ends)."""
    n, c, ld_dx = 16384, 50257, 50264
    g = torch.Generator().manual_seed(50257)
    x = (torch.randn(n, c, generator=g) * 3).bfloat16()
    tgt = torch.randint(0, c, (n,), generator=g)
    tx, tt = dev(x), dev(tgt)
    out = torch.empty((), device="cuda")
    lse = torch.empty(n, device="cuda")
    tw = torch.empty((), device="cuda")
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    ws_n = lib().mi355x_cross_entropy_workspace_bytes(n)
    ws = workspace(ws_n)
    call("mi355x_cross_entropy_fwd", p(out), p(tw), p(lse), p(tx), CODE[torch.bfloat16], c, p(tt), n, c,
         1, -100, p(err), p(ws), ws_n, None)
    # f64 log-sum-exp of every row, in chunks
    else_ = torch.empty(n, dtype=torch.float64)
    picked = torch.empty(n, dtype=torch.float64)
    for r0 in range(0, n, 1024):
        xc = x[r0:r0 + 1024].double()
        else_[r0:r0 + 1024] = torch.logsumexp(xc, 1)
        picked[r0:r0 + 1024] = xc.gather(1, tgt[r0:r0 + 1024, None])[:, 0]
    tol_close(host(lse).double().numpy(), else_.numpy(), atol=1e-4, rtol=1e-5, what="ce lse cfg3")
    eloss = float((else_ - picked).mean())
    tol_close(host(out).double().numpy(), eloss, atol=1e-4, rtol=1e-5, what="ce loss cfg3")
    assert host(tw).item() == n and host(err).item() == 0
    del tx
    tx = dev(x)
    dx = torch.empty(n, ld_dx, dtype=torch.bfloat16, device="cuda")
    gout = dev(torch.tensor(1.0))
    call("mi355x_cross_entropy_bwd", p(dx), CODE[torch.bfloat16], ld_dx, p(tx), CODE[torch.bfloat16], c, p(lse),
         p(tt), p(gout), 1, p(tw), n, c, -100, None)
    rows = _rows(n, 64)
    logp = O.log_softmax(x[rows].double().numpy())
    dnll = O.nll_loss_backward(np.float64(1.0), (len(rows), c), tgt[rows].numpy(), None, "mean", -100, n)
    edx = O.log_softmax_backward(dnll, logp)
    got = host(dx[rows]).double().numpy()
    tol_close(got[:, :c], edx, atol=1e-12, rtol=2e-2, what="ce dlogits cfg3")
    assert (got[:, c:] == 0).all()


def test_log_softmax_cfg3_logits_match_oracle(kernels):
    """Stand-alone log_softmax forward and backward at the logits' size, bf16
    [16384, 50257] (the register-resident row kernels), on sampled rows."""
    n, c = 16384, 50257
    g = torch.Generator().manual_seed(16384)
    x = (torch.randn(n, c, generator=g) * 3).bfloat16()
    tx = dev(x)
    y = torch.empty(n, c, dtype=torch.bfloat16, device="cuda")
    call("mi355x_softmax_fwd", p(y), CODE[torch.bfloat16], p(tx), CODE[torch.bfloat16], n, c, 1, None)
    rows = _rows(n, 64)
    tol_close(host(y[rows]).double().numpy(), O.log_softmax(x[rows].double().numpy()), atol=2e-2, rtol=2e-2,
              what="log_softmax cfg3")
    del tx
    dy = torch.randn(n, c, generator=g).bfloat16()
    tdy = dev(dy)
    dx = torch.empty(n, c, dtype=torch.bfloat16, device="cuda")
    call("mi355x_softmax_bwd", p(dx), CODE[torch.bfloat16], p(tdy), CODE[torch.bfloat16], p(y),
         CODE[torch.bfloat16], n, c, 1, None)
    edx = O.log_softmax_backward(dy[rows].double().numpy(), host(y[rows]).double().numpy())
    tol_close(host(dx[rows]).double().numpy(), edx, atol=2e-2, rtol=2e-2, what="log_softmax bwd cfg3")


@pytest.mark.parametrize("approx", [0, 1])
def test_gelu_cfg3_fc_activation_matches_oracle(kernels, approx):
    """GELU forward and backward on the fc activation of config 3, bf16
    [16384, 3072], every element against the f64 oracle."""
    g = torch.Generator().manual_seed(3072 + approx)
    x = (torch.randn(16384, 3072, generator=g) * 2).bfloat16()
    dy = torch.randn(16384, 3072, generator=g).bfloat16()
    tx, tdy = dev(x), dev(dy)
    n = x.numel()
    mode = "tanh" if approx else "none"
    y = torch.empty_like(tx)
    call("mi355x_gelu_fwd", p(y), p(tx), n, approx, CODE[torch.bfloat16], None)
    xd = x.double().numpy()
    tol_close(host(y).double().numpy(), O.gelu(xd, mode), atol=1e-2, rtol=1e-2, what="gelu cfg3")
    dx = torch.empty_like(tx)
    call("mi355x_gelu_bwd", p(dx), p(tdy), p(tx), n, approx, CODE[torch.bfloat16], None)
    tol_close(host(dx).double().numpy(), O.gelu_backward(dy.double().numpy(), xd, mode), atol=1e-2, rtol=1e-2,
              what="gelu bwd cfg3")


def test_gemma_tied_lm_head_gemm_matches_oracle(kernels):
    """The Gemma-3-1B prefill's largest GEMM: the tied lm_head, logits =
    x W^T with M = 4096, N = 262144, K = 1152 (2.5 TFLOP), bf16 in and out,
    W read in place; f64 oracle on sampled rows crossing every row tile,
    all 262144 columns."""
    M, N, K = 4096, 262144, 1152
    g = torch.Generator().manual_seed(262144)
    X = torch.randn(M, K, generator=g).bfloat16()
    W = (torch.randn(N, K, generator=g) * 0.02).bfloat16()
    tx, tw = dev(X), dev(W)
    y = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    _gemm_ex(y, N, tx, K, 1, tw, 1, K, M, N, K)
    rows = _rows(M, 37)
    want = X[rows].double().numpy() @ W.double().numpy().T
    tol_close(host(y[rows]).double().numpy(), want, atol=2e-2, rtol=2e-2, what="gemma lm_head")
