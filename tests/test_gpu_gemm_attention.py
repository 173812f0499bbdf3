"""GPU parity of the MFMA GEMM and fused flash attention through the C ABI.

GEMM: the oracle is the f64 product of the bf16-rounded inputs (exact up to
f64), tolerance grows with sqrt(K).  Attention: f64 oracle of the same
bf16 inputs; bf16 outputs within atol = rtol = 2e-2."""

import math

import numpy as np
import pytest
import torch

from abi import CODE, bhs, call, dev, host, i64, lib, np64, p, tol_close, workspace  # noqa: F401
from oracle import ops as O

pytestmark = pytest.mark.gpu

G = torch.Generator().manual_seed(1234)


def randn(*shape):
    return torch.randn(*shape, generator=G)


def _gemm(c, a, b, m, n, k, a_rs, a_cs, b_rs, b_cs, dt, bias=None, beta=0, batch=1, a_bs=0, b_bs=0, c_bs=0):
    ws_n = lib().mi355x_gemm_workspace_bytes(p(a), a_rs, a_cs, a_bs, p(b), b_rs, b_cs, b_bs, CODE[dt],
                                             batch, m, n, k)
    ws = workspace(ws_n) if ws_n else None
    call("mi355x_gemm", p(c), CODE[c.dtype], n if c.dim() == 2 else c.stride(-2), c_bs,
         p(a), a_rs, a_cs, a_bs, p(b), b_rs, b_cs, b_bs, CODE[dt], p(bias),
         CODE[bias.dtype] if bias is not None else 0, beta, batch, m, n, k, p(ws), ws_n, None)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("layout", ["NT", "NN", "TN", "TT"])
@pytest.mark.parametrize("mnk", [(256, 384, 768), (357, 789, 333), (1, 50, 64), (64, 1, 17), (130, 66, 1)])
def test_gemm_layouts_and_shapes(kernels, dtype, layout, mnk):
    m, n, k = mnk
    A = randn(m, k).to(dtype)
    B = randn(k, n).to(dtype) * 0.1
    bias = (randn(n) * 0.1).to(dtype)
    # A: "N" = row-major [m,k]; "T" = stored [k,m]
    if layout[0] == "N":
        ta = dev(A)
        a_rs, a_cs = k, 1
    else:
        ta = dev(A.t().contiguous())
        a_rs, a_cs = 1, m
    if layout[1] == "N":
        tb = dev(B)
        b_rs, b_cs = n, 1
    else:
        tb = dev(B.t().contiguous())
        b_rs, b_cs = 1, k
    if m == 1 and a_rs == 1:
        a_rs = k
    c = torch.empty(m, n, dtype=dtype, device="cuda")
    _gemm(c, ta, tb, m, n, k, a_rs, a_cs, b_rs, b_cs, dtype, bias=dev(bias))
    exp = O.addmm(A.double().numpy(), B.double().numpy(), bias.double().numpy())
    if dtype == torch.float32:
        tol = 1e-4 * math.sqrt(k)
    else:
        tol = 2e-2 * max(1.0, math.sqrt(k) / 16)
    tol_close(np64(c), exp, atol=tol, rtol=2e-2 if dtype != torch.float32 else 1e-4, what=f"{layout}{mnk}")


@pytest.mark.parametrize("layout", ["NT", "NN", "TN", "TT"])
def test_gemm_k_tail_on_padded_rows_in_place(kernels, layout):
    """K not a multiple of 64 and row counts not a multiple of 8, with rows
    padded to 8 elements (the lm_head backward's dlogits layout): operands are
    read in place and the K tail is masked."""
    m, n, k = 250, 196, 1001
    pad = lambda v: (v + 7) // 8 * 8  # noqa: E731
    A = randn(m, k).bfloat16()
    B = (randn(k, n) * 0.1).bfloat16()
    if layout[0] == "N":  # A stored [m][pad(k)]
        store = torch.zeros(m, pad(k), dtype=torch.bfloat16)
        store[:, :k] = A
        ta, a_rs, a_cs = dev(store), pad(k), 1
    else:  # A stored [k][pad(m)]
        store = torch.zeros(k, pad(m), dtype=torch.bfloat16)
        store[:, :m] = A.t()
        ta, a_rs, a_cs = dev(store), 1, pad(m)
    if layout[1] == "N":  # B stored [k][pad(n)]
        store = torch.zeros(k, pad(n), dtype=torch.bfloat16)
        store[:, :n] = B
        tb, b_rs, b_cs = dev(store), pad(n), 1
    else:  # B stored [n][pad(k)]
        store = torch.zeros(n, pad(k), dtype=torch.bfloat16)
        store[:, :k] = B.t()
        tb, b_rs, b_cs = dev(store), 1, pad(k)
    c = torch.empty(m, n, dtype=torch.float32, device="cuda")
    _gemm(c, ta, tb, m, n, k, a_rs, a_cs, b_rs, b_cs, torch.bfloat16)
    exp = A.double().numpy() @ B.double().numpy()
    tol_close(np64(c), exp, atol=2e-2 * math.sqrt(k / 64), rtol=1e-2, what=f"tail {layout}")


@pytest.mark.parametrize("layout", ["NT", "NN", "TN", "TT"])
def test_gemm_256_tiles_with_k_tail(kernels, layout):
    """M = N = 4096 fill 256 of the 256x256 tiles, so the planner takes them
    (their next-stage loads are spread over the MFMA rows); K = 200 ends
    inside a 64-k stage.  bf16 out, f64 oracle on sampled rows."""
    m, n, k = 4096, 4096, 200
    A = randn(m, k).bfloat16()
    B = (randn(k, n) * 0.1).bfloat16()
    ta, a_rs, a_cs = (dev(A), k, 1) if layout[0] == "N" else (dev(A.t().contiguous()), 1, m)
    tb, b_rs, b_cs = (dev(B), n, 1) if layout[1] == "N" else (dev(B.t().contiguous()), 1, k)
    c = torch.empty(m, n, dtype=torch.bfloat16, device="cuda")
    _gemm(c, ta, tb, m, n, k, a_rs, a_cs, b_rs, b_cs, torch.bfloat16)
    rows = sorted(set(list(range(0, m, 97)) + [255, 256, 511, m - 1]))
    exp = A[rows].double().numpy() @ B.double().numpy()
    tol_close(np64(c)[rows], exp, atol=2e-2, rtol=2e-2, what=f"256 tiles {layout}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_gemm_weight_gradient_tiles_split_k(kernels, dtype):
    """An m-contiguous A (a weight gradient dY^T X) with 256 or more 256x256
    tiles and a long K takes the 32-k 256x256 tiles in two K splits summed
    by a second kernel (the embedding-gradient launch): f32 out, f64 oracle
    on sampled rows."""
    m, n, k = 4096, 4352, 8192  # 16 x 17 = 272 tiles, 2.1 rounds of 256 CUs
    A = (randn(k, m) * 0.5).to(dtype)  # stored [k][m]: m-contiguous
    B = (randn(k, n) * 0.5).to(dtype)  # stored [k][n]: n-contiguous
    ta, tb = dev(A), dev(B)
    c = torch.empty(m, n, dtype=torch.float32, device="cuda")
    _gemm(c, ta, tb, m, n, k, 1, m, n, 1, dtype)
    rows = sorted(set(list(range(0, m, 211)) + [255, 256, m - 1]))
    exp = A[:, rows].double().numpy().T @ B.double().numpy()
    tol_close(np64(c)[rows], exp, atol=2e-2 * math.sqrt(k / 64), rtol=2e-2, what=f"dW split {dtype}")


def test_gemm_accumulate_and_batched(kernels):
    bsz, m, n, k = 3, 100, 72, 96
    A = randn(bsz, m, k).bfloat16()
    B = randn(bsz, k, n).bfloat16()
    C0 = randn(bsz, m, n)
    ta, tb, tc = dev(A), dev(B), dev(C0)
    ws_n = lib().mi355x_gemm_workspace_bytes(p(ta), k, 1, m * k, p(tb), n, 1, k * n, 1, bsz, m, n, k)
    ws = workspace(ws_n) if ws_n else None
    call("mi355x_gemm", p(tc), 0, n, m * n, p(ta), k, 1, m * k, p(tb), n, 1, k * n, 1, None, 0, 1,
         bsz, m, n, k, p(ws), ws_n, None)
    exp = C0.double().numpy() + np.einsum("bmk,bkn->bmn", A.double().numpy(), B.double().numpy())
    tol_close(np64(tc), exp, atol=2e-2, rtol=1e-2, what="batched beta=1")


@pytest.mark.parametrize("m,n,k", [(300, 136, 5120), (200, 136, 6144)])
def test_gemm_batched_split_k_grid_order(kernels, m, n, k):
    """Batched GEMMs with a long K take split K over several batch planes:
    the block -> (split, batch, tile) order spans the whole grid (grids of
    180 and 144 blocks, one not a multiple of the 8 XCDs), and every tile of
    every plane must come out once."""
    bsz = 3
    A = randn(bsz, m, k).bfloat16()
    B = randn(bsz, k, n).bfloat16()
    C0 = randn(bsz, m, n)
    ta, tb, tc = dev(A), dev(B), dev(C0)
    ws_n = lib().mi355x_gemm_workspace_bytes(p(ta), k, 1, m * k, p(tb), n, 1, k * n, 1, bsz, m, n, k)
    assert ws_n > 0  # the split-K partials live in the workspace
    ws = workspace(ws_n)
    call("mi355x_gemm", p(tc), 0, n, m * n, p(ta), k, 1, m * k, p(tb), n, 1, k * n, 1, None, 0, 1,
         bsz, m, n, k, p(ws), ws_n, None)
    exp = C0.double().numpy() + np.einsum("bmk,bkn->bmn", A.double().numpy(), B.double().numpy())
    tol_close(np64(tc), exp, atol=2e-2 * math.sqrt(k / 64), rtol=1e-2, what=f"batched split-K {m}x{n}x{k}")


@pytest.mark.parametrize("n,c_dtype", [(80, torch.float32), (78, torch.float32), (80, torch.bfloat16)])
def test_gemm_split_k_with_bias_and_beta(kernels, n, c_dtype):
    """Small C, long K (the weight-gradient regime) takes the split-K path:
    the 4-column reduction (n % 4 == 0) and the scalar one, f32 and bf16 C."""
    m, k = 96, 8192
    assert lib().mi355x_gemm_workspace_bytes(None, 1, m, 0, None, n, 1, 0, 1, 1, m, n, k) > 0
    A = randn(k, m).bfloat16()  # stored m-contiguous: A(m, k) = A_store[k, m]
    B = randn(k, n).bfloat16()
    bias = randn(n)
    C0 = randn(m, n).to(c_dtype)
    tc = dev(C0)
    _gemm(tc, dev(A), dev(B), m, n, k, 1, m, n, 1, torch.bfloat16, bias=dev(bias), beta=1)
    exp = C0.double().numpy() + A.double().numpy().T @ B.double().numpy() + bias.double().numpy()
    atol = 0.5 if c_dtype == torch.float32 else 1.0
    tol_close(np64(tc), exp, atol=atol, rtol=1e-2, what="split-K")


@pytest.mark.parametrize("K,N", [(768, 2304), (3072, 768)])
def test_gemm_gpt2_training_shapes(kernels, K, N):
    """fwd x W^T, dX = dY W, dW = dY^T X at M = 4096 (cfg 2 shapes, smaller M)."""
    M = 4096
    X = randn(M, K).bfloat16()
    W = (randn(N, K) * 0.02).bfloat16()
    dY = randn(M, N).bfloat16()
    tx, tw, tdy = dev(X), dev(W), dev(dY)
    y = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    _gemm(y, tx, tw, M, N, K, K, 1, 1, K, torch.bfloat16)  # B = W^T: (k, n) at n*K + k
    tol_close(np64(y), X.double().numpy() @ W.double().numpy().T, atol=2e-2, rtol=2e-2, what="fwd")
    dx = torch.empty(M, K, dtype=torch.bfloat16, device="cuda")
    _gemm(dx, tdy, tw, M, K, N, N, 1, K, 1, torch.bfloat16)
    tol_close(np64(dx), dY.double().numpy() @ W.double().numpy(), atol=3e-2, rtol=2e-2, what="dX")
    dw = torch.empty(N, K, dtype=torch.float32, device="cuda")
    _gemm(dw, tdy, tx, N, K, M, 1, N, K, 1, torch.bfloat16)  # A = dY^T: (m,k) at k*N + m
    ref = dY.double().numpy().T @ X.double().numpy()
    tol_close(np64(dw), ref, atol=0.05 * math.sqrt(M / 64), rtol=1e-2, what="dW")


# ---------------------------------------------------------------------------
# attention
# ---------------------------------------------------------------------------
def _attn_fwd(q, k, v, causal, scale=None):
    B, H, Sq, D = q.shape
    Skv = k.shape[2]
    scale = 1.0 / math.sqrt(D) if scale is None else scale
    dense = torch.empty(B, Sq, H, D, dtype=q.dtype, device="cuda")
    o = dense.transpose(1, 2)
    lse = torch.empty(B, H, Sq, device="cuda")
    call("mi355x_attn_fwd", p(o), bhs(o), p(lse), p(q), bhs(q), p(k), bhs(k), p(v), bhs(v),
         B, H, Sq, Skv, D, scale, int(causal), CODE[q.dtype], None)
    return o, lse


def _attn_bwd(do, q, k, v, o, lse, causal, scale=None):
    B, H, Sq, D = q.shape
    Skv = k.shape[2]
    scale = 1.0 / math.sqrt(D) if scale is None else scale
    dq = torch.empty(B, Sq, H, D, dtype=q.dtype, device="cuda").transpose(1, 2)
    dk = torch.empty(B, Skv, H, D, dtype=q.dtype, device="cuda").transpose(1, 2)
    dv = torch.empty(B, Skv, H, D, dtype=q.dtype, device="cuda").transpose(1, 2)
    ws_n = lib().mi355x_attn_bwd_workspace_bytes(B, H, Sq, Skv, D)
    ws = workspace(ws_n)
    call("mi355x_attn_bwd", p(dq), bhs(dq), p(dk), bhs(dk), p(dv), bhs(dv), p(do), bhs(do),
         p(q), bhs(q), p(k), bhs(k), p(v), bhs(v), p(o), bhs(o), p(lse),
         B, H, Sq, Skv, D, scale, int(causal), CODE[q.dtype], p(ws), ws_n, None)
    return dq, dk, dv


# (2, 4, 256, 256, 64), (1, 8, 300, 300, 64) and (4, 2, 130, 130, 128) have B*H*ceil(S/128) % 8 == 0,
# which runs dK/dV and dQ as one launch; the others run them as two.  With
# B*H*ceil(S/128) % 32 == 0 ((1, 8, 512, 512, 64), (2, 4, 512, 512, 128))
# the one launch deals the two block kinds in groups of four slots per XCD
# (alternating per shader engine) instead of alternating slot by slot.
@pytest.mark.parametrize("shape", [(2, 3, 128, 128, 64), (1, 2, 100, 160, 64), (2, 2, 160, 100, 64),
                                   (1, 2, 192, 192, 32), (1, 2, 130, 130, 128), (1, 1, 1, 1, 64),
                                   (2, 4, 256, 256, 64), (1, 8, 300, 300, 64), (4, 2, 130, 130, 128),
                                   (1, 8, 512, 512, 64), (2, 4, 512, 512, 128)])
@pytest.mark.parametrize("causal", [True, False])
def test_attention_fwd_bwd_matches_oracle(kernels, shape, causal):
    B, H, Sq, Skv, D = shape
    q = randn(B, H, Sq, D).bfloat16()
    k = randn(B, H, Skv, D).bfloat16()
    v = randn(B, H, Skv, D).bfloat16()
    do = randn(B, H, Sq, D).bfloat16()
    tq, tk, tv, tdo = dev(q), dev(k), dev(v), dev(do)
    o, lse = _attn_fwd(tq, tk, tv, causal)
    eo, else_ = O.sdpa_forward(q.double().numpy(), k.double().numpy(), v.double().numpy(), causal=causal)
    tol_close(np64(o), eo, atol=2e-2, rtol=2e-2, what="O")
    tol_close(np64(lse), else_, atol=1e-3, rtol=1e-3, what="LSE")
    dq, dk, dv = _attn_bwd(tdo, tq, tk, tv, o, lse, causal)
    edq, edk, edv = O.sdpa_backward(do.double().numpy(), q.double().numpy(), k.double().numpy(),
                                    v.double().numpy(), np64(o), np64(lse), causal=causal)
    tol_close(np64(dv), edv, atol=2e-2, rtol=2e-2, what="dV")
    tol_close(np64(dk), edk, atol=2e-2, rtol=2e-2, what="dK")
    tol_close(np64(dq), edq, atol=2e-2, rtol=2e-2, what="dQ")


def test_attention_special_cases(kernels):
    """S = 1 gives O = V; causal row 0 attends only to key 0."""
    q = randn(1, 2, 64, 64).bfloat16()
    k = randn(1, 2, 64, 64).bfloat16()
    v = randn(1, 2, 64, 64).bfloat16()
    o, lse = _attn_fwd(dev(q[:, :, :1]), dev(k[:, :, :1]), dev(v[:, :, :1]), True)
    assert torch.allclose(host(o).float(), v[:, :, :1].float(), atol=1e-2)
    o, lse = _attn_fwd(dev(q), dev(k), dev(v), True)
    assert torch.allclose(host(o)[:, :, 0].float(), v[:, :, 0].float(), atol=1e-2)
    s00 = (q[:, :, 0].float() * k[:, :, 0].float()).sum(-1) / 8.0
    assert torch.allclose(host(lse)[:, :, 0], s00, atol=1e-3)


def test_attention_gapped_qkv_views(kernels):
    """q/k/v as split+view+transpose of one fused qkv projection (BTHD storage
    with a 3C row stride), as nanoGPT hands them over."""
    B, T, H, D = 2, 256, 4, 64
    C = H * D
    qkv = randn(B, T, 3 * C).bfloat16()
    tqkv = dev(qkv)
    tq, tk, tv = (t.view(B, T, H, D).transpose(1, 2) for t in tqkv.split(C, dim=2))
    assert tq.stride() == (T * 3 * C, D, 3 * C, 1)
    o, lse = _attn_fwd(tq, tk, tv, True)
    q, k, v = (t.view(B, T, H, D).transpose(1, 2).double().numpy() for t in qkv.split(C, dim=2))
    eo, _ = O.sdpa_forward(q, k, v, causal=True)
    tol_close(np64(o), eo, atol=2e-2, rtol=2e-2, what="gapped O")


def test_attention_cfg1_shape_properties(kernels):
    """BASELINE cfg 1 shape [8,12,1024,64]: fwd vs oracle on two heads, and
    sum_j dK_j = 0 (softmax rows are shift-invariant) over the full size."""
    B, H, S, D = 8, 12, 1024, 64
    q = randn(B, H, S, D).bfloat16()
    k = randn(B, H, S, D).bfloat16()
    v = randn(B, H, S, D).bfloat16()
    do = randn(B, H, S, D).bfloat16()
    tq, tk, tv, tdo = dev(q), dev(k), dev(v), dev(do)
    o, lse = _attn_fwd(tq, tk, tv, True)
    sel = (slice(0, 1), slice(0, 2))
    eo, el = O.sdpa_forward(q[sel].double().numpy(), k[sel].double().numpy(), v[sel].double().numpy(), causal=True)
    tol_close(np64(o[sel]), eo, atol=2e-2, rtol=2e-2, what="O cfg1")
    tol_close(np64(lse[sel]), el, atol=1e-3, rtol=1e-3, what="LSE cfg1")
    dq, dk, dv = _attn_bwd(tdo, tq, tk, tv, o, lse, True)
    # dS rows sum to zero, so sum over keys of dK (and of dQ's row contributions) cancels
    tot = host(dk).double().sum(2)
    assert tot.abs().max().item() < 0.5
    # dV columns: sum over keys of dV = sum over queries of dO (P rows sum to 1)
    tol_close(host(dv).double().sum(2).numpy(), do.double().sum(2).numpy(), atol=0.5, rtol=2e-2, what="sum dV")


@pytest.mark.parametrize("m,n,k,layout,batch", [(2304, 768, 16384, "TN", 1), (300, 200, 1001, "NT", 1),
                                                (130, 96, 320, "NN", 2), (1000, 520, 4160, "TN", 1),
                                                (768, 3072, 16384, "TT", 1), (2048, 3072, 1024, "NT", 1),
                                                (4096, 4096, 512, "NT", 1), (4096, 3072, 1000, "NT", 1)])
def test_gemm_ex_round_and_rowsum(kernels, m, n, k, layout, batch):
    """mi355x_gemm_ex with MI355X_GEMM_ROUND (f32 C holding bf16-rounded
    values) and the row sums of A (the linear bias gradient), with and
    without split-K, ragged K and a batch."""
    A = (randn(batch, m, k) * 0.5).bfloat16()
    B = (randn(batch, k, n) * 0.1).bfloat16()
    if layout[0] == "N":
        ta, a_rs, a_cs = dev(A.contiguous()), k, 1
    else:
        ta, a_rs, a_cs = dev(A.transpose(1, 2).contiguous()), 1, m
    if layout[1] == "N":
        tb, b_rs, b_cs = dev(B.contiguous()), n, 1
    else:
        tb, b_rs, b_cs = dev(B.transpose(1, 2).contiguous()), 1, k
    a_bs, b_bs = (m * k, k * n) if batch > 1 else (0, 0)
    c = torch.empty(batch, m, n, device="cuda")
    rs = torch.empty(batch, m, device="cuda")
    ws_n = lib().mi355x_gemm_workspace_bytes(p(ta), a_rs, a_cs, a_bs, p(tb), b_rs, b_cs, b_bs, CODE[torch.bfloat16],
                                             batch, m, n, k)
    ws = workspace(ws_n) if ws_n else None
    call("mi355x_gemm_ex", p(c), CODE[torch.float32], n, m * n, p(ta), a_rs, a_cs, a_bs, p(tb), b_rs, b_cs, b_bs,
         CODE[torch.bfloat16], None, 0, 2, p(rs), CODE[torch.float32], batch, m, n, k, p(ws), ws_n, None)
    got_c, got_rs = host(c), host(rs)
    # ROUND: every stored value is a bf16 value
    assert torch.equal(got_c, got_c.bfloat16().float())
    assert torch.equal(got_rs, got_rs.bfloat16().float())
    exp_c = torch.bmm(A.double(), B.double()).numpy()
    exp_rs = A.double().sum(2).numpy()
    tol_close(got_c.numpy(), exp_c, atol=2e-2 * math.sqrt(k / 64), rtol=1e-2, what="C")
    tol_close(got_rs.numpy(), exp_rs, atol=2e-2 * math.sqrt(k / 64), rtol=1e-2, what="rowsum")


def _attn_fwd_ex(q, k, v, causal, window, scale=None):
    B, H, Sq, D = q.shape
    Hk, Skv = k.shape[1], k.shape[2]
    scale = 1.0 / math.sqrt(D) if scale is None else scale
    o = torch.empty(B, Sq, H, D, dtype=q.dtype, device="cuda").transpose(1, 2)
    lse = torch.empty(B, H, Sq, device="cuda")
    call("mi355x_attn_fwd_ex", p(o), bhs(o), p(lse), p(q), bhs(q), p(k), bhs(k), p(v), bhs(v),
         B, H, Hk, Sq, Skv, D, scale, int(causal), window, CODE[q.dtype], None)
    return o, lse


@pytest.mark.parametrize("d", [64, 128, 256])
@pytest.mark.parametrize("heads,kv_heads", [(4, 1), (4, 2), (2, 2)])
@pytest.mark.parametrize("s,window", [(130, 0), (300, 7), (300, 64), (200, 200), (257, 100)])
def test_attention_fwd_ex_gqa_window_matches_oracle(kernels, d, heads, kv_heads, s, window):
    """Grouped K/V heads, causal sliding window and head_dim 256 (the
    Gemma-3-shaped prefill): O and LSE against the oracle."""
    q = randn(1, heads, s, d).bfloat16()
    k = randn(1, kv_heads, s, d).bfloat16()
    v = randn(1, kv_heads, s, d).bfloat16()
    o, lse = _attn_fwd_ex(dev(q), dev(k), dev(v), True, window)
    eo, el = O.sdpa_forward(q.double().numpy(), k.double().numpy(), v.double().numpy(), causal=True, window=window)
    tol_close(np64(o), eo, atol=2e-2, rtol=2e-2, what=f"O d{d} h{heads}/{kv_heads} w{window}")
    tol_close(np64(lse), el, atol=1e-2, rtol=1e-3, what="LSE")


def test_attention_fwd_ex_rejects_bad_arguments(kernels):
    q = dev(randn(1, 3, 64, 64).bfloat16())
    k = dev(randn(1, 2, 64, 64).bfloat16())
    o = torch.empty(1, 64, 3, 64, dtype=torch.bfloat16, device="cuda").transpose(1, 2)
    lse = torch.empty(1, 3, 64, device="cuda")
    rc = lib().mi355x_attn_fwd_ex(p(o), bhs(o), p(lse), p(q), bhs(q), p(k), bhs(k), p(k), bhs(k),
                                  1, 3, 2, 64, 64, 64, 0.125, 1, 0, CODE[torch.bfloat16], None)
    assert rc != 0 and b"multiple of kv_heads" in lib().mi355x_last_error()
    rc = lib().mi355x_attn_fwd_ex(p(o), bhs(o), p(lse), p(q), bhs(q), p(q), bhs(q), p(q), bhs(q),
                                  1, 3, 3, 64, 64, 64, 0.125, 0, 16, CODE[torch.bfloat16], None)
    assert rc != 0 and b"needs causal" in lib().mi355x_last_error()


# ---------------------------------------------------------------------------
# f32 kernels: f32 inputs, any head_dim up to 256, grouped / windowed backward
# ---------------------------------------------------------------------------
def _attn_gen(q, k, v, do, causal, window, scale=None):
    B, H, Sq, D = q.shape
    Hk, Skv = k.shape[1], k.shape[2]
    scale = 1.0 / math.sqrt(D) if scale is None else scale
    dt = CODE[q.dtype]
    o = torch.empty(B, Sq, H, D, dtype=q.dtype, device="cuda").transpose(1, 2)
    lse = torch.empty(B, H, Sq, device="cuda")
    call("mi355x_attn_fwd_gen", p(o), bhs(o), p(lse), p(q), bhs(q), p(k), bhs(k), p(v), bhs(v),
         B, H, Hk, Sq, Skv, D, scale, int(causal), window, dt, None)
    dq = torch.empty(B, Sq, H, D, dtype=q.dtype, device="cuda").transpose(1, 2)
    dk = torch.empty(B, Skv, Hk, D, dtype=q.dtype, device="cuda").transpose(1, 2)
    dv = torch.empty(B, Skv, Hk, D, dtype=q.dtype, device="cuda").transpose(1, 2)
    ws_n = lib().mi355x_attn_bwd_gen_workspace_bytes(B, H, Hk, Sq, Skv, D)
    ws = workspace(ws_n)
    call("mi355x_attn_bwd_gen", p(dq), bhs(dq), p(dk), bhs(dk), p(dv), bhs(dv), p(do), bhs(do),
         p(q), bhs(q), p(k), bhs(k), p(v), bhs(v), p(o), bhs(o), p(lse),
         B, H, Hk, Sq, Skv, D, scale, int(causal), window, dt, p(ws), ws_n, None)
    return o, lse, dq, dk, dv


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape", [(2, 3, 3, 70, 70, 40), (1, 2, 2, 33, 90, 64), (1, 4, 2, 100, 100, 96),
                                   (1, 4, 1, 64, 64, 200), (2, 2, 2, 50, 50, 256), (1, 1, 1, 1, 1, 8)])
@pytest.mark.parametrize("mode", ["full", "causal", "window"])
def test_attention_f32_kernels_match_oracle(kernels, dtype, shape, mode):
    """mi355x_attn_fwd_gen / mi355x_attn_bwd_gen against the f64 oracle: f32
    and bf16 inputs, head_dims the tuned MFMA kernels do not take (40, 96,
    200, 256), Sq != Skv, grouped K/V heads (dK/dV summed over each group)
    and a causal sliding window.  The bf16 backward at head_dim 64 and 256
    runs the grouped MFMA kernels, the rest the f32 kernels."""
    B, H, Hk, Sq, Skv, D = shape
    causal = mode != "full"
    window = 17 if mode == "window" else 0
    if window and Sq != Skv:
        pytest.skip("windows are defined for Sq == Skv")
    g = torch.Generator().manual_seed(hash((shape, mode)) % 1000)
    q, do = (torch.randn(B, H, Sq, D, generator=g).to(dtype) for _ in range(2))
    k, v = (torch.randn(B, Hk, Skv, D, generator=g).to(dtype) for _ in range(2))
    o, lse, dq, dk, dv = _attn_gen(dev(q), dev(k), dev(v), dev(do), causal, window)
    n = lambda t: t.double().numpy()  # noqa: E731
    eo, el = O.sdpa_forward(n(q), n(k), n(v), causal=causal, window=window)
    tol = dict(atol=1e-4, rtol=1e-4) if dtype == torch.float32 else dict(atol=2e-2, rtol=2e-2)
    tol_close(np64(o), eo, what="O", **tol)
    tol_close(np64(lse), el, atol=1e-4, rtol=1e-4, what="LSE")
    edq, edk, edv = O.sdpa_backward(n(do), n(q), n(k), n(v), np64(o), np64(lse), causal=causal, window=window)
    gtol = dict(atol=2e-4, rtol=2e-4) if dtype == torch.float32 else dict(atol=2e-2, rtol=2e-2)
    tol_close(np64(dv), edv, what="dV", **gtol)
    tol_close(np64(dk), edk, what="dK", **gtol)
    tol_close(np64(dq), edq, what="dQ", **gtol)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", [(2, 4, 2, 130, 130, 64), (1, 6, 2, 200, 200, 128), (1, 4, 1, 96, 160, 256),
                                   (1, 8, 1, 300, 300, 64)])
@pytest.mark.parametrize("mode", ["full", "causal", "window"])
def test_grouped_mfma_backward_matches_oracle(kernels, dtype, shape, mode):
    """The grouped/windowed MFMA backward (attn_bwd_gqa_*: per-query-head
    dK/dV partials summed in head order, dQ per query head) at head_dim 64,
    128 and 256 with ragged 64-row tiles, Sq != Skv (top-left causal) and
    windows that end inside a tile, against the f64 oracle at atol = rtol =
    2e-2."""
    B, H, Hk, Sq, Skv, D = shape
    causal = mode != "full"
    window = 37 if mode == "window" else 0
    if window and Sq != Skv:
        pytest.skip("windows are defined for Sq == Skv")
    g = torch.Generator().manual_seed(sum(shape) + len(mode))
    q, do = (torch.randn(B, H, Sq, D, generator=g).to(dtype) for _ in range(2))
    k, v = (torch.randn(B, Hk, Skv, D, generator=g).to(dtype) for _ in range(2))
    o, lse, dq, dk, dv = _attn_gen(dev(q), dev(k), dev(v), dev(do), causal, window)
    n = lambda t: t.double().numpy()  # noqa: E731
    edq, edk, edv = O.sdpa_backward(n(do), n(q), n(k), n(v), np64(o), np64(lse), causal=causal, window=window)
    tol_close(np64(dv), edv, atol=2e-2, rtol=2e-2, what="dV")
    tol_close(np64(dk), edk, atol=2e-2, rtol=2e-2, what="dK")
    tol_close(np64(dq), edq, atol=2e-2, rtol=2e-2, what="dQ")
