"""GPU parity of the HBM-bound kernels, called through the C ABI, against the
oracle (and bit-exact where the op is integer/index/copy work)."""

import ctypes
import math

import numpy as np
import pytest
import torch

from abi import (CODE, AdamWTensor, bhs, call, dev, host, i64, lib, np64, p, tol_close,  # noqa: F401
                 workspace)
from oracle import ops as O

pytestmark = pytest.mark.gpu

G = torch.Generator().manual_seed(20260718)


def randn(*shape, dtype=torch.float32):
    return torch.randn(*shape, generator=G).to(dtype)


# ---------------------------------------------------------------------------
# copies / casts / elementwise
# ---------------------------------------------------------------------------
def test_cast_f32_to_bf16_is_rne_bit_exact(kernels):
    x = randn(1000, 257) * 37.0
    x[0, :4] = torch.tensor([float("inf"), float("-inf"), float("nan"), 1e-40])
    src = dev(x)
    out = torch.empty(x.shape, dtype=torch.bfloat16, device="cuda")
    call("mi355x_copy", p(out), 1, i64(*out.stride()), p(src), 0, i64(*src.stride()), i64(*x.shape), 2, None)
    expect = x.to(torch.bfloat16)
    got = host(out)
    assert torch.equal(got.view(torch.int16)[1:], expect.view(torch.int16)[1:])
    assert torch.isnan(got[0, 2])


def test_strided_broadcast_copy(kernels):
    x = randn(64, 48)
    src = dev(x)
    # transpose view of src into a dense [48, 64] bf16, and broadcast a row
    out = torch.empty(48, 64, dtype=torch.bfloat16, device="cuda")
    call("mi355x_copy", p(out), 1, i64(64, 1), p(src), 0, i64(1, 48), i64(48, 64), 2, None)
    assert torch.equal(host(out), x.t().to(torch.bfloat16))
    row = dev(randn(1, 64))
    out2 = torch.empty(5, 64, device="cuda")
    call("mi355x_copy", p(out2), 0, i64(64, 1), p(row), 0, i64(0, 1), i64(5, 64), 2, None)
    assert torch.equal(host(out2), host(row).expand(5, 64))


@pytest.mark.parametrize("op,fn", [(0, lambda a, b: a + 0.5 * b), (1, lambda a, b: a - 0.5 * b),
                                   (2, lambda a, b: a * b), (4, torch.maximum), (11, lambda a, b: a > b)])
def test_map_binary_broadcast_exact(kernels, op, fn):
    a, b = randn(33, 70), randn(1, 70)
    ta, tb = dev(a), dev(b)
    out_dt = torch.bool if op == 11 else torch.float32
    out = torch.empty(33, 70, dtype=out_dt, device="cuda")
    ins = (ctypes.c_void_p * 3)(p(ta), p(tb), None)
    dts = (ctypes.c_int * 3)(0, 0, 0)
    call("mi355x_map", op, p(out), CODE[out_dt], 2, ins, dts, i64(70, 1, 70, 1, 0, 1), i64(33, 70), 2, 0.5, 0.0, None)
    assert torch.equal(host(out), fn(a, b).to(out_dt))


@pytest.mark.parametrize("op,fn", [(0, lambda a, b: torch.add(a, b, alpha=0.5)),
                                   (1, lambda a, b: torch.sub(a, b, alpha=0.5)),
                                   (2, torch.mul), (3, torch.div)])
@pytest.mark.parametrize("cols", [64, 70])
def test_map_bf16_dense_binary(kernels, op, fn, cols):
    """bf16 (op) bf16 -> bf16 over dense [33, cols]: 64 columns take the
    8-wide kernel, 70 the generic one; both compute in f32 and round once,
    bit for bit as torch does on the CPU."""
    a, b = randn(33, cols).bfloat16(), randn(33, cols).bfloat16()
    ta, tb = dev(a), dev(b)
    out = torch.empty(33, cols, dtype=torch.bfloat16, device="cuda")
    ins = (ctypes.c_void_p * 3)(p(ta), p(tb), None)
    dts = (ctypes.c_int * 3)(CODE[torch.bfloat16], CODE[torch.bfloat16], 0)
    call("mi355x_map", op, p(out), CODE[torch.bfloat16], 2, ins, dts, i64(cols, 1, cols, 1, cols, 1),
         i64(33, cols), 2, 0.5, 0.0, None)
    assert torch.equal(host(out), fn(a, b))


@pytest.mark.parametrize("op,fn", [(0, lambda a, b: a + 0.5 * b), (1, lambda a, b: a - 0.5 * b),
                                   (2, lambda a, b: a * b), (3, lambda a, b: a / b)])
@pytest.mark.parametrize("ydt", [torch.float32, torch.bfloat16])
def test_map_row_broadcast_fast_path(kernels, op, fn, ydt):
    """x [5, 6, 64] (op) y [6, 64] broadcast over the leading dim: the dense
    row-broadcast kernel (a position embedding added to every sequence)."""
    a, b = randn(5, 6, 64), randn(6, 64).to(ydt)
    ta, tb = dev(a), dev(b)
    out = torch.empty(5, 6, 64, device="cuda")
    ins = (ctypes.c_void_p * 3)(p(ta), p(tb), None)
    dts = (ctypes.c_int * 3)(0, CODE[ydt], 0)
    call("mi355x_map", op, p(out), 0, 2, ins, dts, i64(384, 64, 1, 384, 64, 1, 0, 64, 1), i64(5, 6, 64), 3,
         0.5, 0.0, None)
    assert torch.equal(host(out), fn(a, b.float()))


def test_map_scalar_operand_and_integer_math(kernels):
    x = torch.arange(-20, 20, dtype=torch.int64)
    tx = dev(x)
    out = torch.empty(40, dtype=torch.int64, device="cuda")
    ins = (ctypes.c_void_p * 3)(p(tx), None, None)
    dts = (ctypes.c_int * 3)(4, 4, 0)
    # floor_divide by scalar 3 (NULL input reads s1)
    call("mi355x_map", 20, p(out), 4, 2, ins, dts, i64(1, 1, 0), i64(40), 1, 0.0, 3.0, None)
    assert torch.equal(host(out), torch.floor_divide(x, 3))
    call("mi355x_map", 19, p(out), 4, 2, ins, dts, i64(1, 1, 0), i64(40), 1, 0.0, 7.0, None)
    assert torch.equal(host(out), torch.remainder(x, 7))


def test_fill_and_arange(kernels):
    out = torch.empty(1000, dtype=torch.int64, device="cuda")
    call("mi355x_arange", p(out), 4, 1000, 5.0, 3.0, None)
    assert torch.equal(host(out), torch.arange(5, 5 + 3 * 1000, 3))
    f = torch.empty(7, 9, dtype=torch.bfloat16, device="cuda")
    call("mi355x_fill", p(f), 1, i64(9, 1), i64(7, 9), 2, 0.1, None)
    assert torch.equal(host(f), torch.full((7, 9), 0.1, dtype=torch.bfloat16))


# ---------------------------------------------------------------------------
# reductions / index
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("shape,axis", [((16384, 768), 0), ((64, 50257), 1), ((3, 1 << 20), 1), ((5, 7, 9), 1)])
def test_reduce_sum_matches_oracle(kernels, shape, axis):
    x = randn(*shape)
    tx = dev(x)
    outer = math.prod(shape[:axis])
    r = shape[axis]
    inner = math.prod(shape[axis + 1:])
    out = torch.empty(outer * inner, device="cuda")
    ws_n = lib().mi355x_reduce_workspace_bytes(outer, r, inner)
    ws = workspace(ws_n)
    call("mi355x_reduce", 0, p(out), 0, p(tx), 0, outer, r, inner, r * inner, inner, 1, p(ws), ws_n, None)
    expect = x.double().numpy().reshape(outer, r, inner).sum(1).reshape(-1)
    tol_close(np64(out), expect, atol=1e-3, rtol=1e-5, what="sum")


@pytest.mark.parametrize("rows,cols", [(16384, 2304), (7, 72), (1000, 50304)])
def test_bias_grad_column_sum_bf16(kernels, rows, cols):
    """sum(dY, 0) over a bf16 [rows, cols] gradient (the vectorised column-sum
    path), accumulated in f32, rounded once to bf16."""
    x = randn(rows, cols).bfloat16()
    tx = dev(x)
    out = torch.empty(cols, dtype=torch.bfloat16, device="cuda")
    ws_n = lib().mi355x_reduce_workspace_bytes(1, rows, cols)
    ws = workspace(ws_n)
    call("mi355x_reduce", 0, p(out), 1, p(tx), 1, 1, rows, cols, rows * cols, cols, 1, p(ws), ws_n, None)
    expect = x.double().numpy().sum(0)
    tol_close(np64(out), expect, atol=2e-2 * math.sqrt(rows / 64), rtol=1e-2, what="colsum")


def test_reduce_max_norm_mean(kernels):
    x = randn(37, 1000)
    x[3, 5] = float("nan")
    tx = dev(x)
    out = torch.empty(37, device="cuda")
    for op, fn in ((2, lambda a: np.max(a, 1)), (4, lambda a: np.sqrt((a ** 2).sum(1))), (1, lambda a: a.mean(1))):
        call("mi355x_reduce", op, p(out), 0, p(tx), 0, 37, 1000, 1, 1000, 1, 1, None, 0, None)
        tol_close(np64(out), fn(x.double().numpy()), atol=1e-5, rtol=1e-5, what=f"op{op}")


def test_argmax_bit_exact_with_ties_and_nan(kernels):
    x = torch.randint(0, 5, (64, 300), generator=G).float()
    x[7, 100] = float("nan")
    tx = dev(x)
    out = torch.empty(64, dtype=torch.int64, device="cuda")
    call("mi355x_argreduce", 0, p(out), None, p(tx), 0, 64, 300, 1, 300, 1, 1, None)
    assert torch.equal(host(out), torch.argmax(x, 1))
    out2 = torch.empty(300, dtype=torch.int64, device="cuda")
    call("mi355x_argreduce", 1, p(out2), None, p(tx), 0, 1, 64, 300, 0, 300, 1, None)
    assert torch.equal(host(out2), torch.argmin(x, 0))


def test_index_select_and_embedding_forward_bit_exact(kernels):
    w = randn(50257, 768)
    idx = torch.randint(0, 50257, (4, 256), generator=G)
    tw, ti = dev(w), dev(idx)
    out = torch.empty(4 * 256, 768, device="cuda")
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    call("mi355x_embedding_fwd", p(out), p(tw), 0, p(ti), 1024, 50257, 768, 768, p(err), None)
    assert torch.equal(host(out), w[idx.reshape(-1)])
    assert host(err).item() == 0
    bad = dev(torch.tensor([0, 50257, -1]))
    out3 = torch.empty(3, 768, device="cuda")
    call("mi355x_embedding_fwd", p(out3), p(tw), 0, p(bad), 3, 50257, 768, 768, p(err), None)
    assert host(err).item() == 1
    assert torch.equal(host(out3)[1:], torch.zeros(2, 768))


def test_embedding_backward_bit_exact_vs_sequential_f32(kernels):
    n, num, dim = 4096, 300, 96
    idx = torch.randint(0, num, (n,), generator=G)
    idx[:50] = 7  # heavy repetition
    g = randn(n, dim)
    tg, ti = dev(g), dev(idx)
    gw = torch.empty(num, dim, device="cuda")
    ws_n = lib().mi355x_embedding_bwd_workspace_bytes(n, num)
    ws = workspace(ws_n)
    call("mi355x_embedding_bwd", p(gw), p(tg), 0, p(ti), n, num, dim, 3, p(ws), ws_n, None)
    expect = O.embedding_backward_f32(g.numpy(), idx.numpy(), num, padding_idx=3)
    assert np.array_equal(host(gw).numpy(), expect)
    # and ATen's own CPU kernel gives the same bits
    ref = torch.ops.aten.embedding_dense_backward(g, idx, num, 3, False)
    assert torch.equal(host(gw), ref)


@pytest.mark.parametrize("n,num,dim,dtype", [(4096, 300, 96, torch.float32), (16384, 50304, 768, torch.float32),
                                             (1000, 70, 30, torch.float32), (512, 90, 64, torch.bfloat16)])
def test_embedding_backward_accumulate_equals_dense_then_add(kernels, n, num, dim, dtype):
    """base + embedding gradient in one pass (the tied-embedding case):
    out of place and in place, the bits of the dense gradient followed by
    the elementwise add; rows no index names and the padding row keep base's
    bits.  Includes the nanoGPT shape (16384 ids over 50304 rows)."""
    idx = torch.randint(0, num, (n,), generator=G)
    idx[:50] = 7
    pad = 3
    g = randn(n, dim).to(dtype)
    base = randn(num, dim).to(dtype)
    tg, ti, tb = dev(g), dev(idx), dev(base)
    ws_n = lib().mi355x_embedding_bwd_workspace_bytes(n, num)
    ws = workspace(ws_n)
    code = CODE[dtype]
    dense = torch.empty(num, dim, dtype=dtype, device="cuda")
    call("mi355x_embedding_bwd", p(dense), p(tg), code, p(ti), n, num, dim, pad, p(ws), ws_n, None)
    want = (host(tb).float() + host(dense).float()).to(dtype)
    out = torch.full_like(tb, float("nan"))
    call("mi355x_embedding_bwd_accumulate", p(out), p(tb), p(tg), code, p(ti), n, num, dim, pad, p(ws), ws_n, None)
    assert torch.equal(host(out), want)
    assert torch.equal(host(tb), base)  # base untouched out of place
    call("mi355x_embedding_bwd_accumulate", p(tb), p(tb), p(tg), code, p(ti), n, num, dim, pad, p(ws), ws_n, None)
    assert torch.equal(host(tb), want)
    absent = torch.ones(num, dtype=torch.bool)
    absent[idx] = False
    absent[pad] = True
    assert torch.equal(host(out)[absent], base[absent])


# ---------------------------------------------------------------------------
# layer norm / gelu / softmax / nll
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("dtype,rows,cols", [(torch.float32, 16384, 768), (torch.float32, 33, 1000),
                                             (torch.bfloat16, 300, 768), (torch.float32, 7, 4099),
                                             (torch.float32, 8197, 768), (torch.bfloat16, 3, 256),
                                             (torch.float32, 100, 2048)])
def test_layer_norm_fwd_bwd(kernels, dtype, rows, cols):
    x = randn(rows, cols) * 3 + 1
    g, b = randn(cols), randn(cols)
    dy = randn(rows, cols)
    xq, gq, bq, dyq = (t.to(dtype) for t in (x, g, b, dy))
    tx, tg, tb, tdy = dev(xq), dev(gq), dev(bq), dev(dyq)
    y = torch.empty(rows, cols, dtype=dtype, device="cuda")
    mean = torch.empty(rows, device="cuda")
    rstd = torch.empty(rows, device="cuda")
    call("mi355x_layer_norm_fwd", p(y), p(mean), p(rstd), p(tx), p(tg), p(tb), rows, cols, 1e-5, CODE[dtype], None)
    if dtype == torch.float32:
        # the autocast variant: the same y plus its bf16 rounding from the same kernel
        y2 = torch.empty_like(y)
        low = torch.empty(rows, cols, dtype=torch.bfloat16, device="cuda")
        call("mi355x_layer_norm_fwd_ex", p(y2), p(low), CODE[torch.bfloat16], None, None, p(tx), p(tg), p(tb),
             rows, cols, 1e-5, CODE[dtype], None)
        assert torch.equal(host(y2), host(y))
        assert torch.equal(host(low), host(y).bfloat16())
    ey, em, er = O.layer_norm(xq.double().numpy(), gq.double().numpy(), bq.double().numpy())
    atol = 1e-4 if dtype == torch.float32 else 2e-2
    tol_close(np64(y), ey, atol=atol, rtol=atol, what="ln y")
    tol_close(np64(mean), em[:, 0], atol=1e-5, rtol=1e-5, what="ln mean")
    tol_close(np64(rstd), er[:, 0], atol=1e-5, rtol=1e-4, what="ln rstd")
    dx = torch.empty_like(tx)
    dg = torch.empty_like(tg)
    db = torch.empty_like(tb)
    ws_n = lib().mi355x_layer_norm_bwd_workspace_bytes(rows, cols)
    ws = workspace(ws_n)
    call("mi355x_layer_norm_bwd", p(dx), p(dg), p(db), p(tdy), p(tx), p(mean), p(rstd), p(tg), rows, cols,
         CODE[dtype], p(ws), ws_n, None)
    edx, edg, edb = O.layer_norm_backward(dyq.double().numpy(), xq.double().numpy(), em, er, gq.double().numpy())
    tol_close(np64(dx), edx, atol=atol * 5, rtol=atol, what="ln dx")
    scale = math.sqrt(rows)
    tol_close(np64(dg), edg, atol=atol * scale, rtol=atol, what="ln dgamma")
    tol_close(np64(db), edb, atol=atol * scale, rtol=atol, what="ln dbeta")


@pytest.mark.parametrize("dtype,rows,cols", [(torch.float32, 16384, 768), (torch.float32, 33, 1000),
                                             (torch.float32, 7, 4099), (torch.float32, 100, 2048),
                                             (torch.bfloat16, 300, 768), (torch.float32, 5, 770)])
@pytest.mark.parametrize("affine", [True, False])
def test_layer_norm_output_deferred_to_apply_is_bit_identical(kernels, dtype, rows, cols, affine):
    """The autocast forward writes only the 16-bit copy and the statistics
    (y = null); mi355x_layer_norm_apply later computes y from x and those
    statistics.  That y must be the forward's own y bit for bit, on the wave
    path (cols a multiple of 4), on the any-width block path (4099, 770 with
    an odd row pitch) and, for the fused residual add, from its x_out."""
    x = randn(rows, cols) * 3 + 1
    g, b = randn(cols), randn(cols)
    xq, gq, bq = (t.to(dtype) for t in (x, g, b))
    tx, tg, tb = dev(xq), dev(gq), dev(bq)
    pg, pb = (p(tg), p(tb)) if affine else (None, None)
    low_dt = torch.bfloat16 if dtype == torch.float32 else dtype

    def stats():
        return torch.empty(rows, device="cuda"), torch.empty(rows, device="cuda")

    y = torch.empty(rows, cols, dtype=dtype, device="cuda")
    mean, rstd = stats()
    low = torch.empty(rows, cols, dtype=low_dt, device="cuda") if dtype == torch.float32 else None
    call("mi355x_layer_norm_fwd_ex", p(y), p(low) if low is not None else None, CODE[low_dt], p(mean), p(rstd),
         p(tx), pg, pb, rows, cols, 1e-5, CODE[dtype], None)
    y2 = torch.full_like(y, float("nan"))
    mean2, rstd2 = stats()
    if low is not None:
        low2 = torch.empty_like(low)
        call("mi355x_layer_norm_fwd_ex", None, p(low2), CODE[low_dt], p(mean2), p(rstd2), p(tx), pg, pb,
             rows, cols, 1e-5, CODE[dtype], None)
        assert torch.equal(host(low2), host(low))
        assert torch.equal(host(mean2), host(mean)) and torch.equal(host(rstd2), host(rstd))
    else:
        mean2, rstd2 = mean, rstd
    call("mi355x_layer_norm_apply", p(y2), p(tx), p(mean2), p(rstd2), pg, pb, rows, cols, CODE[dtype], None)
    assert torch.equal(host(y2), host(y))
    if dtype == torch.float32 and cols % 4 == 0 and cols <= 2048:
        r = dev(randn(rows, cols).bfloat16())
        ya, xo = torch.empty_like(y), torch.empty_like(y)
        lowa = torch.empty_like(low)
        ma, ra = stats()
        call("mi355x_layer_norm_fwd_add", p(ya), p(lowa), CODE[low_dt], p(ma), p(ra), p(xo), p(tx), p(r),
             CODE[torch.bfloat16], pg, pb, rows, cols, 1e-5, CODE[dtype], None)
        yb, xo2 = torch.full_like(y, float("nan")), torch.empty_like(y)
        lowb = torch.empty_like(low)
        mb, rb = stats()
        call("mi355x_layer_norm_fwd_add", None, p(lowb), CODE[low_dt], p(mb), p(rb), p(xo2), p(tx), p(r),
             CODE[torch.bfloat16], pg, pb, rows, cols, 1e-5, CODE[dtype], None)
        assert torch.equal(host(xo2), host(xo)) and torch.equal(host(lowb), host(lowa))
        call("mi355x_layer_norm_apply", p(yb), p(xo2), p(mb), p(rb), pg, pb, rows, cols, CODE[dtype], None)
        assert torch.equal(host(yb), host(ya))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("approx", [0, 1])
def test_gelu(kernels, dtype, approx):
    """f32 storage uses the libm erf/tanh; 16-bit storage branch-free forms
    (the Numerical Recipes erfc, relative error < 1.2e-7, and a sigmoid form
    of 1 + tanh), whose error must vanish in the rounding: besides the
    tolerance, at least 99.9% of the results for x >= -3 equal the f64
    oracle rounded to the storage type (the rest sit on a rounding boundary).
    Below -3 the oracle's own 1 + erf and 1 + tanh lose their relative
    precision (to 0 past x ~ -8.3 and -7.3), so only the tolerance applies."""
    n = 16384 * 3 + 5
    x = randn(n) * 4
    dy = randn(n)
    xq, dyq = x.to(dtype), dy.to(dtype)
    tx, tdy = dev(xq), dev(dyq)
    y = torch.empty_like(tx)
    call("mi355x_gelu_fwd", p(y), p(tx), n, approx, CODE[dtype], None)
    mode = "tanh" if approx else "none"
    tol = {torch.float32: 1e-5, torch.bfloat16: 1e-2, torch.float16: 2e-3}[dtype]
    want_y = O.gelu(xq.double().numpy(), mode)
    tol_close(np64(y), want_y, atol=tol, rtol=tol, what="gelu")
    dx = torch.empty_like(tx)
    call("mi355x_gelu_bwd", p(dx), p(tdy), p(tx), n, approx, CODE[dtype], None)
    want_dx = O.gelu_backward(dyq.double().numpy(), xq.double().numpy(), mode)
    tol_close(np64(dx), want_dx, atol=tol, rtol=tol, what="gelu bwd")
    if dtype != torch.float32:
        for got, want, what in ((y, want_y, "gelu"), (dx, want_dx, "gelu bwd")):
            keep = xq >= -3
            same = (host(got)[keep] == torch.from_numpy(want).to(dtype)[keep]).double().mean().item()
            assert same >= 0.999, f"{what}: only {same:.5f} of the results round like the oracle"
        # below -3, against closed forms without the cancellation
        from scipy.special import erfc, expit
        xt = xq.double().numpy()
        tail = xt < -3
        if approx:
            k = math.sqrt(2.0 / math.pi)
            s = expit(2 * k * (xt + 0.044715 * xt**3))
            ty, tdx = xt * s, dyq.double().numpy() * (s + 2 * xt * s * (1 - s) * k * (1 + 3 * 0.044715 * xt**2))
        else:
            cdf = 0.5 * erfc(-xt / math.sqrt(2.0))
            ty = xt * cdf
            tdx = dyq.double().numpy() * (cdf + xt * np.exp(-0.5 * xt**2) / math.sqrt(2 * math.pi))
        tol_close(np64(y)[tail], ty[tail], atol=1e-7, rtol=tol, what="gelu tail")
        tol_close(np64(dx)[tail], tdx[tail], atol=1e-7, rtol=tol, what="gelu bwd tail")


# Rows longer than 1024 of one dtype run the register-resident kernels: odd
# lengths make every row start at a different phase of its 16-byte chunks;
# (5, 50257, f32) takes 16 chunks per thread, (3, 140001, bf16) is past their
# capacity and takes the streaming kernels.
@pytest.mark.parametrize("rows,cols,dtype", [(64, 50257, torch.bfloat16), (300, 1000, torch.float32),
                                             (17, 3, torch.float32), (8, 4096, torch.float32),
                                             (5, 50257, torch.float32), (6, 1027, torch.float16),
                                             (7, 2048, torch.bfloat16), (3, 140001, torch.bfloat16)])
@pytest.mark.parametrize("log", [0, 1])
def test_softmax_fwd_bwd(kernels, rows, cols, dtype, log):
    x = randn(rows, cols) * 3
    x[1, :] = float("-inf") if cols > 3 else x[1, :]
    x[2, 0] = float("-inf")
    if rows > 3:
        x[3, cols // 2] = float("nan")  # a NaN poisons its row only
    if rows > 4 and cols > 16:
        # a NaN whose 16-byte chunk is otherwise -inf (the chunk maximum is
        # the only NaN test) still poisons the row
        x[4, :16] = float("-inf")
        x[4, 5] = float("nan")
    xq = x.to(dtype)
    tx = dev(xq)
    y = torch.empty(rows, cols, dtype=dtype, device="cuda")
    call("mi355x_softmax_fwd", p(y), CODE[dtype], p(tx), CODE[dtype], rows, cols, log, None)
    with np.errstate(invalid="ignore"):
        ey = (O.log_softmax if log else O.softmax)(xq.double().numpy())
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    tol_close(np64(y), ey, atol=tol, rtol=tol, what="softmax")
    dy = randn(rows, cols).to(dtype)
    tdy = dev(dy)
    yy = torch.where(torch.isnan(y), torch.zeros_like(y), y)
    dx = torch.empty_like(y)
    call("mi355x_softmax_bwd", p(dx), CODE[dtype], p(tdy), CODE[dtype], p(yy), CODE[dtype], rows, cols, log, None)
    fn = O.log_softmax_backward if log else O.softmax_backward
    tol_close(np64(dx), fn(dy.double().numpy(), np64(yy)), atol=tol * 10, rtol=tol * 10, what="softmax bwd")


@pytest.mark.parametrize("reduction", [0, 1, 2])
def test_nll_fwd_bwd(kernels, reduction):
    n, c = 1000, 50257
    logp = torch.log_softmax(randn(n, c), 1)
    tgt = torch.randint(0, c, (n,), generator=G)
    tgt[::7] = -100
    w = None
    tl, tt = dev(logp), dev(tgt)
    out = torch.empty(n if reduction == 0 else (), device="cuda")
    tw = torch.empty((), device="cuda")
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    call("mi355x_nll_fwd", p(out), p(tw), p(tl), 0, p(tt), None, n, c, reduction, -100, p(err), None, 0, None)
    red = {0: "none", 1: "mean", 2: "sum"}[reduction]
    eo, etw = O.nll_loss(logp.numpy(), tgt.numpy(), w, red, -100)
    tol_close(np64(out), eo, atol=1e-4, rtol=1e-5, what="nll")
    assert host(tw).item() == etw
    assert host(err).item() == 0
    go = dev(randn(n) if reduction == 0 else torch.tensor(1.7))
    gi = torch.empty(n, c, device="cuda")
    call("mi355x_nll_bwd", p(gi), p(go), p(tt), None, p(tw), n, c, reduction, -100, 0, None)
    egi = O.nll_loss_backward(np64(go), (n, c), tgt.numpy(), None, red, -100, etw)
    assert np.array_equal(host(gi).numpy(), egi.astype(np.float32))
    bad = dev(torch.tensor([0, c + 5]))
    call("mi355x_nll_fwd", p(out), p(tw), p(tl), 0, p(bad), None, 2, c, 1, -100, p(err), None, 0, None)
    assert host(err).item() == 1


@pytest.mark.parametrize("reduction", [0, 1, 2])
@pytest.mark.parametrize("dtype,n,c", [(torch.bfloat16, 257, 50257), (torch.float32, 64, 1000),
                                       (torch.float16, 33, 4001)])
def test_fused_cross_entropy_matches_log_softmax_nll_chain(kernels, reduction, dtype, n, c):
    """The fused kernels against the oracle of the chain they replace:
    nll_loss(log_softmax(x)) forward, log_softmax_backward(nll_backward)
    backward (reduction none/mean/sum, ignore_index rows, odd row stride)."""
    x = (randn(n, c + 3) * 4).to(dtype)[:, :c]  # rows with a gap: stride c + 3
    tgt = torch.randint(0, c, (n,), generator=G)
    tgt[::5] = -100
    tx, tt = dev(x.contiguous()), dev(tgt)
    xs = torch.empty(n, c + 3, dtype=dtype, device="cuda")[:, :c]
    xs.copy_(tx)
    ld = c + 3
    out = torch.empty(n if reduction == 0 else (), device="cuda")
    lse = torch.empty(n, device="cuda")
    tw = torch.empty((), device="cuda")
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    ws_n = lib().mi355x_cross_entropy_workspace_bytes(n)
    ws = workspace(ws_n)
    call("mi355x_cross_entropy_fwd", p(out), p(tw), p(lse), p(xs), CODE[dtype], ld, p(tt), n, c,
         reduction, -100, p(err), p(ws), ws_n, None)
    red = {0: "none", 1: "mean", 2: "sum"}[reduction]
    logp = O.log_softmax(x.double().numpy())
    eo, etw = O.nll_loss(logp, tgt.numpy(), None, red, -100)
    tol_close(np64(out), eo, atol=1e-4, rtol=1e-5, what="ce loss")
    assert host(tw).item() == etw and host(err).item() == 0
    g = randn(n) if reduction == 0 else torch.tensor(1.3)
    tg = dev(g)
    ld_dx = (c + 7) // 8 * 8
    dx = torch.full((n, ld_dx), 7.0, dtype=dtype, device="cuda")
    call("mi355x_cross_entropy_bwd", p(dx), CODE[dtype], ld_dx, p(xs), CODE[dtype], ld, p(lse), p(tt),
         p(tg), reduction, p(tw), n, c, -100, None)
    dnll = O.nll_loss_backward(g.double().numpy(), (n, c), tgt.numpy(), None, red, -100, etw)
    edx = O.log_softmax_backward(dnll, logp)
    tol = 1e-6 if dtype == torch.float32 else 2e-2
    tol_close(np64(dx)[:, :c], edx, atol=tol * 1e-2 + 1e-7, rtol=tol, what="ce dx")
    assert (host(dx)[:, c:] == 0).all()


def test_fused_cross_entropy_nan_and_infinite_logits(kernels):
    """A NaN logit makes its row's loss NaN and leaves the other rows alone;
    -inf logits (masked classes) are legal and get zero gradient."""
    n, c = 5, 3001
    x = randn(n, c).bfloat16()
    x[1, 17] = float("nan")
    x[2, :1000] = float("-inf")
    x[4, :16] = float("-inf")  # a NaN in an otherwise -inf 16-byte chunk
    x[4, 5] = float("nan")
    tgt = torch.tensor([5, 6, 2000, 7, 100])
    tx, tt = dev(x), dev(tgt)
    out, lse, tw = torch.empty(n, device="cuda"), torch.empty(n, device="cuda"), torch.empty((), device="cuda")
    ws_n = lib().mi355x_cross_entropy_workspace_bytes(n)
    ws = workspace(ws_n)
    call("mi355x_cross_entropy_fwd", p(out), p(tw), p(lse), p(tx), CODE[torch.bfloat16], c, p(tt), n, c,
         0, -100, None, p(ws), ws_n, None)
    got = host(out)
    assert math.isnan(got[1].item()) and math.isnan(got[4].item())
    exp = torch.nn.functional.cross_entropy(x.float(), tgt, reduction="none")
    for i in (0, 2, 3):
        assert abs(got[i].item() - exp[i].item()) < 1e-4
    ld_dx = (c + 7) // 8 * 8
    dx = torch.empty(n, ld_dx, dtype=torch.bfloat16, device="cuda")
    call("mi355x_cross_entropy_bwd", p(dx), CODE[torch.bfloat16], ld_dx, p(tx), CODE[torch.bfloat16], c, p(lse),
         p(tt), p(dev(torch.ones(n))), 0, None, n, c, -100, None)
    d = host(dx).float()
    assert (d[2, :1000] == 0).all() and torch.isfinite(d[2]).all() and torch.isfinite(d[0]).all()


@pytest.mark.parametrize("reduction", [1, 2])
@pytest.mark.parametrize("dtype,n,c,ld", [(torch.bfloat16, 16384, 50257, 50257), (torch.bfloat16, 300, 50304, 50304),
                                          (torch.float16, 40, 4000, 4003), (torch.float32, 64, 1000, 1001),
                                          (torch.bfloat16, 9, 8, 8), (torch.float32, 7, 32752, 32752)])
def test_cross_entropy_fwd_bwd_is_the_two_calls_in_one_pass(kernels, reduction, dtype, n, c, ld):
    """mi355x_cross_entropy_fwd_bwd writes the values of mi355x_cross_entropy_fwd
    followed by mi355x_cross_entropy_bwd (loss, total_weight, lse, dx): the
    nanoGPT shape (rows of 50257 bf16, so every phase of row start), odd row
    strides, the longest f32 row it takes, ignored and NaN rows, padding
    columns; a longer row is refused."""
    x = (randn(n, ld) * 4).to(dtype)
    tgt = torch.randint(0, c, (n,), generator=G)
    tgt[::7] = -100
    if n > 3:
        x[3, 2] = float("nan")
    tx, tt = dev(x), dev(tgt)
    g = dev(torch.tensor(1.7))
    ws_n = lib().mi355x_cross_entropy_workspace_bytes(n)
    ws = workspace(ws_n)
    ld_dx = (c + 7) // 8 * 8
    res = []
    for fused in (False, True):
        out, tw = torch.empty((), device="cuda"), torch.empty((), device="cuda")
        lse = torch.empty(n, device="cuda")
        dx = torch.full((n, ld_dx), 7.0, dtype=dtype, device="cuda")
        err = torch.zeros(1, dtype=torch.int32, device="cuda")
        if fused:
            call("mi355x_cross_entropy_fwd_bwd", p(out), p(tw), p(lse), p(dx), ld_dx, p(tx), CODE[dtype], ld, p(tt),
                 p(g), n, c, reduction, -100, p(err), p(ws), ws_n, None)
        else:
            call("mi355x_cross_entropy_fwd", p(out), p(tw), p(lse), p(tx), CODE[dtype], ld, p(tt), n, c,
                 reduction, -100, p(err), p(ws), ws_n, None)
            call("mi355x_cross_entropy_bwd", p(dx), CODE[dtype], ld_dx, p(tx), CODE[dtype], ld, p(lse), p(tt),
                 p(g), reduction, p(tw), n, c, -100, None)
        res.append([host(t) for t in (out, tw, lse, dx, err)])
    for a, b, what in zip(res[0], res[1], ("loss", "total", "lse", "dx", "err")):
        # equal values (a NaN's sign bit may differ: the operand order of one
        # subtraction is the compiler's)
        torch.testing.assert_close(a, b, rtol=0, atol=0, equal_nan=True, msg=what)
    if dtype == torch.float32 and c == 32752:  # past 8192 16-byte chunks per row: refused before any access
        big = 32769
        rc = lib().mi355x_cross_entropy_fwd_bwd(p(out), p(tw), p(lse), p(dx), (big + 7) // 8 * 8, p(tx), CODE[dtype],
                                                 big, p(tt), p(g), n, big, reduction, -100, None, p(ws), ws_n, None)
        assert rc == 3  # MI355X_EUNSUPPORTED


# ---------------------------------------------------------------------------
# optimizer
# ---------------------------------------------------------------------------
def _adam_descs(params, grads, ms, vs, steps, vmax=None):
    n = len(params)
    d = (AdamWTensor * n)()
    for i in range(n):
        d[i].param, d[i].grad, d[i].exp_avg, d[i].exp_avg_sq = p(params[i]), p(grads[i]), p(ms[i]), p(vs[i])
        d[i].max_exp_avg_sq = p(vmax[i]) if vmax else None
        d[i].step = p(steps[i])
        d[i].numel = params[i].numel()
    return d


@pytest.mark.parametrize("amsgrad,maximize,wd", [(False, False, 0.1), (True, False, 0.1), (False, True, 0.0)])
def test_fused_adamw_matches_oracle(kernels, amsgrad, maximize, wd):
    sizes = [768 * 768, 3, 50257, 1, 4 * 65536 + 17] + [10] * 40
    ps = [randn(s) for s in sizes]
    gs = [randn(s) for s in sizes]
    ms = [randn(s) * 0.1 for s in sizes]
    vs = [randn(s).abs() * 0.01 for s in sizes]
    vm = [v + 0.001 for v in vs]
    step = 7.0
    tp, tg, tm, tv = ([dev(x) for x in xs] for xs in (ps, gs, ms, vs))
    tvm = [dev(x) for x in vm] if amsgrad else None
    steps = [dev(torch.tensor(step)) for _ in sizes]
    d = _adam_descs(tp, tg, tm, tv, steps, tvm)
    flags = (1 if amsgrad else 0) | (2 if maximize else 0)
    if amsgrad:
        call("mi355x_fused_adamw", d, len(sizes), 6e-4, None, 0.9, 0.95, wd, 1e-8, flags, None, None, None)
        lows = None
    else:
        # the variant that also writes bf16 copies of the updated params (every other one here)
        lows = [torch.empty(s_, dtype=torch.bfloat16, device="cuda") if i % 2 == 0 else None
                for i, s_ in enumerate(sizes)]
        lp = (ctypes.c_void_p * len(sizes))(*[p(x) if x is not None else None for x in lows])
        call("mi355x_fused_adamw_ex", d, lp, CODE[torch.bfloat16], len(sizes), 6e-4, None, 0.9, 0.95, wd, 1e-8,
             flags, None, None, None, None)
        for i, x in enumerate(lows):
            if x is not None:
                assert torch.equal(host(x), host(tp[i]).bfloat16()), i
    for i in range(len(sizes)):
        exp = O.adamw_step(ps[i].numpy(), gs[i].numpy(), ms[i].numpy(), vs[i].numpy(), step, 6e-4, 0.9, 0.95,
                           wd, 1e-8, maximize, amsgrad, vm[i].numpy() if amsgrad else None)
        tol_close(np64(tp[i]), exp[0], atol=1e-6, rtol=1e-5, what=f"p{i}")
        tol_close(np64(tm[i]), exp[1], atol=1e-6, rtol=1e-5, what=f"m{i}")
        tol_close(np64(tv[i]), exp[2], atol=1e-7, rtol=1e-5, what=f"v{i}")


@pytest.mark.parametrize("maximize", [False, True])
def test_fused_adamw_grad_mul_is_the_scale_pass_fused(kernels, maximize):
    """grad_mul (a pending clip_grad_norm_ scale) gives the bits of the
    separate in-place multiply (mi355x_foreach_apply, as _foreach_mul_ runs
    it) followed by the step, and leaves the gradients as they were."""
    sizes = [768 * 768 + 3, 50257, 5, 4 * 65536 + 17]
    ps = [randn(s) for s in sizes]
    gs = [randn(s) for s in sizes]
    ms = [randn(s) * 0.1 for s in sizes]
    vs = [randn(s).abs() * 0.01 for s in sizes]
    coef = dev(torch.tensor(0.3712))
    runs = []
    for fused in (False, True):
        tp, tg, tm, tv = ([dev(x) for x in xs] for xs in (ps, gs, ms, vs))
        steps = [dev(torch.tensor(3.0)) for _ in sizes]
        if not fused:
            call("mi355x_foreach_apply", 2, (ctypes.c_void_p * len(sizes))(*[p(t) for t in tg]), None, None, None,
                 i64(*sizes), len(sizes), CODE[torch.float32], 0.0, p(coef), None)
        d = _adam_descs(tp, tg, tm, tv, steps)
        call("mi355x_fused_adamw_ex", d, None, 0, len(sizes), 6e-4, None, 0.9, 0.95, 0.1, 1e-8,
             2 if maximize else 0, None, None, p(coef) if fused else None, None)
        runs.append((tp, tm, tv, tg))
    for i in range(len(sizes)):
        for a, b in zip(runs[0][:3], runs[1][:3]):
            assert torch.equal(host(a[i]), host(b[i])), i
        assert torch.equal(host(runs[1][3][i]), gs[i]), i


def test_fused_adamw_found_inf_skips_and_wd0_keeps_inf(kernels):
    pp = torch.tensor([float("inf"), 1.0, 2.0])
    tp, tg, tm, tv = dev(pp), dev(torch.ones(3)), dev(torch.zeros(3)), dev(torch.zeros(3))
    step = dev(torch.tensor(1.0))
    fi = dev(torch.tensor(1.0))
    d = _adam_descs([tp], [tg], [tm], [tv], [step])
    call("mi355x_fused_adamw", d, 1, 1e-3, None, 0.9, 0.999, 0.0, 1e-8, 0, None, p(fi), None)
    assert torch.equal(host(tp), pp)
    call("mi355x_fused_adamw", d, 1, 1e-3, None, 0.9, 0.999, 0.0, 1e-8, 0, None, None, None)
    out = host(tp)
    assert math.isinf(out[0].item()) and not math.isnan(out[0].item())


def test_foreach_norm_and_apply(kernels):
    sizes = [100000, 7, 768, 65] + [3] * 70
    xs = [randn(s) for s in sizes]
    tx = [dev(x) for x in xs]
    outs = [torch.empty((), device="cuda") for _ in sizes]
    numels = i64(*sizes)
    ws_n = lib().mi355x_foreach_norm_workspace_bytes(numels, len(sizes))
    ws = workspace(ws_n)
    ptrs_out = (ctypes.c_void_p * len(sizes))(*[p(o) for o in outs])
    ptrs_in = (ctypes.c_void_p * len(sizes))(*[p(t) for t in tx])
    call("mi355x_foreach_norm", ptrs_out, 0, ptrs_in, 0, numels, len(sizes), 2.0, p(ws), ws_n, None)
    for o, x in zip(outs, xs):
        assert abs(host(o).item() - O.l2_norm(x.numpy())) <= 1e-5 * max(1.0, O.l2_norm(x.numpy()))
    coef = dev(torch.tensor(0.25))
    call("mi355x_foreach_apply", 2, ptrs_in, None, None, None, numels, len(sizes), 0, 0.0, p(coef), None)
    for t, x in zip(tx, xs):
        assert torch.equal(host(t), x * 0.25)


@pytest.mark.parametrize("ord_", [float("inf"), 2.0, 1.0])
def test_foreach_norm_propagates_nan(kernels, ord_):
    """A NaN anywhere gives a NaN norm, as torch's does, for every order:
    in a 16-byte-aligned chunk, in the scalar tail and in a second 32768-
    element chunk of a multi-chunk tensor (clip_grad_norm_(norm_type=inf,
    error_if_nonfinite=True) must see NaN gradients)."""
    sizes = [3 * 32768 + 5, 1001, 40000]
    xs = [randn(s) for s in sizes]
    xs[0][70000] = float("nan")   # third chunk, aligned body
    xs[1][1000] = float("nan")    # scalar tail of a 1001-element tensor
    tx = [dev(x) for x in xs]
    n = len(sizes)
    outs = [torch.empty((), device="cuda") for _ in sizes]
    numels = i64(*sizes)
    ws_n = lib().mi355x_foreach_norm_workspace_bytes(numels, n)
    ws = workspace(ws_n)
    ptr = lambda ts: (ctypes.c_void_p * n)(*[p(t) for t in ts])  # noqa: E731
    call("mi355x_foreach_norm", ptr(outs), 0, ptr(tx), 0, numels, n, ord_, p(ws), ws_n, None)
    got = [host(o).item() for o in outs]
    assert math.isnan(got[0]) and math.isnan(got[1]) and math.isfinite(got[2]), got


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_foreach_norm_orders_and_apply_ops(kernels, dtype):
    """Every norm order and the list/scalar forms of ADD, ADDCMUL, LERP and
    SQRT, on sizes that exercise the 16-byte paths, their odd tails and a
    tensor that starts off a 16-byte boundary."""
    sizes = [3 * 32768 + 5, 16384 * 2, 1001, 9]
    base = [randn(s + 1).to(dtype) for s in sizes]
    xs = [b[1:] if i == 3 else b[:-1] for i, b in enumerate(base)]  # the last one is misaligned
    tbase = [dev(b) for b in base]
    tx = [tb[1:] if i == 3 else tb[:-1] for i, tb in enumerate(tbase)]
    numels = i64(*sizes)
    n = len(sizes)
    ws_n = lib().mi355x_foreach_norm_workspace_bytes(numels, n)
    ws = workspace(ws_n)
    ptr = lambda ts: (ctypes.c_void_p * n)(*[p(t) for t in ts])
    for ord_, ref in ((2.0, lambda v: v.double().norm()), (1.0, lambda v: v.double().abs().sum()),
                      (float("inf"), lambda v: v.double().abs().max())):
        outs = [torch.empty((), device="cuda") for _ in sizes]
        call("mi355x_foreach_norm", ptr(outs), 0, ptr(tx), CODE[dtype], numels, n, ord_, p(ws), ws_n, None)
        for o, x in zip(outs, xs):
            r = ref(x).item()
            assert abs(host(o).item() - r) <= 1e-5 * max(1.0, r), (ord_, host(o).item(), r)
    ys = [randn(s).to(dtype) for s in sizes]
    zs = [(randn(s).abs() + 0.5).to(dtype) for s in sizes]
    ty, tz = [dev(y) for y in ys], [dev(z) for z in zs]
    atol = 1e-6 if dtype == torch.float32 else 2e-2
    cur = [x.float() for x in xs]
    call("mi355x_foreach_apply", 0, ptr(tx), ptr(ty), None, None, numels, n, CODE[dtype], 0.5, None, None)
    cur = [(c + 0.5 * y.float()).to(dtype).float() for c, y in zip(cur, ys)]
    scal = (ctypes.c_double * n)(*[0.1 * (i + 1) for i in range(n)])
    call("mi355x_foreach_apply", 41, ptr(tx), ptr(ty), ptr(tz), scal, numels, n, CODE[dtype], 0.0, None, None)
    cur = [(c + 0.1 * (i + 1) * y.float() * z.float()).to(dtype).float() for i, (c, y, z) in enumerate(zip(cur, ys, zs))]
    call("mi355x_foreach_apply", 43, ptr(tx), ptr(tz), None, None, numels, n, CODE[dtype], 0.25, None, None)
    cur = [(c + 0.25 * (z.float() - c)).to(dtype).float() for c, z in zip(cur, zs)]
    cur = [c.abs() for c in cur]
    for t, c in zip(tx, cur):
        t.copy_(c.to(dtype).to(t.device))
    call("mi355x_foreach_apply", 65, ptr(tx), None, None, None, numels, n, CODE[dtype], 0.0, None, None)
    cur = [c.sqrt().to(dtype).float() for c in cur]
    for i, (t, c) in enumerate(zip(tx, cur)):
        tol_close(host(t).float().numpy(), c.double().numpy(), atol=atol, rtol=atol, what=f"apply {i}")
    # the misaligned tensor's neighbours in its base allocation are untouched
    assert torch.equal(host(tbase[3])[:1], base[3][:1])


@pytest.mark.parametrize("cols", [1152, 256, 100])
@pytest.mark.parametrize("dtype,wdt", [(torch.float32, torch.float32), (torch.bfloat16, torch.float32),
                                        (torch.bfloat16, torch.bfloat16)])
def test_rms_norm_fwd_matches_oracle(kernels, cols, dtype, wdt):
    rows = 37
    x = (randn(rows, cols) * 2.0).to(dtype)
    w = (1.0 + 0.1 * randn(cols)).to(wdt)
    y = torch.empty(rows, cols, dtype=dtype, device="cuda")
    rstd = torch.empty(rows, device="cuda")
    tx, tw = dev(x), dev(w)  # held: a freed temporary's memory would be reused by the next allocation
    call("mi355x_rms_norm_fwd", p(y), p(rstd), p(tx), p(tw), CODE[wdt], 0.0, rows, cols, 1e-6, CODE[dtype], None)
    ey, er = O.rms_norm(x.double().numpy(), w.double().numpy(), eps=1e-6)
    tol = 1e-5 if dtype == torch.float32 else 1e-2
    tol_close(np64(y), ey, atol=tol, rtol=tol, what="y")
    tol_close(np64(rstd), er, atol=1e-6, rtol=1e-5, what="rstd")


@pytest.mark.parametrize("rows,cols", [(37, 1152), (37, 256), (37, 100), (4096, 1152)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_rms_norm_bwd_matches_oracle(kernels, rows, cols, dtype):
    """The fused rms_norm backward (Gemma's 1 + w scale) against the f64
    oracle, from the forward's own rstd; (4096, 1152) is the Gemma-3-1B
    residual norm of a 4096-token sequence."""
    x = (randn(rows, cols) * 2.0).to(dtype)
    w = (0.1 * randn(cols)).to(dtype)
    dy = randn(rows, cols).to(dtype)
    tx, tw, tdy = dev(x), dev(w), dev(dy)
    y = torch.empty(rows, cols, dtype=dtype, device="cuda")
    rstd = torch.empty(rows, device="cuda")
    call("mi355x_rms_norm_fwd", p(y), p(rstd), p(tx), p(tw), CODE[dtype], 1.0, rows, cols, 1e-6, CODE[dtype], None)
    dx = torch.empty(rows, cols, dtype=dtype, device="cuda")
    dw = torch.empty(cols, dtype=dtype, device="cuda")
    ws_n = lib().mi355x_layer_norm_bwd_workspace_bytes(rows, cols)
    ws = workspace(ws_n)
    call("mi355x_rms_norm_bwd", p(dx), p(dw), p(tdy), p(tx), p(rstd), p(tw), 1.0, rows, cols, CODE[dtype],
         p(ws), ws_n, None)
    edx, edw = O.rms_norm_backward(dy.double().numpy(), x.double().numpy(), w.double().numpy(), eps=1e-6,
                                   weight_offset=1.0)
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    tol_close(np64(dx), edx, atol=tol, rtol=tol, what="dx")
    tol_close(np64(dw), edw, atol=tol * math.sqrt(rows), rtol=tol, what="dw")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_rope_forward_and_inverse(kernels, dtype):
    """Rotary embedding on a [B,H,T,D] view with BTHD storage: against the
    rotate_half formula, and inverse(forward(x)) = x on a true rotation."""
    B, H, T, D = 2, 3, 37, 64
    xs = randn(B, T, H, D).to(dtype)
    x = dev(xs).transpose(1, 2)
    inv = 1.0 / (10000.0 ** (torch.arange(0, D, 2, dtype=torch.float64) / D))
    ang = torch.arange(T, dtype=torch.float64)[:, None] * inv[None, :]
    ang = torch.cat([ang, ang], -1)
    cos, sin = dev(ang.cos().to(dtype)), dev(ang.sin().to(dtype))
    y = torch.empty(B, T, H, D, dtype=dtype, device="cuda").transpose(1, 2)
    z = torch.empty_like(y)
    call("mi355x_rope", p(y), i64(*y.stride()[:3]), p(x), i64(*x.stride()[:3]), p(cos), p(sin), B, H, T, D, 0,
         CODE[dtype], None)
    call("mi355x_rope", p(z), i64(*z.stride()[:3]), p(y), i64(*y.stride()[:3]), p(cos), p(sin), B, H, T, D, 1,
         CODE[dtype], None)
    xf = xs.double().transpose(1, 2)
    c, sn = host(cos).double(), host(sin).double()
    want = xf * c + torch.cat([-xf[..., D // 2:], xf[..., :D // 2]], -1) * sn
    tol = 1e-5 if dtype == torch.float32 else 1e-2
    tol_close(np64(y), want.numpy(), atol=tol, rtol=tol, what="rope")
    tol_close(np64(z), xf.numpy(), atol=2 * tol, rtol=2 * tol, what="inverse")


@pytest.mark.parametrize("approximate", [0, 1])
def test_geglu_bit_exact_vs_gelu_then_mul(kernels, approximate):
    n = 4096 + 5
    gate, up = dev(randn(n).bfloat16()), dev(randn(n).bfloat16())
    y = torch.empty(n, dtype=torch.bfloat16, device="cuda")
    call("mi355x_geglu_fwd", p(y), p(gate), p(up), n, approximate, CODE[torch.bfloat16], None)
    a = torch.empty_like(y)
    call("mi355x_gelu_fwd", p(a), p(gate), n, approximate, CODE[torch.bfloat16], None)
    want = (host(a).float() * host(up).float()).bfloat16()
    assert torch.equal(host(y), want)


@pytest.mark.parametrize("approximate", [0, 1])
@pytest.mark.parametrize("n", [4096 + 5, 4096 * 6912])
def test_geglu_bwd_bit_exact_vs_its_aten_chain(kernels, approximate, n):
    """The fused GeGLU backward against the kernels of the chain it replaces
    (d_up = grad * gelu(gate), d_gate = gelu_backward(grad * up, gate), each
    product rounded to bf16): bit-exact; n = 4096 x 6912 is a Gemma-3-1B MLP
    activation of a 4096-token sequence."""
    grad, gate, up = (dev((randn(n) * 2).bfloat16()) for _ in range(3))
    dg, du = torch.empty_like(gate), torch.empty_like(gate)
    call("mi355x_geglu_bwd", p(dg), p(du), p(grad), p(gate), p(up), n, approximate, CODE[torch.bfloat16], None)
    a = torch.empty_like(gate)
    call("mi355x_gelu_fwd", p(a), p(gate), n, approximate, CODE[torch.bfloat16], None)
    want_du = (host(a).float() * host(grad).float()).bfloat16()
    gu = dev((host(grad).float() * host(up).float()).bfloat16())
    want_dg = torch.empty_like(gate)
    call("mi355x_gelu_bwd", p(want_dg), p(gu), p(gate), n, approximate, CODE[torch.bfloat16], None)
    assert torch.equal(host(du), want_du)
    assert torch.equal(host(dg), host(want_dg))


def test_multi_tensor_kernels_across_batches_with_empty_tensors(kernels):
    """Lists longer than one launch's 160 tensors, with empty tensors among
    them (first, inside a batch and at a batch boundary): foreach norm,
    foreach apply and fused AdamW locate every chunk of every tensor."""
    g = torch.Generator().manual_seed(12)
    sizes = [0] + [int(s) for s in torch.randint(1, 3000, (158,), generator=g)] + [0, 0, 5000] + \
            [int(s) for s in torch.randint(0, 40, (200,), generator=g)] + [70000, 0]
    xs = [torch.randn(s, generator=g) for s in sizes]
    tx = [dev(x) for x in xs]
    n = len(sizes)
    outs = [torch.empty((), device="cuda") for _ in sizes]
    numels = i64(*sizes)
    ws_n = lib().mi355x_foreach_norm_workspace_bytes(numels, n)
    ws = workspace(ws_n)
    ptrs_out = (ctypes.c_void_p * n)(*[p(o) for o in outs])
    ptrs_in = (ctypes.c_void_p * n)(*[p(t) for t in tx])
    call("mi355x_foreach_norm", ptrs_out, 0, ptrs_in, 0, numels, n, 2.0, p(ws), ws_n, None)
    for i, (o, x) in enumerate(zip(outs, xs)):
        assert abs(host(o).item() - x.double().norm().item()) <= 1e-5 * max(1.0, x.double().norm().item()), i
    coef = dev(torch.tensor(0.5))
    call("mi355x_foreach_apply", 2, ptrs_in, None, None, None, numels, n, 0, 0.0, p(coef), None)
    for i, (t, x) in enumerate(zip(tx, xs)):
        assert torch.equal(host(t), x * 0.5), i
    gs = [torch.randn(s, generator=g) for s in sizes]
    ms = [torch.zeros(s) for s in sizes]
    vs = [torch.zeros(s) for s in sizes]
    tg, tm, tv = ([dev(x) for x in xs_] for xs_ in (gs, ms, vs))
    steps = [dev(torch.tensor(1.0)) for _ in sizes]
    d = _adam_descs(tx, tg, tm, tv, steps)
    call("mi355x_fused_adamw", d, n, 1e-3, None, 0.9, 0.999, 0.01, 1e-8, 0, None, None, None)
    for i in range(n):
        exp = O.adamw_step((xs[i] * 0.5).numpy(), gs[i].numpy(), ms[i].numpy(), vs[i].numpy(), 1.0, 1e-3, 0.9,
                           0.999, 0.01, 1e-8, False, False, None)
        tol_close(np64(tx[i]), exp[0], atol=1e-6, rtol=1e-5, what=f"p{i}")
