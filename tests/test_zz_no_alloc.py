"""mi355x_attn_bwd_noalloc (the entry point that allocates nothing) against
mi355x_attn_bwd with a caller workspace, through the C ABI: bit-identical
gradients on two calls in a row, the second with a smaller input (the
scratch array keeps the first call's contents), and the size limit."""

import math

import pytest
import torch

from abi import CODE, bhs, call, dev, host, lib, p  # noqa: F401
from test_gpu_gemm_attention import _attn_bwd, _attn_fwd

pytestmark = pytest.mark.gpu


def _bwd_noalloc(do, q, k, v, o, lse, causal):
    B, H, Sq, D = q.shape
    Skv = k.shape[2]
    dq = torch.empty(B, Sq, H, D, dtype=q.dtype, device="cuda").transpose(1, 2)
    dk = torch.empty(B, Skv, H, D, dtype=q.dtype, device="cuda").transpose(1, 2)
    dv = torch.empty(B, Skv, H, D, dtype=q.dtype, device="cuda").transpose(1, 2)
    call("mi355x_attn_bwd_noalloc", p(dq), bhs(dq), p(dk), bhs(dk), p(dv), bhs(dv), p(do), bhs(do),
         p(q), bhs(q), p(k), bhs(k), p(v), bhs(v), p(o), bhs(o), p(lse),
         B, H, Sq, Skv, D, 1.0 / math.sqrt(D), int(causal), CODE[q.dtype], None)
    return dq, dk, dv


@pytest.mark.parametrize("causal", [True, False])
def test_attn_bwd_noalloc_matches_workspace_entry(kernels, causal):
    g = torch.Generator().manual_seed(77)
    for shape in ((2, 12, 1024, 64), (1, 3, 200, 64)):  # second call smaller
        B, H, S, D = shape
        q, k, v, do = (dev(torch.randn(B, H, S, D, generator=g).bfloat16()) for _ in range(4))
        o, lse = _attn_fwd(q, k, v, causal)
        ref = _attn_bwd(do, q, k, v, o, lse, causal)
        got = _bwd_noalloc(do, q, k, v, o, lse, causal)
        for name, a, b in zip(("dq", "dk", "dv"), got, ref):
            assert torch.equal(host(a), host(b)), f"{name} differs at {shape}"


def test_attn_bwd_noalloc_rejects_shapes_beyond_its_scratch(kernels):
    t = dev(torch.zeros(1, 1, 64, 64).bfloat16())
    lse = torch.zeros(1, 1, 64, device="cuda")
    s = bhs(t)
    # 4096 * 1024 query rows need 32 MiB + 256 bytes: one row too many is refused before any launch
    rc = lib().mi355x_attn_bwd_noalloc(p(t), s, p(t), s, p(t), s, p(t), s, p(t), s, p(t), s, p(t), s, p(t), s,
                                       p(lse), 4096, 1024, 1, 1, 64, 0.125, 1, CODE[torch.bfloat16], None)
    assert rc != 0 and b"scratch" in lib().mi355x_last_error()
