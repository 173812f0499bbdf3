"""Write tests/golden/golden_ops.npz: seeded tiny inputs and the outputs stock
PyTorch CPU ATen computes for them.

Stock PyTorch CPU in f32 is the reference's own oracle for every hot-path op
(torch_mojo_backend/testing.py:186-229, tests/test_eager_kernels.py:
10083-10094, tests/test_eager_optimizer_ops.py:65-435); the reference ships
no golden vectors of its own, so these fixtures record that oracle's outputs
once, with the torch version that produced them.  They pin oracle/ops.py in
tests/test_oracle.py.

    python tests/golden/make_golden.py
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import torch
import torch.nn.functional as F

OUT = Path(__file__).with_name("golden_ops.npz")


def main():
    g = torch.Generator().manual_seed(20260718)
    rnd = lambda *s: torch.randn(s, generator=g)  # noqa: E731
    d: dict[str, np.ndarray] = {}

    def put(name, t):
        d[name] = t.detach().clone().numpy() if isinstance(t, torch.Tensor) else np.asarray(t)

    # layer norm [5, 24], affine, eps 1e-5: fwd, mean, rstd, and the three grads
    x = rnd(5, 24).requires_grad_()
    w = (1 + 0.1 * rnd(24)).requires_grad_()
    b = (0.1 * rnd(24)).requires_grad_()
    y, mean, rstd = torch.ops.aten.native_layer_norm(x, [24], w, b, 1e-5)
    dy = rnd(5, 24)
    y.backward(dy)
    for k, v in dict(x=x, w=w, b=b, y=y, mean=mean, rstd=rstd, dy=dy, dx=x.grad, dw=w.grad, db=b.grad).items():
        put("ln_" + k, v)

    # GELU exact and tanh, fwd + bwd, [64] over [-6, 6]
    for approx in ("none", "tanh"):
        x = torch.linspace(-6, 6, 64).requires_grad_()
        y = F.gelu(x, approximate=approx)
        dy = rnd(64)
        y.backward(dy)
        for k, v in dict(x=x, y=y, dy=dy, dx=x.grad).items():
            put(f"gelu_{approx}_{k}", v)

    # softmax / log_softmax over the last dim of [4, 33], fwd + bwd
    for name, fn in (("softmax", torch.softmax), ("log_softmax", torch.log_softmax)):
        x = (3 * rnd(4, 33)).requires_grad_()
        y = fn(x, -1)
        dy = rnd(4, 33)
        y.backward(dy)
        for k, v in dict(x=x, y=y, dy=dy, dx=x.grad).items():
            put(f"{name}_{k}", v)

    # NLL on log-probabilities [7, 11], with ignore_index and class weights
    logp = torch.log_softmax(rnd(7, 11), -1)
    tgt = torch.tensor([3, 0, 10, -100, 5, 5, 1])
    wt = torch.rand(11, generator=g) + 0.5
    put("nll_logp", logp)
    put("nll_target", tgt)
    put("nll_weight", wt)
    for red in ("mean", "sum", "none"):
        for use_w in (False, True):
            lp = logp.clone().requires_grad_()
            out = F.nll_loss(lp, tgt, weight=wt if use_w else None, reduction=red, ignore_index=-100)
            gout = rnd(*out.shape)
            out.backward(gout)
            tag = f"nll_{red}_{'w' if use_w else 'nw'}"
            put(tag + "_out", out)
            put(tag + "_gout", gout)
            put(tag + "_dlogp", lp.grad)

    # embedding [13, 6] gathered at [3, 5] ids with repeats; dense backward
    wgt = rnd(13, 6).requires_grad_()
    ids = torch.tensor([[1, 4, 4, 12, 0], [7, 1, 1, 1, 3], [12, 12, 2, 9, 4]])
    e = F.embedding(ids, wgt)
    de = rnd(3, 5, 6)
    e.backward(de)
    for k, v in dict(weight=wgt, ids=ids, out=e, dout=de, dweight=wgt.grad).items():
        put("emb_" + k, v)

    # SDPA f32: causal square, non-causal, causal Sq != Skv (top-left), fwd + bwd
    for tag, (B, H, Sq, Skv, D), causal in (("causal", (2, 2, 9, 9, 8), True),
                                            ("full", (1, 3, 6, 10, 4), False),
                                            ("rect", (2, 2, 5, 7, 3), True)):
        q, k, v = (rnd(B, H, s, D).requires_grad_() for s in (Sq, Skv, Skv))
        o = F.scaled_dot_product_attention(q, k, v, is_causal=causal)
        do = rnd(B, H, Sq, D)
        o.backward(do)
        s = (q @ k.transpose(-1, -2)) / D**0.5
        if causal:
            s = s.masked_fill(torch.ones(Sq, Skv, dtype=torch.bool).triu(1), float("-inf"))
        lse = torch.logsumexp(s, -1)
        for kk, vv in dict(q=q, k=k, v=v, o=o, lse=lse, do=do, dq=q.grad, dk=k.grad, dv=v.grad).items():
            put(f"sdpa_{tag}_{kk}", vv)

    # addmm [6, 5] = bias + [6, 9] @ [9, 5]
    a, bm, bias = rnd(6, 9), rnd(9, 5), rnd(5)
    for k, v in dict(a=a, b=bm, bias=bias, out=torch.addmm(bias, a, bm)).items():
        put("addmm_" + k, v)

    # AdamW, fused CPU kernel, two steps on one [40] param
    p = rnd(40).requires_grad_()
    put("adamw_p0", p)
    opt = torch.optim.AdamW([p], lr=6e-4, betas=(0.9, 0.95), weight_decay=0.1, eps=1e-8, fused=True)
    for i in range(2):
        gr = rnd(40)
        put(f"adamw_g{i}", gr)
        p.grad = gr.clone()
        opt.step()
        put(f"adamw_p{i + 1}", p)
    st = opt.state[p]
    put("adamw_m2", st["exp_avg"])
    put("adamw_v2", st["exp_avg_sq"])

    # _foreach_norm over two tensors (clip_grad_norm_'s total norm)
    t1, t2 = rnd(17), rnd(3, 5)
    put("norm_t1", t1)
    put("norm_t2", t2)
    put("norm_total", torch.linalg.vector_norm(torch.stack(torch._foreach_norm([t1, t2]))))

    d["torch_version"] = np.array(torch.__version__)
    np.savez_compressed(OUT, **d)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(d)} arrays)")


if __name__ == "__main__":
    main()
