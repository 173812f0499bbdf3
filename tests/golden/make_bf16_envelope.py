"""Write the stock-PyTorch bf16-autocast loss envelope of the headline run.

Runs on a GPU box with stock PyTorch-ROCm (the `cuda` device; neither the
mojo device nor this repository's kernels are involved): the nanoGPT-124M
run of tests/golden/loss_curve_b16_t1024_f32cpu.json (same seed, weights,
batches, optimizer and clip), under bf16 autocast, once as is and once per
perturbation seed with every initial weight scaled by (1 + 1e-6 N(0, 1)).
The spread of these curves is how far bf16 rounding alone moves this run
from the f32 curve; the device's bf16 curve is tested against it.

    python tests/golden/make_bf16_envelope.py [--seeds 12] [--steps 50]
"""

import argparse
import json
import sys
import time
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT / "torch-mojo-backend_amd"))

from torch_mojo_backend.gpt2 import (  # noqa: E402
    BETAS, GRAD_CLIP, LEARNING_RATE, WEIGHT_DECAY, GPT, GPTConfig, make_batches, training_step,
)

FIXTURE = Path(__file__).with_name("loss_curve_b16_t1024_f32cpu.json")


def run_curve(cfg, perturb_seed, steps):
    torch.manual_seed(cfg["seed"])
    model = GPT(GPTConfig())
    if perturb_seed is not None:
        g = torch.Generator().manual_seed(perturb_seed)
        with torch.no_grad():
            for p in model.parameters():
                p.mul_(1.0 + 1e-6 * torch.randn(p.shape, generator=g))
    model.to("cuda")
    opt = model.configure_optimizers(WEIGHT_DECAY, LEARNING_RATE, BETAS, fused=True)
    batches = make_batches(cfg["batch"], cfg["block"], cfg["vocab"], cfg["batches_cycled"], cfg["data_seed"], "cuda")
    losses = []
    for step in range(steps):
        x, y = batches[step % len(batches)]
        loss = training_step(model, opt, x, y, autocast_dtype=torch.bfloat16, device_type="cuda", grad_clip=GRAD_CLIP)
        losses.append(loss.item())
    return losses


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--seeds", type=int, default=12)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--out", default=str(Path(__file__).with_name("loss_envelope_b16_t1024_bf16_torch.json")))
    args = ap.parse_args()
    assert torch.cuda.is_available(), "needs a GPU with stock PyTorch-ROCm"
    cfg = json.loads(FIXTURE.read_text())["config"]
    curves = {}
    for s in [None] + list(range(1, args.seeds + 1)):
        t0 = time.perf_counter()
        curves["unperturbed" if s is None else f"seed{s}"] = run_curve(cfg, s, args.steps)
        print(s, f"{time.perf_counter() - t0:.1f}s", flush=True)
    vals = list(curves.values())
    out = {
        "config": dict(cfg, dtype="bfloat16 autocast", device=torch.cuda.get_device_name(0), torch=torch.__version__,
                       perturbation="initial weights * (1 + 1e-6 N(0,1)) per seed"),
        "curves": curves,
        "lo": [min(c[i] for c in vals) for i in range(args.steps)],
        "hi": [max(c[i] for c in vals) for i in range(args.steps)],
    }
    Path(args.out).write_text(json.dumps(out, indent=1))


if __name__ == "__main__":
    main()
