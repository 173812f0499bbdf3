"""Write the f32 CPU loss curve of the nanoGPT-124M training run (fixture).

BASELINE config 3 shapes: GPT-2 small (12 layers, 768 wide, 12 heads, vocab
50257, bias, tied lm_head), batch 16 x 1024 tokens of seeded uniform ids
(2 batches cycled, as current_bench/bench_nanogpt_train.py does with its
default --batches 2), AdamW(lr 6e-4, betas (0.9, 0.95), wd 0.1 on >=2-D
params, fused CPU kernel), clip_grad_norm_ 1.0, 50 steps, seed 1337.
Stock PyTorch CPU in f32 is the reference's own oracle for this run.

    python tests/golden/make_loss_curve.py [--steps 50] [--out ...]
"""

import argparse
import json
import os
import sys
import time
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT / "torch-mojo-backend_amd"))

from torch_mojo_backend.gpt2 import (  # noqa: E402
    BETAS, GRAD_CLIP, LEARNING_RATE, WEIGHT_DECAY, GPT, GPTConfig, make_batches, training_step,
)

SEED = 1337
DATA_SEED = 20260718


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--batch", type=int, default=16)
    ap.add_argument("--block", type=int, default=1024)
    ap.add_argument("--out", default=str(Path(__file__).with_name("loss_curve_b16_t1024_f32cpu.json")))
    args = ap.parse_args()
    torch.set_num_threads(os.cpu_count())
    torch.manual_seed(SEED)
    model = GPT(GPTConfig())
    opt = model.configure_optimizers(WEIGHT_DECAY, LEARNING_RATE, BETAS, fused=True)
    batches = make_batches(args.batch, args.block, 50257, 2, DATA_SEED, "cpu")
    losses, times = [], []
    for step in range(args.steps):
        x, y = batches[step % len(batches)]
        t0 = time.perf_counter()
        loss = training_step(model, opt, x, y, grad_clip=GRAD_CLIP)
        times.append(time.perf_counter() - t0)
        losses.append(loss.item())
        print(step, losses[-1], f"{times[-1]:.1f}s", flush=True)
    out = {
        "config": {"batch": args.batch, "block": args.block, "vocab": 50257, "n_layer": 12,
                   "n_embd": 768, "n_head": 12, "seed": SEED, "data_seed": DATA_SEED,
                   "batches_cycled": 2, "dtype": "float32", "device": "cpu",
                   "torch": torch.__version__, "threads": torch.get_num_threads()},
        "losses": losses,
        "step_seconds": times,
    }
    Path(args.out).write_text(json.dumps(out, indent=1))


if __name__ == "__main__":
    main()
