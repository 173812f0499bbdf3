"""GPT-2 small (nanoGPT-shaped) model used by the benchmark and the
end-to-end tests.

The reference times nanoGPT's own `model.py` imported from a local checkout
(current_bench/bench_nanogpt_train.py:33,49-60,117-150); that checkout is not
available here, so this is an independent module with the same architecture
and training semantics: pre-LayerNorm blocks, fused qkv projection, causal
`scaled_dot_product_attention`, exact-erf GELU MLP (4x), final LayerNorm,
lm_head tied to the token embedding, N(0, 0.02) init with the residual
projections scaled by 1/sqrt(2*n_layer), cross-entropy over the vocabulary,
and AdamW with decay on >=2-D parameters only.  It is plain PyTorch: it runs
unchanged on "cpu" (the fp32 oracle run) and on "mojo".
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn as nn
import torch.nn.functional as F


@dataclass
class GPTConfig:
    block_size: int = 1024
    vocab_size: int = 50257
    n_layer: int = 12
    n_head: int = 12
    n_embd: int = 768
    bias: bool = True


class CausalSelfAttention(nn.Module):
    def __init__(self, cfg: GPTConfig):
        super().__init__()
        assert cfg.n_embd % cfg.n_head == 0
        self.c_attn = nn.Linear(cfg.n_embd, 3 * cfg.n_embd, bias=cfg.bias)
        self.c_proj = nn.Linear(cfg.n_embd, cfg.n_embd, bias=cfg.bias)
        self.n_head = cfg.n_head
        self.n_embd = cfg.n_embd

    def forward(self, x):
        B, T, C = x.shape
        q, k, v = self.c_attn(x).split(self.n_embd, dim=2)
        hd = C // self.n_head
        q = q.view(B, T, self.n_head, hd).transpose(1, 2)
        k = k.view(B, T, self.n_head, hd).transpose(1, 2)
        v = v.view(B, T, self.n_head, hd).transpose(1, 2)
        y = F.scaled_dot_product_attention(q, k, v, attn_mask=None, dropout_p=0.0, is_causal=True)
        y = y.transpose(1, 2).contiguous().view(B, T, C)
        return self.c_proj(y)


class MLP(nn.Module):
    def __init__(self, cfg: GPTConfig):
        super().__init__()
        self.c_fc = nn.Linear(cfg.n_embd, 4 * cfg.n_embd, bias=cfg.bias)
        self.gelu = nn.GELU()
        self.c_proj = nn.Linear(4 * cfg.n_embd, cfg.n_embd, bias=cfg.bias)

    def forward(self, x):
        return self.c_proj(self.gelu(self.c_fc(x)))


class Block(nn.Module):
    def __init__(self, cfg: GPTConfig):
        super().__init__()
        self.ln_1 = nn.LayerNorm(cfg.n_embd, bias=cfg.bias)
        self.attn = CausalSelfAttention(cfg)
        self.ln_2 = nn.LayerNorm(cfg.n_embd, bias=cfg.bias)
        self.mlp = MLP(cfg)

    def forward(self, x):
        x = x + self.attn(self.ln_1(x))
        x = x + self.mlp(self.ln_2(x))
        return x


class GPT(nn.Module):
    def __init__(self, cfg: GPTConfig):
        super().__init__()
        self.config = cfg
        self.transformer = nn.ModuleDict(
            dict(
                wte=nn.Embedding(cfg.vocab_size, cfg.n_embd),
                wpe=nn.Embedding(cfg.block_size, cfg.n_embd),
                h=nn.ModuleList([Block(cfg) for _ in range(cfg.n_layer)]),
                ln_f=nn.LayerNorm(cfg.n_embd, bias=cfg.bias),
            )
        )
        self.lm_head = nn.Linear(cfg.n_embd, cfg.vocab_size, bias=False)
        self.transformer.wte.weight = self.lm_head.weight  # tied
        self.apply(self._init_weights)
        for name, p in self.named_parameters():
            if name.endswith("c_proj.weight"):
                nn.init.normal_(p, mean=0.0, std=0.02 / math.sqrt(2 * cfg.n_layer))

    @staticmethod
    def _init_weights(module):
        if isinstance(module, nn.Linear):
            nn.init.normal_(module.weight, mean=0.0, std=0.02)
            if module.bias is not None:
                nn.init.zeros_(module.bias)
        elif isinstance(module, nn.Embedding):
            nn.init.normal_(module.weight, mean=0.0, std=0.02)

    def num_params(self) -> int:
        return sum(p.numel() for p in self.parameters())

    def forward(self, idx, targets=None):
        b, t = idx.shape
        pos = torch.arange(0, t, dtype=torch.long, device=idx.device)
        x = self.transformer.wte(idx) + self.transformer.wpe(pos)
        for block in self.transformer.h:
            x = block(x)
        x = self.transformer.ln_f(x)
        logits = self.lm_head(x)
        loss = None
        if targets is not None:
            loss = F.cross_entropy(logits.view(-1, logits.size(-1)), targets.view(-1), ignore_index=-1)
        return logits, loss

    def configure_optimizers(self, weight_decay, learning_rate, betas, fused=True):
        params = [p for p in self.parameters() if p.requires_grad]
        decay = [p for p in params if p.dim() >= 2]
        nodecay = [p for p in params if p.dim() < 2]
        groups = [
            {"params": decay, "weight_decay": weight_decay},
            {"params": nodecay, "weight_decay": 0.0},
        ]
        kwargs = {"fused": True} if fused else {"foreach": False}
        return torch.optim.AdamW(groups, lr=learning_rate, betas=betas, **kwargs)


# nanoGPT train.py hyper-parameters (bench_nanogpt_train.py:36-40)
WEIGHT_DECAY = 0.1
LEARNING_RATE = 6e-4
BETAS = (0.9, 0.95)
GRAD_CLIP = 1.0


def make_batches(batch_size, block_size, vocab_size, count, seed, device):
    """Seeded uniform token ids on the host, copied to `device`; targets are
    the ids shifted by one (bench_nanogpt_train.py:90-108)."""
    g = torch.Generator().manual_seed(seed)
    out = []
    for _ in range(count):
        tokens = torch.randint(0, vocab_size, (batch_size, block_size + 1), generator=g)
        out.append((tokens[:, :-1].contiguous().to(device), tokens[:, 1:].contiguous().to(device)))
    return out


def training_step(model, optimizer, inputs, targets, autocast_dtype=None, device_type="mojo",
                  grad_clip=GRAD_CLIP):
    """nanoGPT's train.py loop body: forward (optionally under autocast),
    backward, clip_grad_norm_, optimizer step, zero_grad(set_to_none)."""
    if autocast_dtype is not None:
        with torch.autocast(device_type=device_type, dtype=autocast_dtype):
            _, loss = model(inputs, targets)
    else:
        _, loss = model(inputs, targets)
    loss.backward()
    if grad_clip:
        torch.nn.utils.clip_grad_norm_(model.parameters(), grad_clip)
    optimizer.step()
    optimizer.zero_grad(set_to_none=True)
    return loss
