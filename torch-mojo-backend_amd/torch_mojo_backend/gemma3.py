"""A Gemma-3-1B-shaped decoder for the prefill workload (forward only).

The shapes are those of Gemma 3 1B: 26 layers, d_model 1152, 4 query heads
sharing 1 K/V head (grouped-query attention), head_dim 256, GeGLU MLP with
d_ff 6912, RMSNorm before and after each sub-block plus on q and k,
rotary position embeddings (base 10k on local layers, 1M on global ones),
five local sliding-window (512) layers to each global causal layer, a tied
262144-entry embedding scaled by sqrt(d_model), bf16.  Weights are random
N(0, 0.02); there is no checkpoint loading (no network).

The model is written with plain torch ops so that it runs unchanged on the
CPU (the parity reference) and on the mojo device, where the ops land on the
gfx950 kernels: linear -> GEMM, RMSNorm (1 + w) -> the fused RMSNorm, SDPA
with enable_gqa / a sliding-window mask from torch_mojo_backend.masks -> the
grouped-query windowed flash forward, RoPE and GeGLU -> their fused kernels
(torch_mojo_backend.ops, which falls back to the plain formulas off the
device).
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import ops
from .masks import sliding_window_causal_mask


@dataclass
class Gemma3Config:
    vocab_size: int = 262144
    hidden: int = 1152
    layers: int = 26
    heads: int = 4
    kv_heads: int = 1
    head_dim: int = 256
    d_ff: int = 6912
    window: int = 512
    global_every: int = 6  # layers 5, 11, 17, 23 are global: five local to one global
    rope_local_base: float = 10000.0
    rope_global_base: float = 1000000.0
    eps: float = 1e-6


class RMSNorm(nn.Module):
    """Gemma's RMSNorm: x / rms(x) * (1 + weight), statistics and scale in f32,
    result in x's dtype."""

    def __init__(self, dim, eps):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.zeros(dim))

    def forward(self, x):
        return ops.rms_norm(x, self.weight, self.eps, weight_offset=1.0)


def rope_tables(seq_len, dim, base, device, dtype):
    """cos, sin [seq_len, dim] of the half-split rotary embedding."""
    inv = 1.0 / (base ** (torch.arange(0, dim, 2, dtype=torch.float64) / dim))
    ang = torch.arange(seq_len, dtype=torch.float64)[:, None] * inv[None, :]
    ang = torch.cat([ang, ang], dim=-1)
    return ang.cos().to(dtype).to(device), ang.sin().to(dtype).to(device)


def apply_rope(x, cos, sin):
    """x * cos + rotate_half(x) * sin (one fused kernel on the mojo device)."""
    return ops.rotary_embedding(x, cos, sin)


class Attention(nn.Module):
    def __init__(self, cfg: Gemma3Config, local: bool):
        super().__init__()
        self.cfg, self.local = cfg, local
        h, hk, d = cfg.heads, cfg.kv_heads, cfg.head_dim
        self.q_proj = nn.Linear(cfg.hidden, h * d, bias=False)
        self.k_proj = nn.Linear(cfg.hidden, hk * d, bias=False)
        self.v_proj = nn.Linear(cfg.hidden, hk * d, bias=False)
        self.o_proj = nn.Linear(h * d, cfg.hidden, bias=False)
        self.q_norm = RMSNorm(d, cfg.eps)
        self.k_norm = RMSNorm(d, cfg.eps)

    def forward(self, x, rope, mask):
        b, t, _ = x.shape
        c = self.cfg
        # the per-head norms run on the projections' dense [B, T, H, D] rows,
        # before the head transpose (the same rows, no copy)
        q = self.q_norm(self.q_proj(x).view(b, t, c.heads, c.head_dim)).transpose(1, 2)
        k = self.k_norm(self.k_proj(x).view(b, t, c.kv_heads, c.head_dim)).transpose(1, 2)
        v = self.v_proj(x).view(b, t, c.kv_heads, c.head_dim).transpose(1, 2)
        cos, sin = rope
        q, k = apply_rope(q, cos, sin), apply_rope(k, cos, sin)
        scale = 1.0 / math.sqrt(c.head_dim)
        if self.local:
            y = F.scaled_dot_product_attention(q, k, v, attn_mask=mask, scale=scale, enable_gqa=True)
        else:
            y = F.scaled_dot_product_attention(q, k, v, is_causal=True, scale=scale, enable_gqa=True)
        return self.o_proj(y.transpose(1, 2).reshape(b, t, c.heads * c.head_dim))


class MLP(nn.Module):
    def __init__(self, cfg: Gemma3Config):
        super().__init__()
        self.gate_proj = nn.Linear(cfg.hidden, cfg.d_ff, bias=False)
        self.up_proj = nn.Linear(cfg.hidden, cfg.d_ff, bias=False)
        self.down_proj = nn.Linear(cfg.d_ff, cfg.hidden, bias=False)

    def forward(self, x):
        return self.down_proj(ops.geglu(self.gate_proj(x), self.up_proj(x), approximate="tanh"))


class Block(nn.Module):
    def __init__(self, cfg: Gemma3Config, local: bool):
        super().__init__()
        self.local = local
        self.input_norm = RMSNorm(cfg.hidden, cfg.eps)
        self.attn = Attention(cfg, local)
        self.post_attn_norm = RMSNorm(cfg.hidden, cfg.eps)
        self.pre_ffw_norm = RMSNorm(cfg.hidden, cfg.eps)
        self.mlp = MLP(cfg)
        self.post_ffw_norm = RMSNorm(cfg.hidden, cfg.eps)

    def forward(self, x, rope_local, rope_global, mask):
        rope = rope_local if self.local else rope_global
        x = x + self.post_attn_norm(self.attn(self.input_norm(x), rope, mask))
        return x + self.post_ffw_norm(self.mlp(self.pre_ffw_norm(x)))


class Gemma3(nn.Module):
    def __init__(self, cfg: Gemma3Config):
        super().__init__()
        self.cfg = cfg
        self.embed = nn.Embedding(cfg.vocab_size, cfg.hidden)
        self.blocks = nn.ModuleList(
            Block(cfg, local=(i + 1) % cfg.global_every != 0) for i in range(cfg.layers)
        )
        self.norm = RMSNorm(cfg.hidden, cfg.eps)
        for name, p in self.named_parameters():
            if p.dim() >= 2:
                nn.init.normal_(p, mean=0.0, std=0.02)
        # rotary tables and the sliding-window mask of the last (length,
        # device, dtype) seen: built on the host and copied over, they cost
        # more than a third of a prefill's host time when rebuilt per call
        self._tables = {}

    def _rope_and_mask(self, t, dev, dt):
        key = (t, str(dev), dt)
        hit = self._tables.get(key)
        if hit is None:
            c = self.cfg
            hit = (rope_tables(t, c.head_dim, c.rope_local_base, dev, dt),
                   rope_tables(t, c.head_dim, c.rope_global_base, dev, dt),
                   sliding_window_causal_mask(t, c.window, dev))
            self._tables = {key: hit}
        return hit

    def forward(self, idx):
        """Logits [B, T, vocab] of one prefill over token ids idx [B, T]."""
        b, t = idx.shape
        c = self.cfg
        dev, dt = idx.device, self.embed.weight.dtype
        x = self.embed(idx) * torch.tensor(c.hidden ** 0.5, dtype=dt, device=dev)
        rope_local, rope_global, mask = self._rope_and_mask(t, dev, dt)
        for blk in self.blocks:
            x = blk(x, rope_local, rope_global, mask)
        x = self.norm(x)
        return F.linear(x, self.embed.weight)
