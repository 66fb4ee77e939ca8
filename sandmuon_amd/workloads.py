"""Synthetic workloads for the benchmark and the parity tests.

The reference ships no model code (its GPT trainer is not archived), so the
GPT-2-style model below is a benchmark harness with the parameter names the
reference's q/k/v sharing rule and module_filter expect
(transformer.h.N.attn.{q,k,v}_proj, .c_proj, mlp.c_fc, mlp.c_proj; names per
paper/data/centered_screen/arms/baseline/manifest.json:76-79).  At the
103M configuration it has 103,176,192 parameters, 63,700,992 of them in the
54 selected matrices.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np
import torch
from torch import nn
from torch.nn import functional as F


@dataclass(frozen=True)
class GPTConfig:
    vocab: int = 50257
    ctx: int = 1024
    layers: int = 9
    width: int = 768
    heads: int = 12
    mlp: int = 3072


GPT_103M = GPTConfig()
GPT_2048 = GPTConfig(layers=24, width=2048, heads=16, mlp=8192)
GPT_TINY = GPTConfig(vocab=97, ctx=16, layers=2, width=32, heads=2, mlp=128)


class Attention(nn.Module):
    def __init__(self, cfg: GPTConfig):
        super().__init__()
        self.heads = cfg.heads
        self.q_proj = nn.Linear(cfg.width, cfg.width)
        self.k_proj = nn.Linear(cfg.width, cfg.width)
        self.v_proj = nn.Linear(cfg.width, cfg.width)
        self.c_proj = nn.Linear(cfg.width, cfg.width)

    def forward(self, x):
        b, t, c = x.shape
        h = self.heads
        q = self.q_proj(x).view(b, t, h, c // h).transpose(1, 2)
        k = self.k_proj(x).view(b, t, h, c // h).transpose(1, 2)
        v = self.v_proj(x).view(b, t, h, c // h).transpose(1, 2)
        y = F.scaled_dot_product_attention(q, k, v, is_causal=True)
        return self.c_proj(y.transpose(1, 2).reshape(b, t, c))


class MLP(nn.Module):
    def __init__(self, cfg: GPTConfig):
        super().__init__()
        self.c_fc = nn.Linear(cfg.width, cfg.mlp)
        self.c_proj = nn.Linear(cfg.mlp, cfg.width)

    def forward(self, x):
        return self.c_proj(F.gelu(self.c_fc(x)))


class Block(nn.Module):
    def __init__(self, cfg: GPTConfig):
        super().__init__()
        self.ln_1 = nn.LayerNorm(cfg.width)
        self.attn = Attention(cfg)
        self.ln_2 = nn.LayerNorm(cfg.width)
        self.mlp = MLP(cfg)

    def forward(self, x):
        x = x + self.attn(self.ln_1(x))
        return x + self.mlp(self.ln_2(x))


class GPT(nn.Module):
    def __init__(self, cfg: GPTConfig):
        super().__init__()
        self.cfg = cfg
        self.transformer = nn.ModuleDict(dict(
            wte=nn.Embedding(cfg.vocab, cfg.width),
            wpe=nn.Embedding(cfg.ctx, cfg.width),
            h=nn.ModuleList([Block(cfg) for _ in range(cfg.layers)]),
            ln_f=nn.LayerNorm(cfg.width),
        ))

    def init_weights(self, seed: int) -> None:
        g = torch.Generator().manual_seed(seed)
        with torch.no_grad():
            for name, p in self.named_parameters():
                if p.ndim == 2:
                    std = 0.02 / math.sqrt(2 * self.cfg.layers) if name.endswith("c_proj.weight") else 0.02
                    p.copy_(torch.randn(p.shape, generator=g) * std)
                elif name.endswith(".bias"):
                    p.zero_()
                else:
                    p.fill_(1.0)

    def forward(self, idx, targets=None):
        b, t = idx.shape
        pos = torch.arange(t, device=idx.device)
        x = self.transformer.wte(idx) + self.transformer.wpe(pos)
        for block in self.transformer.h:
            x = block(x)
        x = self.transformer.ln_f(x)
        logits = x @ self.transformer.wte.weight.t()
        if targets is None:
            return logits
        return F.cross_entropy(logits.float().view(-1, logits.shape[-1]), targets.view(-1))


def transformer_filter(name: str, module: nn.Module) -> bool:
    """Historical selection: every nn.Linear under transformer.h (README.md:43-47)."""
    return name.startswith("transformer.h.") and isinstance(module, nn.Linear)


# ------------------------------------------------------------ inputs ---
def rng(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(seed))


def s8_cfg2_batch(seed: int, batch: int, rows: int, cols: int) -> torch.Tensor:
    """cfg2 inputs: N(0,1) with diagonal row/column scales log-uniform in [1e-2, 1e2]."""
    r = rng(seed)
    x = r.standard_normal((batch, rows, cols))
    dr = np.exp(r.uniform(math.log(1e-2), math.log(1e2), (batch, rows, 1)))
    dc = np.exp(r.uniform(math.log(1e-2), math.log(1e2), (batch, 1, cols)))
    return torch.from_numpy((x * dr * dc).astype(np.float32))


def stats_cfg3_tensor(seed: int, rows: int, cols: int, dtype=torch.bfloat16, device="cpu") -> torch.Tensor:
    """cfg3 activations: x ~ N(mu_c, sigma_c), mu_c ~ N(0, .3), sigma_c log-uniform [.1, 10]."""
    r = rng(seed)
    mu = r.normal(0.0, 0.3, cols)
    sigma = np.exp(r.uniform(math.log(0.1), math.log(10.0), cols))
    g = torch.Generator(device="cpu").manual_seed(seed)
    x = torch.randn(rows, cols, generator=g) * torch.from_numpy(sigma).float() + torch.from_numpy(mu).float()
    return x.to(dtype).to(device)
