"""Seeded synthetic feature pools for the benchmark configurations.

Generated on the CPU with torch.Generator so that the GPU path and the CPU
oracle see bit-identical inputs; the caller moves them to the device.

  plumbing_tokens(n)      config 1: (n, 1370, 1024) iid N(0,1), each token L2-normalised
  pool_tokens(n, layers)  config 2: per layer l, normalise(G_l + mu_l) with G_l iid
                          N(0,1) (n, 1370, 1024) and one shared mu_l ~ N(0,1)^1024
                          (offset scale 1.0), seed = seed + l
  msm_features(n, p, c)   kernel-only pools: (n, p, c) iid N(0,1), L2-normalised rows
"""
from __future__ import annotations

import torch


def _normalise(x: torch.Tensor) -> torch.Tensor:
    return x / x.norm(dim=-1, keepdim=True)


def plumbing_tokens(n: int = 8, tokens: int = 1370, c: int = 1024, seed: int = 42) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    return _normalise(torch.randn((n, tokens, c), generator=g, dtype=torch.float32))


def pool_tokens(n: int = 83, layers: int = 4, tokens: int = 1370, c: int = 1024, seed: int = 42,
                offset_scale: float = 1.0) -> list[torch.Tensor]:
    out = []
    for l in range(layers):
        g = torch.Generator().manual_seed(seed + l)
        mu = torch.randn((c,), generator=g, dtype=torch.float32) * offset_scale
        x = torch.randn((n, tokens, c), generator=g, dtype=torch.float32)
        x += mu
        out.append(_normalise(x))
    return out


def msm_features(n: int, p: int, c: int, seed: int = 42) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    return _normalise(torch.randn((n, p, c), generator=g, dtype=torch.float32))
