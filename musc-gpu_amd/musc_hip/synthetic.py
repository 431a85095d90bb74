"""Seeded synthetic feature pools for the benchmark configurations.

Generated on the CPU with torch.Generator so that the GPU path and the CPU
oracle see bit-identical inputs; the caller moves them to the device.

  plumbing_tokens(n)      config 1: (n, 1370, 1024) iid N(0,1), each token L2-normalised
  pool_tokens(n, layers)  config 2: per layer l, normalise(G_l + mu_l) with G_l iid
                          N(0,1) (n, 1370, 1024) and one shared mu_l ~ N(0,1)^1024
                          (offset scale 1.0), seed = seed + l
  msm_features(n, p, c)   kernel-only pools: (n, p, c) iid N(0,1), L2-normalised rows
  attention_blocks(...)   config 4: per block, tokens y ~ N(0,1) (B*T, 1024) projected by
                          W ~ N(0, 0.02^2) (1024, 3*1024) into (B*H, T, 64) q, k, v
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


def attention_blocks(blocks: int = 24, b: int = 4, heads: int = 16, tokens: int = 1370, d: int = 64,
                     seed: int = 42, device: torch.device | str = 'cpu'):
    """Config 4: yields one (q, k, v) triple of fp32 (b*heads, tokens, d) tensors per block.
    y and W are drawn on the CPU; the projection y @ W runs on `device`."""
    g = torch.Generator().manual_seed(seed)
    width = heads * d
    for _ in range(blocks):
        y = torch.randn((b * tokens, width), generator=g).to(device)
        w = (torch.randn((width, 3 * width), generator=g) * 0.02).to(device)
        qkv = (y @ w).reshape(b, tokens, 3, heads, d).permute(2, 0, 3, 1, 4).reshape(3, b * heads, tokens, d)
        yield tuple(x.contiguous() for x in qkv)


# CLIP image normalisation constants (OpenAI CLIP preprocessing)
CLIP_MEAN = (0.48145466, 0.4578275, 0.40821073)
CLIP_STD = (0.26862954, 0.26130258, 0.27577711)


def images(n: int = 160, size: int = 518, seed: int = 42, anomaly_fraction: float = 0.05) -> tuple[torch.Tensor, list]:
    """Config 5: n uniform[0,1] RGB images; round(n * anomaly_fraction) of them carry one
    random rectangle shifted in intensity.  Returns (CLIP-normalised (n, 3, size, size)
    fp32, indices of the anomalous images)."""
    g = torch.Generator().manual_seed(seed)
    x = torch.rand((n, 3, size, size), generator=g)
    k = int(round(n * anomaly_fraction))
    idx = torch.randperm(n, generator=g)[:k].tolist()
    for i in idx:
        h, w = (int(v) for v in torch.randint(size // 16, size // 4, (2,), generator=g))
        y0, x0 = (int(v) for v in torch.randint(0, size - max(h, w), (2,), generator=g))
        shift = float(torch.rand((), generator=g)) * 0.6 + 0.2
        x[i, :, y0:y0 + h, x0:x0 + w] = (x[i, :, y0:y0 + h, x0:x0 + w] + shift).clamp(0, 1)
    mean = torch.tensor(CLIP_MEAN).view(1, 3, 1, 1)
    std = torch.tensor(CLIP_STD).view(1, 3, 1, 1)
    return (x - mean) / std, sorted(idx)
