"""CPU oracle for LNAMD aggregation, the L2 normalisation and the super_fast pooling.
TEST INFRASTRUCTURE ONLY (imported by tests/, smoke() and bench.py's CPU leg).

* `lnamd_embed` restates the reference's original LNAMD._embed
  (models/modules/_LNAMD.py:72-129) with its PatchMaker.patchify (:16-35) and
  MeanMapper (:54-61): drop the class token, reshape to (B, C, side, side), a
  fresh nn.LayerNorm([C, side, side]) (unit weight, zero bias, eps 1e-5), then for
  r > 1 an r x r Unfold with zero padding (r-1)//2 followed by
  adaptive_avg_pool1d(C*r*r -> C) per patch.  Returns (B, P, L, C) fp32.
* `aggregate_direct` restates the accelerated path's identity
  (models/modules/_encoder_gpu.py:14-42, _aggregation_cache.py:15-58):
  F.layer_norm + F.avg_pool2d(r, stride 1, pad r//2, count_include_pad=True).
* `lnamd_bruteforce_f64` is an independent float64 loop over the definition,
  used to pin both.
* `l2_normalise` restates models/musc.py:238 (features /= ||features|| over C).
* `super_fast_pool` restates models/modules/_super_fast.py:17-27 (fp32
  adaptive_avg_pool2d 37x37 -> 28x28).
"""
from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn.functional as F


def _spatial(token: torch.Tensor) -> torch.Tensor:
    b, t, c = token.shape
    side = math.isqrt(t - 1)
    x = token[:, 1:, :].reshape(b, side, side, c)
    return x.permute(0, 3, 1, 2)


def lnamd_embed(features: list[torch.Tensor], r: int) -> torch.Tensor:
    """Original LNAMD._embed on CPU fp32 tensors: list of (B, T, C) -> (B, P, L, C)."""
    feats = [f.detach().to('cpu', torch.float32) for f in features]
    b = feats[0].shape[0]
    layers = []
    for f in feats:
        x = _spatial(f)
        x = torch.nn.LayerNorm([x.shape[1], x.shape[2], x.shape[3]])(x)
        layers.append(x)
    if r != 1:
        pad = int((r - 1) / 2)
        unfold = torch.nn.Unfold(kernel_size=r, stride=1, padding=pad, dilation=1)
        out = []
        for x in layers:
            u = unfold(x)                                        # (B, C*r*r, P)
            u = u.reshape(x.shape[0], x.shape[1], r, r, -1).permute(0, 4, 1, 2, 3)
            out.append(u)
        layers = out
    else:
        layers = [x.reshape(x.shape[0], x.shape[1], -1, 1, 1).permute(0, 2, 1, 3, 4) for x in layers]
    layers = [x.reshape(-1, *x.shape[-3:]) for x in layers]     # (B*P, C, r, r)
    pooled = []
    c = layers[0].shape[1]
    for x in layers:
        y = x.reshape(len(x), 1, -1)
        pooled.append(F.adaptive_avg_pool1d(y, c).squeeze(1))    # (B*P, C)
    stacked = torch.stack(pooled, dim=1)                          # (B*P, L, C)
    return stacked.reshape(b, -1, *stacked.shape[-2:]).detach()   # _LNAMD.py:127


def aggregate_direct(features: list[torch.Tensor], r: int, eps: float = 1e-5, device='cpu') -> torch.Tensor:
    """layer_norm + avg_pool2d(count_include_pad) identity: (B, T, C) list -> (B, P, L, C).

    Runs in fp32 on `device` (None: where the tokens live; full-size parity checks run
    it on the GPU box's device, as the reference's accelerated aggregation does)."""
    values = []
    for f in features:
        x = _spatial(f.detach().to(f.device if device is None else device, torch.float32))
        x = F.layer_norm(x, x.shape[1:], None, None, eps)
        if r != 1:
            x = F.avg_pool2d(x, r, stride=1, padding=r // 2, count_include_pad=True)
        values.append(x.flatten(2).transpose(1, 2))
    return torch.stack(values, dim=2)


def l2_normalise(features: torch.Tensor) -> torch.Tensor:
    """models/musc.py:238 -- divide by the L2 norm over the last dimension (no epsilon)."""
    return features / features.norm(dim=-1, keepdim=True)


def lnamd_bruteforce_f64(tokens: np.ndarray, r: int, eps: float = 1e-5) -> np.ndarray:
    """Float64 loops: (B, T, C) one layer -> (B, P, C) LayerNorm + zero-padded box mean."""
    tokens = np.asarray(tokens, dtype=np.float64)
    b, t, c = tokens.shape
    side = math.isqrt(t - 1)
    out = np.zeros((b, side * side, c))
    h = r // 2
    for img in range(b):
        x = tokens[img, 1:, :].reshape(side, side, c)
        mu = x.mean()
        var = ((x - mu) ** 2).mean()
        y = (x - mu) / math.sqrt(var + eps)
        for i in range(side):
            for j in range(side):
                acc = np.zeros(c)
                for di in range(-h, h + 1):
                    for dj in range(-h, h + 1):
                        ii, jj = i + di, j + dj
                        if 0 <= ii < side and 0 <= jj < side:
                            acc += y[ii, jj]
                out[img, i * side + j] = acc / (r * r)
    return out


def super_fast_pool(features: torch.Tensor, grid: int = 28) -> torch.Tensor:
    """(B, P, L, C) on a side x side grid -> (B, grid*grid, L, C), fp32 adaptive average."""
    b, p, layers, c = features.shape
    side = math.isqrt(p)
    spatial = features.permute(0, 2, 3, 1).reshape(b, layers * c, side, side)
    pooled = F.adaptive_avg_pool2d(spatial.float(), (grid, grid)).to(features.dtype)
    return pooled.reshape(b, layers, c, grid * grid).permute(0, 3, 1, 2).contiguous()


def adaptive_pool_bruteforce_f64(x: np.ndarray, out: int) -> np.ndarray:
    """(H, W) -> (out, out): cell (i, j) averages rows floor(i*H/out)..ceil((i+1)*H/out)-1."""
    x = np.asarray(x, dtype=np.float64)
    hgt, wid = x.shape
    res = np.empty((out, out))
    for i in range(out):
        r0, r1 = (i * hgt) // out, -(-((i + 1) * hgt) // out)
        for j in range(out):
            c0, c1 = (j * wid) // out, -(-((j + 1) * wid) // out)
            res[i, j] = x[r0:r1, c0:c1].mean()
    return res
