"""super_fast aggregation: layer 5, r=3, patch grid pooled 37x37 -> 28x28.

Mirrors models/modules/_super_fast.py:7-40: `SuperFastAggregation` wraps the
per-division aggregation, checks its one-layer/r=3/37x37 contract (ValueError
otherwise) and adaptively average-pools the grid to PATCH_GRID x PATCH_GRID in
fp32, returning the features' dtype.  With this package's own aggregation and
tokens the LNAMD kernel supports, LNAMD and the pooling are one pass
(musc_lnamd_pooled_f32); otherwise the wrapped aggregation runs and its output is
pooled by musc_adaptive_pool_f32.
"""
from __future__ import annotations

import math

import torch

from . import _lnamd_hip
from . import _runtime as rt
from ._aggregation_cache import RadiusAggregationCache

PATCH_GRID = 28


def adaptive_pool(features: torch.Tensor, grid: int = PATCH_GRID) -> torch.Tensor:
    """(B, P, ...) features on a side x side grid -> (B, grid*grid, ...) fp32 adaptive averages."""
    rt.require_device_tensor(features, 'features')
    b, p = features.shape[:2]
    side = math.isqrt(p)
    if side * side != p:
        raise ValueError('patch count must be a square grid')
    rest = features.shape[2:]
    ch = 1
    for d in rest:
        ch *= d
    x = features.float().contiguous()
    with torch.cuda.device(x.device):
        out = torch.empty((b, grid * grid) + tuple(rest), dtype=torch.float32, device=x.device)
        rc = rt.library().musc_adaptive_pool_f32(x.data_ptr(), b, side, ch, grid, out.data_ptr(), rt.stream(x.device))
        rt.check(rc, 'musc_adaptive_pool_f32')
    return out


class SuperFastAggregation:
    def __init__(self):
        self.base = RadiusAggregationCache()

    def clear(self):
        self.base.clear()

    def __call__(self, layer, tokens, return_cpu=True):
        if isinstance(self.base, RadiusAggregationCache) and tokens and _lnamd_hip.supported(layer, tokens):
            side = math.isqrt(tokens[0].shape[1] - 1)
            if side != 37 or len(tokens) != 1 or layer.r != 3:
                raise ValueError('super_fast requires one layer, r=3 and a 37x37 source patch grid')
            pooled = _lnamd_hip.lnamd(tokens, [3], layout='rbplc', pool_side=PATCH_GRID)[0]
            return pooled.cpu() if return_cpu else pooled
        features = self.base(layer, tokens, return_cpu=False)
        b, p, layers, c = features.shape
        side = math.isqrt(p)
        if side != 37 or side * side != p or layers != 1 or layer.r != 3:
            raise ValueError('super_fast requires one layer, r=3 and a 37x37 source patch grid')
        pooled = adaptive_pool(features, PATCH_GRID).to(features.dtype)
        return pooled.cpu() if return_cpu else pooled


def new_aggregation():
    return SuperFastAggregation()
