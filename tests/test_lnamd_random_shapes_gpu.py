"""LNAMD over seeded random shapes and options, against the oracle's restatement.

The fixed cases of test_lnamd_gpu.py and test_lnamd_pooled_gpu.py pin each option; this
sweep draws 30 combinations: 1-4 images, grid sides 1-40, 4-1024 channels (C % 4 == 0,
the kernel's contract), 1-5 layers, up to four odd radii up to 9 in any order, fp32 or
fp16 tokens, with or without the class token, both output layouts, the fused L2
normalisation, the raw window sums and the fused adaptive pooling to a smaller grid.
Every output is checked against the oracle's layer_norm + avg_pool2d(count_include_pad)
restatement (models/modules/_encoder_gpu.py:14-42; the identity with the original
LNAMD._embed is pinned in test_oracle.py) at the reference's 2e-5 gate
(tools/benchmark_support.py:11), pooled outputs against adaptive_avg_pool2d of it
(models/modules/_super_fast.py:17-27), raw sums after both sides are L2-normalised
(each raw row is its feature row times a positive constant).
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from musc_hip import _lnamd_hip
from oracle import lnamd as ol

pytestmark = pytest.mark.gpu
ATOL = 2e-5


def _case(k):
    rng = np.random.default_rng(500 + k)
    b = int(rng.integers(1, 5))
    side = int(rng.choice([1, 2, 3, 5, 8, 13, 20, 28, 37, 40]))
    c = int(rng.choice([4, 8, 36, 64, 100, 256, 768, 1024]))
    layers = int(rng.integers(1, 6))
    radii = [int(r) for r in rng.choice([1, 3, 5, 7, 9], size=int(rng.integers(1, 5)), replace=False)]
    fp16 = bool(rng.integers(0, 2))
    has_cls = bool(rng.integers(0, 4))          # mostly with the class token, as the encoder gives
    layout = str(rng.choice(['rbplc', 'rlbpc']))
    mode = str(rng.choice(['plain', 'l2norm', 'raw', 'pool', 'pool_raw']))
    pool = int(rng.integers(1, side + 1)) if mode.startswith('pool') else None
    return b, side, c, layers, radii, fp16, has_cls, layout, mode, pool


def _row_unit(x):
    return x / x.norm(dim=-1, keepdim=True).clamp_min(1e-30)


@pytest.mark.parametrize('k', range(30))
def test_random_lnamd_against_oracle(device, k):
    b, side, c, layers, radii, fp16, has_cls, layout, mode, pool = _case(k)
    g = torch.Generator().manual_seed(k)
    feats = [torch.randn((b, side * side + 1, c), generator=g) * 1.5 + torch.randn((c,), generator=g)
             for _ in range(layers)]
    if fp16:
        feats = [f.half().float() for f in feats]
    dt = torch.float16 if fp16 else torch.float32
    dev = [(f if has_cls else f[:, 1:]).to(dt).to(device) for f in feats]
    out = _lnamd_hip.lnamd(dev, radii, layout=layout, has_cls=has_cls, l2norm=(mode == 'l2norm'),
                           raw_sums=mode in ('raw', 'pool_raw'), pool_side=pool).cpu()
    p = side * side if pool is None else pool * pool
    expect = (len(radii), b, p, layers, c) if layout == 'rbplc' else (len(radii), layers, b, p, c)
    assert out.shape == expect
    worst = 0.0
    for ri, r in enumerate(radii):
        ref = ol.aggregate_direct(feats, r)                                     # (B, side^2, L, C)
        if pool is not None:
            grid = ref.permute(0, 2, 3, 1).reshape(b * layers, c, side, side)
            grid = F.adaptive_avg_pool2d(grid, pool)
            ref = grid.reshape(b, layers, c, pool * pool).permute(0, 3, 1, 2)
        got = out[ri] if layout == 'rbplc' else out[ri].permute(1, 2, 0, 3)
        if mode == 'l2norm':
            ref = ol.l2_normalise(ref)
        if mode in ('raw', 'pool_raw'):
            ref, got = _row_unit(ref), _row_unit(got)
        err = (got - ref).abs().max().item()
        worst = max(worst, err)
        assert math.isfinite(err) and err <= ATOL, (r, err)
    print(f'case {k}: b={b} side={side} c={c} layers={layers} radii={radii} fp16={fp16} cls={has_cls} '
          f'{layout} {mode} pool={pool}: {worst:.2e}', flush=True)
