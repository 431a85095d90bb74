"""LNAMD with the adaptive pooling fused into the same pass (musc_lnamd_pooled_f32) vs
the oracle's LNAMD -> adaptive_avg_pool2d chain (models/modules/_LNAMD.py:72-129,
models/modules/_super_fast.py:17-27) and vs the two-kernel GPU path."""
from types import SimpleNamespace

import pytest
import torch
import torch.nn.functional as F

from oracle import lnamd as ol
from musc_hip import _lnamd_hip, _super_fast

pytestmark = pytest.mark.gpu


def _tokens(n, side, c, layers, seed, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    return [(torch.randn((n, 1 + side * side, c), generator=g) * 2 + torch.randn((c,), generator=g)).to(dtype)
            for _ in range(layers)]


def _pool_ref(feats, side, pool):
    # (B, P, L, C) -> adaptive_avg_pool2d on each (L*C) plane -> (B, pool^2, L, C), float64
    b, p, l, c = feats.shape
    x = feats.double().permute(0, 2, 3, 1).reshape(b, l * c, side, side)
    y = F.adaptive_avg_pool2d(x, (pool, pool))
    return y.reshape(b, l, c, pool * pool).permute(0, 3, 1, 2)


def test_super_fast_shape_vs_oracle(device):
    # config 3's aggregation: r = 3 on 37 x 37, pooled to 28 x 28
    toks = _tokens(3, 37, 64, 1, 21)
    got = _lnamd_hip.lnamd([t.to(device) for t in toks], [3], layout='rbplc', pool_side=28)[0].cpu()
    ref = ol.super_fast_pool(ol.lnamd_embed(toks, 3))
    assert got.shape == (3, 784, 1, 64)
    torch.testing.assert_close(got.double(), ref.double(), rtol=0, atol=2e-6)


@pytest.mark.parametrize('side,pool', [(37, 28), (37, 10), (13, 5), (9, 9), (12, 1), (16, 8)])
@pytest.mark.parametrize('layout', ['rbplc', 'rlbpc'])
def test_pool_sizes_radii_layers(device, side, pool, layout):
    toks = _tokens(2, side, 32, 2, side * 100 + pool)
    dev = [t.to(device) for t in toks]
    full = _lnamd_hip.lnamd(dev, [5, 1, 3], layout='rbplc').cpu()           # (R, B, P, L, C)
    got = _lnamd_hip.lnamd(dev, [5, 1, 3], layout=layout, pool_side=pool).cpu()
    for ri in range(3):
        ref = _pool_ref(full[ri], side, pool)                                # (B, pool^2, L, C)
        g = got[ri] if layout == 'rbplc' else got[ri].permute(1, 2, 0, 3)   # (L, B, P, C) -> (B, P, L, C)
        torch.testing.assert_close(g.double(), ref, rtol=1e-5, atol=1e-6)


def test_raw_sums_pooled_rows_are_scaled_features(device):
    # raw pooled sums = per-row positive multiples of the exact pooled features
    toks = _tokens(2, 37, 48, 1, 31)
    dev = [t.to(device) for t in toks]
    raw = _lnamd_hip.lnamd(dev, [3], layout='rlbpc', raw_sums=True, pool_side=28)[0, 0].cpu().double()
    ref = ol.super_fast_pool(ol.lnamd_embed(toks, 3))[:, :, 0].double()      # (B, 784, C)
    cos = (raw * ref).sum(-1) / (raw.norm(dim=-1) * ref.norm(dim=-1))
    assert (cos > 1 - 1e-9).all()


def test_fp16_tokens(device):
    toks = _tokens(2, 37, 64, 1, 41, dtype=torch.float16)
    got = _lnamd_hip.lnamd([t.to(device) for t in toks], [3], pool_side=28)[0].cpu()
    ref = ol.super_fast_pool(ol.lnamd_embed([t.float() for t in toks], 3))
    torch.testing.assert_close(got.double(), ref.double(), rtol=0, atol=2e-6)


def test_rejections(device):
    toks = [t.to(device) for t in _tokens(1, 9, 16, 1, 51)]
    with pytest.raises(ValueError):
        _lnamd_hip.lnamd(toks, [3], pool_side=10)
    with pytest.raises(ValueError):
        _lnamd_hip.lnamd(toks, [3], pool_side=0)
    with pytest.raises(ValueError):
        _lnamd_hip.lnamd(toks, [3], pool_side=5, l2norm=True)


def test_super_fast_plugin_fused_equals_two_pass(device):
    toks = [t.to(device) for t in _tokens(2, 37, 64, 1, 61)]
    layer = _lnamd_hip.LNAMD(device=device, feature_dim=64, feature_layer=[5], r=3)
    fused = _super_fast.new_aggregation()(layer, toks, return_cpu=False)
    unpooled = _lnamd_hip.lnamd(toks, [3], layout='rbplc')[0]
    two_pass = _super_fast.adaptive_pool(unpooled, 28)
    assert fused.shape == (2, 784, 1, 64)
    torch.testing.assert_close(fused, two_pass, rtol=1e-5, atol=1e-6)
    with pytest.raises(ValueError, match='super_fast requires'):
        _super_fast.new_aggregation()(_lnamd_hip.LNAMD(device=device, feature_dim=64, feature_layer=[5], r=1),
                                      toks, return_cpu=False)
