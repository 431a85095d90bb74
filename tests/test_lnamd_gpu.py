"""LNAMD parity on the GPU: libmusc_hip vs the oracle restatements."""
import numpy as np
import pytest
import torch

from oracle import lnamd as ol
from musc_hip import _lnamd_hip
from musc_hip._aggregation_cache import RadiusAggregationCache

pytestmark = pytest.mark.gpu
ATOL = 2e-5


@pytest.mark.parametrize('r', [1, 3, 5])
def test_golden_plugin(golden, device, r):
    g = golden('lnamd_small.npz')
    toks = torch.from_numpy(g['tokens']).to(device)
    layer = _lnamd_hip.LNAMD(feature_dim=8, feature_layer=[1], r=r)
    out = _lnamd_hip.aggregate_features(layer, [toks], return_cpu=True)
    assert out.shape == (2, 25, 1, 8) and out.dtype == torch.float32
    np.testing.assert_allclose(out[:, :, 0].numpy(), g[f'r{r}'], rtol=0, atol=ATOL)
    ref = ol.lnamd_embed([toks.cpu()], r)
    np.testing.assert_allclose(out.numpy(), ref.numpy(), rtol=0, atol=ATOL)


@pytest.mark.parametrize('c', [1024, 768, 36])
def test_multi_radius_layouts(device, c):
    g = torch.Generator().manual_seed(c)
    feats = [torch.randn((3, 1370, c), generator=g) + torch.randn((c,), generator=g) for _ in range(2)]
    dev = [f.to(device) for f in feats]
    rb = _lnamd_hip.lnamd(dev, [1, 3, 5], layout='rbplc').cpu()
    rl = _lnamd_hip.lnamd(dev, [1, 3, 5], layout='rlbpc').cpu()
    assert rb.shape == (3, 3, 1369, 2, c) and rl.shape == (3, 2, 3, 1369, c)
    assert torch.equal(rb.permute(0, 3, 1, 2, 4), rl)
    for k, r in enumerate((1, 3, 5)):
        ref = ol.aggregate_direct(feats, r)
        err = (rb[k] - ref).abs().max().item()
        assert err <= ATOL, f'r={r}: {err}'
        ref_u = ol.lnamd_embed(feats, r)
        assert (rb[k] - ref_u).abs().max().item() <= ATOL


@pytest.mark.parametrize('side,c', [(20, 64), (7, 100), (1, 8)])
def test_wide_radii_in_any_order(device, side, c):
    # the library takes up to four odd radii up to 9 in any order (the output keeps the
    # caller's order), and any square grid: small grids where the window exceeds the grid
    g = torch.Generator().manual_seed(side * 1000 + c)
    feats = [torch.randn((2, side * side + 1, c), generator=g) * 2 + 0.5 for _ in range(3)]
    radii = [9, 1, 7, 3]
    dev = [f.to(device) for f in feats]
    out = _lnamd_hip.lnamd(dev, radii, layout='rbplc').cpu()
    assert out.shape == (4, 2, side * side, 3, c)
    normed = _lnamd_hip.lnamd(dev, radii, layout='rbplc', l2norm=True).cpu()
    for k, r in enumerate(radii):
        ref = ol.aggregate_direct(feats, r)
        err = (out[k] - ref).abs().max().item()
        assert err <= ATOL, f'r={r}: {err}'
        err = (normed[k] - ol.l2_normalise(ref)).abs().max().item()
        assert err <= ATOL, f'r={r} (L2): {err}'


def test_fused_l2norm(device):
    g = torch.Generator().manual_seed(5)
    feats = [torch.randn((4, 1370, 1024), generator=g) for _ in range(3)]
    out = _lnamd_hip.lnamd([f.to(device) for f in feats], [1, 3, 5], l2norm=True, layout='rlbpc').cpu()
    for k, r in enumerate((1, 3, 5)):
        ref = ol.l2_normalise(ol.aggregate_direct(feats, r))        # (B, P, L, C)
        for l in range(3):
            err = (out[k, l] - ref[:, :, l]).abs().max().item()
            assert err <= ATOL, f'r={r} l={l}: {err}'


def test_fp16_tokens(device):
    g = torch.Generator().manual_seed(6)
    feats = [torch.randn((2, 1370, 1024), generator=g).half() for _ in range(2)]
    out = _lnamd_hip.lnamd([f.to(device) for f in feats], [3]).cpu()[0]
    ref = ol.aggregate_direct([f.float() for f in feats], 3)
    assert (out - ref).abs().max().item() <= ATOL


def test_radius_cache_reuses_statistics(device):
    g = torch.Generator().manual_seed(7)
    feats = [torch.randn((2, 1370, 64), generator=g).to(device) for _ in range(2)]
    cache = RadiusAggregationCache()
    for r in (1, 3, 5):
        layer = _lnamd_hip.LNAMD(feature_dim=64, feature_layer=[1, 2], r=r)
        got = cache(layer, feats, return_cpu=False)
        plain = _lnamd_hip.aggregate_features(layer, feats, return_cpu=False)
        assert torch.equal(got, plain)
    assert len(cache._stats) == 1
    cache.clear()
    assert len(cache._stats) == 0


def test_constant_image_gives_zero(device):
    toks = torch.full((1, 26, 8), 2.5, device=device)
    out = _lnamd_hip.lnamd([toks], [1, 3, 5])
    assert out.abs().max().item() == 0.0


def test_raw_sums_normalise_to_the_reference_features(device):
    # window sums of (x - mean): scaling by rstd / r^2 gives the plugin output, and
    # L2-normalising gives the features of models/musc.py:238
    g = torch.Generator().manual_seed(9)
    feats = [torch.randn((3, 1370, 1024), generator=g) + 0.5 for _ in range(2)]
    dev = [f.to(device) for f in feats]
    raw = _lnamd_hip.lnamd(dev, [5, 1, 3], raw_sums=True, layout='rlbpc').cpu()
    for k, r in enumerate((5, 1, 3)):
        ref = ol.l2_normalise(ol.aggregate_direct(feats, r))
        for l in range(2):
            got = raw[k, l] / raw[k, l].norm(dim=-1, keepdim=True)
            assert (got - ref[:, :, l]).abs().max().item() <= ATOL
