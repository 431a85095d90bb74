"""Epilogue parity on the GPU (float64; the reference computes it in float64 too)."""
import numpy as np
import pytest
import torch

from oracle import epilogue as oe
from musc_hip import _epilogue_hip

pytestmark = pytest.mark.gpu


def test_golden_bilinear(golden, device):
    g = golden('bilinear_small.npz')
    scores = torch.from_numpy(g['grid'].reshape(1, 1, 1, 25)).to(device)
    for size, key in ((13, 'up13'), (37, 'up37')):
        maps, img = _epilogue_hip.maps_and_scores(scores, size)
        np.testing.assert_allclose(maps[0, 0].cpu().numpy(), g[key], rtol=0, atol=1e-13)
        assert img[0].item() == pytest.approx(g[key].max(), abs=1e-13)


def test_full_size_vs_oracle(device):
    rng = np.random.default_rng(0)
    raw = rng.random((3, 4, 5, 1369))
    maps, img = _epilogue_hip.maps_and_scores(torch.from_numpy(raw).to(device), 518)
    ref_maps, ref_img = oe.maps_and_scores([[torch.from_numpy(raw[r, l]) for l in range(4)] for r in range(3)], 518)
    assert maps.shape == (5, 1, 518, 518)
    np.testing.assert_allclose(maps.cpu().numpy(), ref_maps.numpy(), rtol=0, atol=1e-12)
    np.testing.assert_allclose(img.cpu().numpy(), ref_img.numpy(), rtol=0, atol=1e-12)
    _, img_only = _epilogue_hip.maps_and_scores(torch.from_numpy(raw).to(device), 518, want_maps=False)
    assert torch.equal(img_only.cpu(), img.cpu())


@pytest.mark.parametrize('p,size', [(1, 7), (4, 1), (784, 518), (9, 2), (1369, 37)])
def test_degenerate_and_other_sizes(device, p, size):
    # one-patch grids (every pixel = the score), a 1x1 output (torch's align_corners maps it to
    # grid[0, 0]), the super_fast 28x28 grid, identity size: against the float64 brute force
    rng = np.random.default_rng(p * 10 + size)
    raw = rng.random((2, 3, 4, p))
    maps, img = _epilogue_hip.maps_and_scores(torch.from_numpy(raw).to(device), size)
    ref_maps, ref_img = oe.maps_and_scores([[torch.from_numpy(raw[r, l]) for l in range(3)] for r in range(2)], size)
    np.testing.assert_allclose(maps.cpu().numpy(), ref_maps.numpy(), rtol=0, atol=1e-12)
    np.testing.assert_allclose(img.cpu().numpy(), ref_img.numpy(), rtol=0, atol=1e-12)
    side = int(round(p ** 0.5))
    mean = raw.mean(axis=(0, 1)).reshape(4, side, side)
    brute = np.stack([oe.bilinear_align_corners_f64(m, size) for m in mean])
    np.testing.assert_allclose(maps[:, 0].cpu().numpy(), brute, rtol=0, atol=1e-12)
