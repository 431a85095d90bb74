"""Epilogue and RsCIN over seeded random shapes, against the oracle.

Epilogue (models/musc.py:259-288): 20 draws of radii (1-4), layers (1-5), images (1-9),
score grids of side 1-40 and output sizes 1-600 (upsampling and downsampling), against the
float64 torch restatement (mean over layers, mean over radii, bilinear align_corners,
image maximum) at 1e-12, and six strong downsamplings (grids of 37-128 to 2-17 pixels).  RsCIN (models/modules/_RsCIN.py:5-32): 20 draws of pool sizes
2-200, class-token widths 4-1024 and k lists (k up to the pool size), against the float64
definition on every row (oracle.rscin.check_rscin, 2e-5).
"""
import numpy as np
import pytest
import torch

from musc_hip import _epilogue_hip
from musc_hip._RsCIN_hip import RsCIN
from oracle import epilogue as oe
from oracle import rscin as orc

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize('k', range(20))
def test_random_epilogue(device, k):
    rng = np.random.default_rng(900 + k)
    r, l, n = int(rng.integers(1, 5)), int(rng.integers(1, 6)), int(rng.integers(1, 10))
    side = int(rng.choice([1, 2, 5, 7, 28, 37, 40]))
    size = int(rng.choice([1, 2, side, 64, 224, 518, 600]))
    scores = torch.from_numpy(rng.random((r, l, n, side * side)) * 2.0)
    maps, img = _epilogue_hip.maps_and_scores(scores.to(device), size)
    ref_maps, ref_img = oe.maps_and_scores([[scores[i, j] for j in range(l)] for i in range(r)], size)
    assert maps.shape == (n, 1, size, size) and img.shape == (n,)
    em = (maps.cpu() - ref_maps).abs().max().item()
    ei = (img.cpu() - ref_img).abs().max().item()
    print(f'epilogue {k}: r={r} l={l} n={n} side={side} size={size}: maps {em:.1e}, scores {ei:.1e}', flush=True)
    assert em <= 1e-12 and ei <= 1e-12


@pytest.mark.parametrize('k', range(20))
def test_random_rscin(device, k):
    rng = np.random.default_rng(1900 + k)
    n = int(rng.choice([2, 3, 7, 20, 83, 160, 200]))
    d = int(rng.choice([4, 16, 64, 768, 1024]))
    ks = sorted({int(x) for x in rng.integers(1, n + 1, size=int(rng.integers(1, 4)))})
    cls = rng.standard_normal((n, d)).astype(np.float32)
    cls /= np.linalg.norm(cls, axis=1, keepdims=True)
    raw = rng.random(n) * 2.0 + 0.5
    got = RsCIN(torch.from_numpy(raw).to(device), torch.from_numpy(cls).to(device), ks).cpu().numpy()
    ok, info = orc.check_rscin(got.astype(np.float64), raw, cls, ks, atol=2e-5)
    print(f'rscin {k}: n={n} d={d} k={ks}: {info}', flush=True)
    assert ok, info


@pytest.mark.parametrize('side,size', [(128, 3), (100, 7), (40, 5), (37, 2), (64, 9), (128, 17)])
def test_strong_downsampling(device, side, size):
    # scale (side - 1) / (size - 1) large: a band of output rows would span more grid rows
    # than the kernel stages, so it takes fewer rows per band (down to one)
    rng = np.random.default_rng(side * 100 + size)
    scores = torch.from_numpy(rng.random((2, 3, 2, side * side)))
    maps, img = _epilogue_hip.maps_and_scores(scores.to(device), size)
    ref_maps, ref_img = oe.maps_and_scores([[scores[i, j] for j in range(3)] for i in range(2)], size)
    assert (maps.cpu() - ref_maps).abs().max().item() <= 1e-12
    assert (img.cpu() - ref_img).abs().max().item() <= 1e-12
