"""MSM where the expanded form cancels: duplicated images and near-duplicate patches.

||a||^2 + ||b||^2 - 2 a.b carries a rounding error of the order of eps (||a||^2 +
||b||^2) whatever the distance, so a minimum near 0 keeps only its square root (a few
1e-4 in d for unit rows).  The reference's accelerated MSM recomputes such pairs by
explicit differences (models/modules/_MSM_gpu.py:23-33, 219-228), and so does this
build's refinement stage (musc_msm_refine_f32) for both engines.  The oracle here is
the C float64 brute force over explicit differences (oracle/msm_f64.c), not torch.cdist,
whose matmul path cancels the same way.  Gate: 2e-5 absolute
(tools/benchmark_support.py:11).
"""
import numpy as np
import pytest
import torch

import oracle
from musc_hip import _MSM_hip
from oracle import msm as om

pytestmark = pytest.mark.gpu
ATOL = 2e-5
# planted distances: exact duplicates up to past the refinement bound (d^2 <= max(32 C,
# 4096) eps (||q||^2 + ||r||^2) = 7.8e-3 for unit rows at C = 1024, i.e. d <= 0.088)
DELTAS = (0.0, 1e-7, 1e-6, 1e-5, 1e-4, 1e-3, 3e-3, 1e-2, 3e-2, 0.08, 0.1, 0.2)


def _unit(x):
    return x / np.linalg.norm(x, axis=-1, keepdims=True)


def near_duplicate_pool(n=12, p=300, c=1024, seed=3):
    """Random unit rows; images 3 and 7 duplicate images 0 and 1; in images 5 and 9, patches
    sit at the planted distances from patches of images 2 and 4."""
    rng = np.random.default_rng(seed)
    z = _unit(rng.standard_normal((n, p, c)))
    z[3] = z[0]
    z[7] = z[1]
    planted = []
    for k, d in enumerate(DELTAS):
        for (i, qi), (j, qj) in (((5, 10 + k), (2, 20 + k)), ((9, 100 + 3 * k), (4, 50 + k))):
            u = rng.standard_normal(c)
            u = _unit(u - (u @ z[j, qj]) * z[j, qj])
            z[i, qi] = _unit(z[j, qj] + d * u)     # a unit row about d from z[j, qj]
            planted.append((i, qi, j, qj, d))
    return z.astype(np.float32), planted


@pytest.fixture(scope='module')
def pool():
    return near_duplicate_pool()


@pytest.mark.parametrize('engine', ['fp32', 'split16'])
@pytest.mark.parametrize('scale,normalize', [(1.0, False), (3.7, True), (40.0, False)])
def test_scores_vs_f64_bruteforce(device, pool, engine, scale, normalize):
    z, planted = pool
    zs = z * np.float32(scale)
    n = z.shape[0]
    a, b = om.rank_window(n)
    got = _MSM_hip.MSM(torch.from_numpy(zs).to(device), normalize_rows=normalize, engine=engine).cpu().numpy()
    ref = oracle.msm_scores_f64_c(z if normalize else zs, a, b)
    err = np.abs(got - ref)
    print(f'{engine} x{scale} normalize={normalize}: max err {err.max():.3e}; duplicated images: '
          f'{err[[0, 1, 3, 7]].max():.3e}', flush=True)
    # unnormalised rows scaled by s have distances s times larger: the gate scales with them
    assert err.max() <= ATOL * (1.0 if normalize else scale)


@pytest.mark.parametrize('engine', ['fp32', 'split16'])
def test_duplicated_images_score_exactly_zero_under_the_window(device, engine):
    # every image has a duplicate: each patch's smallest minimum is exactly 0, and with
    # the window [0, 1) the score is that minimum
    rng = np.random.default_rng(8)
    base = _unit(rng.standard_normal((4, 256, 64))).astype(np.float32)
    z = np.concatenate([base, base], 0)
    got = _MSM_hip.MSM(torch.from_numpy(z).to(device), topmin_min=0, topmin_max=1, engine=engine).cpu().numpy()
    assert np.all(got == 0.0), np.abs(got).max()


def test_nearest_distances_at_planted_pairs(device, pool):
    z, planted = pool
    got = _MSM_hip.nearest(torch.from_numpy(z).to(device)).cpu().numpy()
    ref = oracle.msm_nearest_f64_c(z)
    fin = np.isfinite(ref)
    assert np.isinf(got[~fin]).all()
    err = np.abs(got[fin] - ref[fin])
    p = z.shape[1]
    for i, qi, j, qj, d in planted:
        r = ref[i * p + qi, j]
        e = abs(got[i * p + qi, j] - r)
        # below the refinement bound: explicit differences in fp32, a few ulps of d^2 (the
        # expanded form left ~3e-4 near 0); above it the expanded form, within the gate
        tol = 1e-6 + 1e-5 * r if r * r <= 0.9 * 32 * 1.1920929e-7 * 1024 * 2 else ATOL
        assert e <= tol, (i, qi, j, d, got[i * p + qi, j], r)
    assert err.max() <= ATOL
    # the duplicated images: every patch's nearest patch in its twin is at exactly 0
    g3 = got.reshape(z.shape[0], p, z.shape[0])
    for i, j in ((0, 3), (1, 7)):
        assert np.all(g3[i, :, j] == 0.0) and np.all(g3[j, :, i] == 0.0)
