"""The oracle's semantics for zero-norm and non-finite features, pinned on the CPU.

The reference lets NaN through its scoring chain: models/musc.py:238 divides each
feature by its norm with no epsilon (a zero feature becomes 0/0 = NaN), torch.min over
cdist rows propagates NaN (models/modules/_MSM.py:16-17), torch.topk(largest=False)
ranks NaN after every number (:27-28) and the fp32 mean over a window holding a NaN
is NaN (:30); F.interpolate spreads a NaN grid value to every pixel whose 2x2 stencil
holds it, even at weight 0 (musc.py:271-272), numpy's max propagates it into the image
score (:288) and RsCIN's min-max normalisation into every refined score
(_RsCIN.py:27).  The oracle restates those calls, so it inherits the semantics; these
tests pin it against definitions that do not use the same torch calls: the numpy
explicit-difference brute force, the C brute force, a float64 expanded-form brute
force for infinite entries, the float64 bilinear loop and the RsCIN brute force.
"""
import numpy as np
import torch

import oracle
from musc_hip.agreement import nan_aware_match
from oracle import epilogue as oe
from oracle import lnamd as ol
from oracle import msm as om
from oracle import rscin as orc


def unit(x):
    with np.errstate(invalid='ignore', divide='ignore'):
        return x / np.linalg.norm(x, axis=-1, keepdims=True)


def poisoned_pool(seed=0, n=9, p=30, c=16):
    """Unit rows with a NaN row (image 2), a zero row turned NaN by the 0/0 of
    musc.py:238 (image 5) and a whole zero image (image 7: all rows NaN)."""
    rng = np.random.default_rng(seed)
    z = rng.standard_normal((n, p, c)).astype(np.float32)
    z[2, 4, 3] = np.nan
    z[5, 11] = 0.0
    z[7] = 0.0
    return unit(z).astype(np.float32)


def test_msm_nan_rows_match_bruteforces():
    z = poisoned_pool()
    n, p, _ = z.shape
    a, b = om.rank_window(n)
    got = om.MSM(torch.from_numpy(z)).numpy()
    ref = om.msm_bruteforce_f64(z)
    res = nan_aware_match(ref, got, atol=5e-6)
    assert res['pass'], res
    # the NaN rows themselves, and the whole NaN image, score NaN; no other row does
    # (three NaN minima rank last among 8 and the window is [0, 2))
    expect = np.zeros((n, p), dtype=bool)
    expect[2, 4] = expect[5, 11] = True
    expect[7] = True
    assert np.array_equal(np.isnan(got), expect)
    np.testing.assert_allclose(oracle.msm_scores_f64_c(z, a, b), ref, rtol=0, atol=1e-12, equal_nan=True)


def test_msm_nan_inside_the_rank_window_makes_the_score_nan():
    # with the window reaching the NaN ranks, finite rows score NaN too (mean over a NaN)
    z = poisoned_pool(seed=1)
    got = om.MSM(torch.from_numpy(z), 0, 8).numpy()       # window [0, 8): every rank
    ref = om.msm_bruteforce_f64(z, 0, 8)
    assert nan_aware_match(ref, got, atol=5e-6)['pass']
    assert np.isnan(got).all()                             # every row sees the NaN images


def test_msm_infinite_entry_expanded_form():
    # An infinite entry in an unnormalised row: the expanded form ||a||^2 + ||b||^2 - 2 a.b
    # of torch.cdist's matmul path gives inf - inf = NaN where the infinite product's sign
    # is +, and +inf where it is - (or where both terms are +inf).
    rng = np.random.default_rng(3)
    n, p, c = 7, 30, 12
    z = rng.standard_normal((n, p, c)).astype(np.float32)
    z[3, 8, 5] = np.inf
    got_near = om.nearest(torch.from_numpy(z)).numpy()
    got = om.MSM(torch.from_numpy(z)).numpy()
    zz = z.astype(np.float64).reshape(n * p, c)
    with np.errstate(invalid='ignore', over='ignore'):
        sq = (zz * zz).sum(-1)
        d2 = sq[:, None] + sq[None, :] - 2.0 * (zz @ zz.T)
        d = np.sqrt(np.where(np.isnan(d2), d2, np.maximum(d2, 0.0)))   # clamp_min(0) keeps NaN
    near = np.full((n * p, n), np.inf)
    for i in range(n):
        for j in range(n):
            if j != i:
                near[i * p:(i + 1) * p, j] = d[i * p:(i + 1) * p, j * p:(j + 1) * p].min(1)  # np.min keeps NaN
    # both outcomes occur among the distances to the infinite row, so its image's minima are
    # NaN for some query rows and finite (the +inf pair is not the minimum) for others
    col = d[:, 3 * p + 8].reshape(n, p)[[i for i in range(n) if i != 3]]
    assert np.isnan(col).any() and np.isposinf(col).any()
    mins = near[:, 3].reshape(n, p)[[i for i in range(n) if i != 3]]
    assert np.isnan(mins).any() and np.isfinite(mins).any()
    res = nan_aware_match(near, got_near, atol=5e-6)
    assert res['pass'], res
    a, b = om.rank_window(n)
    ref = om.scores_from_nearest_f64(near, n, p, a, b)
    assert nan_aware_match(ref, got, atol=5e-6)['pass']


def test_c_bruteforce_rows_match_full():
    rng = np.random.default_rng(5)
    z = unit(rng.standard_normal((8, 20, 24))).astype(np.float32)
    z[6, 3] = np.nan
    a, b = om.rank_window(8)
    full = oracle.msm_scores_f64_c(z, a, b).reshape(-1)
    rows = np.array([0, 7, 19, 61, 159, 6 * 20 + 3])        # the last is the NaN row
    got = oracle.msm_row_scores_f64_c(z, rows, a, b)
    np.testing.assert_allclose(got, full[rows], rtol=0, atol=0, equal_nan=True)
    assert np.isnan(got[-1]) and np.isfinite(got[:-1]).all()


def test_lnamd_constant_image_becomes_nan_after_l2():
    # a constant-token image: LayerNorm over (C, H, W) gives exact zeros, the box mean keeps
    # them, and musc.py:238's 0/0 makes every feature of that image NaN
    rng = np.random.default_rng(7)
    tok = rng.standard_normal((3, 1 + 16, 8)).astype(np.float32)
    tok[1] = 0.5
    for r in (1, 3):
        f = ol.l2_normalise(ol.lnamd_embed([torch.from_numpy(tok)], r))
        bf = ol.lnamd_bruteforce_f64(tok, r)
        assert (bf[1] == 0).all()
        assert torch.isnan(f[1]).all() and torch.isfinite(f[[0, 2]]).all()


def test_lnamd_nonfinite_token_poisons_its_image():
    # a NaN or +inf token makes the image's LayerNorm statistics non-finite: every output of
    # that image is NaN, the other images are untouched
    rng = np.random.default_rng(8)
    tok = rng.standard_normal((3, 1 + 25, 8)).astype(np.float32)
    tok[0, 7, 2] = np.nan
    tok[2, 13, 5] = np.inf
    for r in (1, 3, 5):
        f = ol.l2_normalise(ol.lnamd_embed([torch.from_numpy(tok)], r))
        assert torch.isnan(f[0]).all() and torch.isnan(f[2]).all() and torch.isfinite(f[1]).all()
        with np.errstate(invalid='ignore'):
            bf = ol.lnamd_bruteforce_f64(tok, r)
        assert np.isnan(bf[0]).all() and np.isnan(bf[2]).all()


def test_epilogue_nan_stencil_and_image_score():
    rng = np.random.default_rng(9)
    grid = rng.random((2, 25))
    grid[0, 12] = np.nan                       # centre of a 5 x 5 grid
    maps, img = oe.maps_and_scores([[torch.from_numpy(grid)]], 13)
    bf = oe.bilinear_align_corners_f64(grid[0].reshape(5, 5), 13)
    assert np.array_equal(np.isnan(maps[0, 0].numpy()), np.isnan(bf))
    assert np.isnan(bf).any() and not np.isnan(bf).all()
    np.testing.assert_allclose(maps[0, 0].numpy(), bf, atol=1e-12, equal_nan=True)
    assert np.isnan(img[0].item()) and np.isfinite(img[1].item())
    assert np.isnan(np.asarray(maps[0, 0]).max())       # numpy's max (musc.py:288) propagates as well


def test_rscin_nan_score_poisons_every_refined_score():
    rng = np.random.default_rng(10)
    cls = rng.standard_normal((12, 8)).astype(np.float32)
    cls /= np.linalg.norm(cls, axis=1, keepdims=True)
    raw = rng.random(12)
    raw[4] = np.nan
    with np.errstate(invalid='ignore'):
        got = orc.rscin(raw, list(cls), [1, 2, 3])
        bf = orc.rscin_bruteforce_f64(raw, cls, [1, 2, 3])
    assert np.isnan(got).all() and np.isnan(bf).all()
