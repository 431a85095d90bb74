"""Pin the CPU oracle before trusting it (CPU only).

Each restatement is checked against something it was not derived from: the
independent float64 brute forces, closed forms, invariants, the committed
golden fixtures, and (for the library calls) torch/scipy routines computing the
same mathematics another way.  A planted mistake in the oracle (a dropped
self-exclusion, a wrong rank window, a transposed operand, align_corners=False,
a missing r*r divisor) makes at least one of these fail.
"""
import math

import numpy as np
import pytest
import scipy.spatial.distance as ssd
import torch
import torch.nn.functional as F

import oracle
from oracle import attention as oa
from oracle import epilogue as oe
from oracle import lnamd as ol
from oracle import msm as om


def unit_rows(x):
    return x / np.linalg.norm(x, axis=-1, keepdims=True)


# --------------------------------------------------------------------------- MSM
def test_rank_window_matches_call_site():
    # models/musc.py:254 uses topmin_min=0, topmin_max=0.3
    assert om.rank_window(8) == (0, 2)
    assert om.rank_window(83) == (0, 24)
    assert om.rank_window(160) == (0, 47)
    assert om.rank_window(5) == (0, 1)
    assert om.rank_window(4) == (0, 0)            # empty window: the reference GPU path rejects N < 5
    assert om.rank_window(11, 0.3, 0.1) == (1, 3)  # reversed fractions are swapped (_MSM.py:25-26)
    assert om.rank_window(11, 0, 4) == (0, 4)      # integer ranks pass through


@pytest.mark.parametrize('case', ['a', 'b', 'c', 'd'])
def test_golden_msm_bruteforce_and_torch(golden, case):
    g = golden('msm_small.npz')
    z = g[f'{case}_z']
    np.testing.assert_allclose(om.nearest_bruteforce_f64(z), g[f'{case}_nearest'], rtol=0, atol=1e-12)
    np.testing.assert_allclose(om.msm_bruteforce_f64(z), g[f'{case}_scores'], rtol=0, atol=1e-12)
    torch_scores = om.MSM(torch.from_numpy(z)).numpy()
    np.testing.assert_allclose(torch_scores, g[f'{case}_scores'], rtol=0, atol=2e-6)
    nn = om.nearest(torch.from_numpy(z)).numpy()
    np.testing.assert_allclose(nn, g[f'{case}_nearest'], rtol=0, atol=2e-6)


def test_c_bruteforce_matches_numpy(golden):
    g = golden('msm_small.npz')
    for case in 'abcd':
        z = g[f'{case}_z']
        k_min, k_max = g[f'{case}_window']
        np.testing.assert_allclose(oracle.msm_nearest_f64_c(z), g[f'{case}_nearest'], rtol=0, atol=1e-12)
        np.testing.assert_allclose(oracle.msm_scores_f64_c(z, int(k_min), int(k_max)), g[f'{case}_scores'],
                                   rtol=0, atol=1e-12)


def test_torch_mm_path_matches_bruteforce():
    # P*(N-1) > 25 rows takes cdist's expanded-norm matmul path (the production path).
    rng = np.random.default_rng(1)
    z = unit_rows(rng.standard_normal((12, 40, 64))).astype(np.float32)
    ref = oracle.msm_scores_f64_c(z, *om.rank_window(12))
    got = om.MSM(torch.from_numpy(z)).numpy()
    np.testing.assert_allclose(got, ref, rtol=0, atol=5e-6)


def test_scipy_cdist_reduction():
    rng = np.random.default_rng(2)
    z = rng.standard_normal((5, 7, 6))
    near = om.nearest_bruteforce_f64(z)
    for i in range(5):
        for j in range(5):
            if i != j:
                np.testing.assert_allclose(near[i * 7:(i + 1) * 7, j], ssd.cdist(z[i], z[j]).min(1), atol=1e-12)


def test_closed_form_identical_images():
    rng = np.random.default_rng(3)
    base = unit_rows(rng.standard_normal((1, 9, 16)))
    z = np.repeat(base, 7, axis=0).astype(np.float32)
    assert np.abs(om.msm_bruteforce_f64(z)).max() == 0.0
    assert np.abs(oracle.msm_scores_f64_c(z, 0, 1)).max() == 0.0


def test_closed_form_one_dimensional_offsets():
    # Z[j] = base + delta_j * u with u a unit vector orthogonal to nothing special:
    # every patch's nearest patch in image j is the same patch, at |delta_j - delta_i|.
    rng = np.random.default_rng(4)
    n, p, c = 11, 6, 12
    base = rng.standard_normal((p, c)) * 10.0
    u = unit_rows(rng.standard_normal(c))
    delta = np.sort(rng.random(n)) * 0.05   # small offsets keep the same-patch match nearest
    z = (base[None] + delta[:, None, None] * u[None, None]).astype(np.float32)
    k_min, k_max = om.rank_window(n)
    expect = np.empty((n, p))
    zd = z.astype(np.float64)
    for i in range(n):
        for q in range(p):
            d = np.sort([np.linalg.norm(zd[j, q] - zd[i, q]) for j in range(n) if j != i])
            expect[i, q] = d[k_min:k_max].mean()
    np.testing.assert_allclose(om.msm_bruteforce_f64(z), expect, rtol=0, atol=1e-12)
    # and the closed form itself, |delta_j - delta_i| up to the float32 storage of z
    for i in range(n):
        d = np.sort([abs(delta[j] - delta[i]) for j in range(n) if j != i])
        assert abs(expect[i, 0] - d[k_min:k_max].mean()) < 1e-5


def test_closed_form_single_patch():
    rng = np.random.default_rng(5)
    z = rng.standard_normal((9, 1, 5)).astype(np.float32)
    d = ssd.cdist(z[:, 0].astype(np.float64), z[:, 0].astype(np.float64))
    k_min, k_max = om.rank_window(9)
    expect = np.array([np.sort(np.delete(d[i], i))[k_min:k_max].mean() for i in range(9)])
    np.testing.assert_allclose(om.msm_bruteforce_f64(z)[:, 0], expect, atol=1e-12)
    np.testing.assert_allclose(om.MSM(torch.from_numpy(z)).numpy()[:, 0], expect, atol=2e-6)


def test_invariants_permutation_and_scale():
    rng = np.random.default_rng(6)
    z = rng.standard_normal((8, 10, 6)).astype(np.float32)
    base = om.msm_bruteforce_f64(z)
    perm = rng.permutation(8)
    np.testing.assert_allclose(om.msm_bruteforce_f64(z[perm]), base[perm], atol=1e-12)
    pp = rng.permutation(10)
    np.testing.assert_allclose(om.msm_bruteforce_f64(z[:, pp]), base[:, pp], atol=1e-12)
    np.testing.assert_allclose(om.msm_bruteforce_f64(z * 4.0), base * 4.0, atol=1e-12)


def test_planted_self_exclusion_bug_is_caught():
    # A restatement that forgot to drop the query image would score 0 everywhere.
    rng = np.random.default_rng(7)
    z = rng.standard_normal((6, 5, 4))
    near = om.nearest_bruteforce_f64(z)
    buggy = near.copy()
    for row in range(30):
        buggy[row, row // 5] = 0.0
    bad = np.array([np.sort(r)[0:1].mean() for r in buggy]).reshape(6, 5)
    assert np.abs(bad - om.msm_bruteforce_f64(z)).max() > 0.1


# --------------------------------------------------------------------------- LNAMD
@pytest.mark.parametrize('r', [1, 3, 5])
def test_golden_lnamd(golden, r):
    g = golden('lnamd_small.npz')
    toks = g['tokens']
    np.testing.assert_allclose(ol.lnamd_bruteforce_f64(toks, r), g[f'r{r}'], atol=1e-12)
    t = torch.from_numpy(toks)
    unfold = ol.lnamd_embed([t], r)[:, :, 0].numpy()
    direct = ol.aggregate_direct([t], r)[:, :, 0].numpy()
    np.testing.assert_allclose(unfold, g[f'r{r}'], atol=2e-6)
    np.testing.assert_allclose(direct, g[f'r{r}'], atol=2e-6)


def test_lnamd_identity_multi_layer_full_grid():
    # The accelerated path's identity (_encoder_gpu.py:1-4) on the real 37x37 grid, 2 layers.
    g = torch.Generator().manual_seed(0)
    feats = [torch.randn((2, 1370, 32), generator=g) for _ in range(2)]
    for r in (1, 3, 5):
        a = ol.lnamd_embed(feats, r)
        b = ol.aggregate_direct(feats, r)
        assert a.shape == (2, 1369, 2, 32)
        torch.testing.assert_close(a, b, rtol=0, atol=3e-6)


def test_lnamd_r1_is_layernorm_and_constant_image_is_zero():
    g = torch.Generator().manual_seed(1)
    t = torch.randn((1, 26, 4), generator=g)
    y = ol.lnamd_embed([t], 1)[0, :, 0]                 # (25, 4)
    x = t[0, 1:].double()
    ref = (x - x.mean()) / torch.sqrt(x.var(unbiased=False) + 1e-5)
    torch.testing.assert_close(y.double(), ref, rtol=0, atol=2e-6)
    const = torch.full((1, 26, 4), 3.25)
    assert ol.lnamd_embed([const], 3).abs().max().item() == 0.0


def test_super_fast_known_answer(golden):
    # tools/test_super_fast.py:42-58: adaptive_avg_pool2d 37x37 -> 28x28 contract
    g = golden('super_fast_pool.npz')
    np.testing.assert_allclose(ol.adaptive_pool_bruteforce_f64(g['x'], 28), g['pooled'], atol=1e-12)
    feats = torch.from_numpy(g['x'].astype(np.float32)).reshape(1, 1369, 1, 1)
    pooled = ol.super_fast_pool(feats)
    assert pooled.shape == (1, 784, 1, 1)
    np.testing.assert_allclose(pooled[0, :, 0, 0].numpy().reshape(28, 28), g['pooled'], atol=1e-3)


def test_l2_normalise():
    x = torch.tensor([[[3.0, 4.0]]])
    torch.testing.assert_close(ol.l2_normalise(x), torch.tensor([[[0.6, 0.8]]]))


# --------------------------------------------------------------------------- epilogue
def test_golden_bilinear(golden):
    g = golden('bilinear_small.npz')
    grid = g['grid']
    for size, key in ((13, 'up13'), (37, 'up37')):
        up = oe.bilinear_align_corners_f64(grid, size)
        np.testing.assert_allclose(up, g[key], atol=1e-14)
        tor = F.interpolate(torch.from_numpy(grid).view(1, 1, 5, 5), size=size, mode='bilinear',
                            align_corners=True)[0, 0].numpy()
        np.testing.assert_allclose(tor, g[key], atol=1e-12)
        # align_corners=True: corners are the grid corners exactly
        for (a, b) in ((0, 0), (0, -1), (-1, 0), (-1, -1)):
            assert up[a, b] == grid[a, b]


def test_maps_and_scores_means_and_max():
    rng = np.random.default_rng(8)
    scores = [[torch.from_numpy(rng.random((3, 25))) for _ in range(4)] for _ in range(3)]
    maps, img = oe.maps_and_scores(scores, 13)
    avg = np.mean([np.mean([s.numpy() for s in per_l], 0) for per_l in scores], 0)
    for i in range(3):
        up = oe.bilinear_align_corners_f64(avg[i].reshape(5, 5), 13)
        np.testing.assert_allclose(maps[i, 0].numpy(), up, atol=1e-12)
        assert img[i].item() == pytest.approx(up.max(), abs=1e-12)
    # the maximum of a bilinear upsampling never exceeds the grid maximum
    assert (img.numpy() <= avg.max(1) + 1e-15).all()


# --------------------------------------------------------------------------- attention
def test_attention_closed_forms():
    rng = np.random.default_rng(9)
    k = rng.standard_normal((2, 7, 4))
    v = rng.standard_normal((2, 7, 4))
    q0 = np.zeros((2, 3, 4))
    np.testing.assert_allclose(oa.attention_f64(q0, k, v, 0.5), np.repeat(v.mean(1, keepdims=True), 3, 1),
                               atol=1e-14)
    q = np.zeros((1, 1, 4))
    kk = np.zeros((1, 5, 4))
    kk[0, 2, 0] = 1.0
    q[0, 0, 0] = 1000.0
    vv = rng.standard_normal((1, 5, 4))
    np.testing.assert_allclose(oa.attention_f64(q, kk, vv, 1.0)[0, 0], vv[0, 2], atol=1e-12)


def test_attention_matches_torch_fp32():
    g = torch.Generator().manual_seed(10)
    q, k, v = (torch.randn((3, 50, 64), generator=g) for _ in range(3))
    ref = torch.softmax((q / 8.0) @ k.transpose(1, 2), -1) @ v
    got = oa.attention_f64(q.numpy(), k.numpy(), v.numpy(), 1 / 8.0)
    np.testing.assert_allclose(ref.numpy(), got, atol=1e-5)


# --------------------------------------------------------------------------- RsCIN
def test_rscin_oracle_vs_bruteforce_and_closed_forms():
    from oracle import rscin as orc
    rng = np.random.default_rng(11)
    cls = rng.standard_normal((20, 16)).astype(np.float32)
    cls /= np.linalg.norm(cls, axis=1, keepdims=True)
    raw = rng.random(20) * 3.0
    for ks in ([1, 2, 3], [1, 8, 9], [4]):
        np.testing.assert_allclose(orc.rscin(raw, list(cls), ks), orc.rscin_bruteforce_f64(raw, cls, ks), atol=2e-6)
    # k = 1 keeps each row's own similarity (1 for unit tokens, the row maximum): scores are just min-max normalised
    np.testing.assert_allclose(orc.rscin(raw, list(cls), [1]), (raw - raw.min()) / (raw.max() - raw.min()), atol=1e-6)
    # 0 in k_list or no tokens: unchanged
    assert orc.rscin(raw, list(cls), [0, 1]) is raw and orc.rscin(raw, None, [1]) is raw


# ---------------------------------------------------------------------------
# Image preprocessing: Pillow's bicubic resampling restated (oracle.preprocess)
# ---------------------------------------------------------------------------

PIL_CASES = [((64, 64), (518, 518)), ((100, 80), (37, 41)), ((1024, 1024), (518, 518)), ((900, 900), (518, 518)),
             ((33, 517), (33, 518)), ((517, 33), (518, 33)), ((40, 40), (40, 40)), ((7, 5), (300, 2)),
             ((700, 840), (518, 518)), ((300, 3), (17, 3)), ((3, 3), (1, 1)), ((224, 224), (518, 518))]


@pytest.mark.parametrize('src,dst', PIL_CASES)
def test_preprocess_resize_matches_pillow(src, dst):
    # Pillow itself is the pin: the restatement must reproduce Image.resize(BICUBIC) byte for byte
    from PIL import Image
    from oracle import preprocess as op
    rng = np.random.default_rng(src[0] * 7 + dst[1])
    h, w = src
    img = rng.integers(0, 256, (h, w, 3), dtype=np.uint8)
    img[: h // 2] = (np.arange(w)[None, :, None] * 7 % 256).astype(np.uint8)   # sharp edges: clipping
    ref = np.asarray(Image.fromarray(img, 'RGB').resize((dst[1], dst[0]), Image.BICUBIC))
    np.testing.assert_array_equal(op.resize_bicubic_u8(img, *dst), ref)


def test_preprocess_coefficients_sum_to_one_and_planted_error_fails():
    from oracle import preprocess as op
    for n_in, n_out in ((1024, 518), (224, 518), (900, 518), (5, 5)):
        bounds, kk, taps = op.coefficients(n_in, n_out)
        assert taps == 2 * int(np.ceil(2 * max(n_in / n_out, 1.0))) + 1
        sums = kk.sum(axis=1)
        assert np.all(np.abs(sums - (1 << op.PRECISION_BITS)) <= taps)    # normalised up to rounding
        assert np.all(bounds[:, 0] >= 0) and np.all(bounds.sum(axis=1) <= n_in)
    # a plausible mistake (rounding the intermediate by truncation) must break the Pillow pin
    from PIL import Image
    rng = np.random.default_rng(3)
    img = rng.integers(0, 256, (50, 60, 3), dtype=np.uint8)
    ref = np.asarray(Image.fromarray(img, 'RGB').resize((23, 19), Image.BICUBIC))
    bh, kh, _ = op.coefficients(60, 23)
    acc = (img.astype(np.int64)[:, bh[5, 0]:bh[5, 0] + bh[5, 1], 0] * kh[5, :bh[5, 1]]).sum(axis=1)
    assert not np.array_equal(np.clip(acc >> op.PRECISION_BITS, 0, 255),
                              np.clip((acc + (1 << (op.PRECISION_BITS - 1))) >> op.PRECISION_BITS, 0, 255))
    assert np.array_equal(op.resize_bicubic_u8(img, 19, 23), ref)


def test_preprocess_to_tensor_normalize_rounding():
    # ToTensor is u / 255 and Normalize (x - m) / s, each a correctly rounded float32
    # operation (torch CPU).  Checked against exact rational arithmetic for every byte:
    # each stage's result must be a float32 nearest to the exact value of that stage
    # (a reciprocal multiply or a fused form would miss for some bytes).
    from fractions import Fraction
    from oracle import preprocess as op

    def nearest(x: np.float32, exact: Fraction) -> bool:
        up = np.nextafter(x, np.float32(np.inf))
        dn = np.nextafter(x, np.float32(-np.inf))
        e = abs(Fraction(float(x)) - exact)
        return e <= abs(Fraction(float(up)) - exact) and e <= abs(Fraction(float(dn)) - exact)

    img = np.arange(256, dtype=np.uint8).reshape(16, 16, 1).repeat(3, axis=2)
    got = op.to_tensor_normalize(img).numpy()
    plain = op.to_tensor_normalize(img, mean=(0.0, 0.0, 0.0), std=(1.0, 1.0, 1.0)).numpy()
    for c in range(3):
        m = np.float32(op.OPENAI_DATASET_MEAN[c])
        sd = np.float32(op.OPENAI_DATASET_STD[c])
        for u in range(256):
            t = plain[c].reshape(-1)[u]
            assert nearest(t, Fraction(u, 255)), u
            r = np.float32(t - m)
            assert nearest(r, Fraction(float(t)) - Fraction(float(m)))
            d = got[c].reshape(-1)[u]
            assert nearest(d, Fraction(float(r)) / Fraction(float(sd))), (c, u)
    assert plain[:, 0, 0].tolist() == [0.0] * 3 and plain[:, -1, -1].tolist() == [1.0] * 3


def test_rscin_check_gate():
    from oracle import rscin as orc
    # check_rscin accepts the float64 definition, reports no fp32 restatement flips on
    # well-separated similarities, and rejects a wrong value
    rng = np.random.default_rng(3)
    cls = rng.standard_normal((12, 64)).astype(np.float32)
    cls /= np.linalg.norm(cls, axis=1, keepdims=True)
    raw = rng.random(12)
    bf = orc.rscin_bruteforce_f64(raw, cls, [1, 2, 3])
    ok, info = orc.check_rscin(bf, raw, cls, [1, 2, 3])
    assert ok and info['fp32_restatement_flips'] == 0
    bad = bf.copy()
    bad[4] += 1e-3
    assert not orc.check_rscin(bad, raw, cls, [1, 2, 3])[0]
