"""Zero-norm and non-finite features: the HIP path against the oracle, NaN positions exact.

The reference lets NaN through its scoring chain (musc.py:238's 0/0 for a zero feature,
torch.min's NaN propagation, topk ranking NaN last, NaN means; models/modules/_MSM.py:16-30),
and the oracle restates it (pinned on the CPU in test_oracle_nan.py).  Here both MSM
engines, the epilogue and RsCIN must reproduce the oracle's NaN positions exactly and its
finite values within the 2e-5 gate.
"""
import numpy as np
import pytest
import torch

from musc_hip import _MSM_hip, _RsCIN_hip, pipeline
from musc_hip.agreement import nan_aware_match
from oracle import epilogue as oe
from oracle import lnamd as ol
from oracle import msm as om
from oracle import rscin as orc

pytestmark = pytest.mark.gpu
ATOL = 2e-5
ENGINES = ['fp32', 'split16']


def _check(ref, got, what):
    res = nan_aware_match(ref, got, atol=ATOL)
    print(f'{what}: {res}', flush=True)
    assert res['pass'], (what, res)
    return res


def _raw_pool(seed, n=10, p=256, c=64):
    g = torch.Generator().manual_seed(seed)
    return torch.randn((n, p, c), generator=g) * 2.0 + 0.3


# p = 256: tiles aligned with the images; p = 300: tiles straddling image boundaries.  With
# the split engine, waves whose rows and columns all have unit norm reduce the dots alone,
# the others (here those holding a NaN-norm row) the distances: both kinds in one pool.
@pytest.mark.parametrize('p', [256, 300])
@pytest.mark.parametrize('engine', ENGINES)
def test_zero_and_nan_rows_with_row_normalisation(device, engine, p):
    # rows scored as z / ||z|| (MUSC_MSM_NORMALIZE_ROWS): a zero row is 0/0 = NaN as in
    # musc.py:238, a row holding a NaN is NaN, a zero image is all NaN
    z = _raw_pool(1, p=p)
    z[2, 5, 7] = float('nan')
    z[4, 9] = 0.0
    z[6] = 0.0
    got = _MSM_hip.MSM(z.to(device), normalize_rows=True, engine=engine).cpu()
    ref = om.MSM(z / z.norm(dim=-1, keepdim=True))
    res = _check(ref.numpy(), got.numpy(), f'{engine} normalised rows')
    assert res['reference_nan'] == 2 + p              # rows (2, 5), (4, 9) and image 6
    # the other images' scores are finite: the NaN minima rank last, outside [0, 2)
    assert torch.isfinite(got[[0, 1, 3, 5, 7, 8, 9]]).all()


@pytest.mark.parametrize('engine', ENGINES)
def test_nan_rows_of_normalised_features(device, engine):
    # features already normalised by the caller (the plugin contract of musc.py:238 + :254)
    z = _raw_pool(2)
    z[1, 0] = 0.0
    z[8, 255, 63] = float('nan')
    zn = z / z.norm(dim=-1, keepdim=True)
    got = _MSM_hip.MSM(zn.to(device), engine=engine).cpu()
    _check(om.MSM(zn).numpy(), got.numpy(), f'{engine} normalised features')


def test_nan_inside_the_rank_window(device):
    # with the window covering every rank the NaN minima are averaged in: all scores NaN
    z = _raw_pool(3)
    z[3] = 0.0
    zn = z / z.norm(dim=-1, keepdim=True)
    for engine in ENGINES:
        got = _MSM_hip.MSM(zn.to(device), topmin_min=0, topmin_max=9, engine=engine).cpu()
        ref = om.MSM(zn, 0, 9)
        _check(ref.numpy(), got.numpy(), f'{engine} full window')
        assert torch.isnan(got).all()


def test_infinite_entry_fp32_engine_nearest_and_scores(device):
    # an infinite entry in an unnormalised row: the expanded form gives NaN or +inf per pair
    # depending on the sign of the other row's entry, exactly as torch.cdist's matmul path
    z = _raw_pool(4)
    z[3, 8, 5] = float('inf')
    z[7, 100, 0] = float('-inf')
    zd = z.to(device)
    near = _MSM_hip.nearest(zd).cpu()
    _check(om.nearest(z).numpy(), near.numpy(), 'fp32 nearest with +-inf entries')
    got = _MSM_hip.MSM(zd).cpu()
    _check(om.MSM(z).numpy(), got.numpy(), 'fp32 scores with +-inf entries')


def test_infinite_minima_below_the_window_start(device):
    # a row whose minima against every other image are +inf (an infinite entry against
    # rows that are negative in that channel: +inf + inf in the expanded form), with a
    # window starting above 0 and b > 32 (the bit-search rank kernel, n <= 192): the
    # window holds only +inf, so the score is +inf (the reference's mean of topk values)
    # n = 300: the one-wave-per-row kernel (n > 192), same rule
    for n in (120, 300):
        g = torch.Generator().manual_seed(11)
        z = torch.randn((n, 16, 64), generator=g)
        z[:, :, 5] = -z[:, :, 5].abs() - 0.1
        z[3, 8, 5] = float('inf')
        z[7, 2] = float('nan')                    # NaN minima rank last in every other row
        zd = z.to(device)
        for lo, hi in ((0.1, 0.3), (0.0, 0.3), (0.2, 0.9)):
            got = _MSM_hip.MSM(zd, topmin_min=lo, topmin_max=hi).cpu()
            ref = om.MSM(z, lo, hi)
            _check(ref.numpy(), got.numpy(), f'n={n}: +inf minima, window ({lo}, {hi})')
            assert got[3, 8] == float('inf')


def test_small_pools_through_the_lds_epilogue(device):
    # P < 128 takes the LDS epilogue of the fp32 engine: same semantics
    g = torch.Generator().manual_seed(5)
    z = torch.randn((9, 37, 24), generator=g)
    z[2, 3] = 0.0
    z[5, 36, 1] = float('nan')
    got = _MSM_hip.MSM(z.to(device), normalize_rows=True).cpu()
    _check(om.MSM(z / z.norm(dim=-1, keepdim=True)).numpy(), got.numpy(), 'fp32 LDS epilogue')


def _poisoned_tokens(seed=6, n=10, side=16, c=64, layers=2):
    g = torch.Generator().manual_seed(seed)
    toks = [torch.randn((n, 1 + side * side, c), generator=g) + torch.randn((c,), generator=g)
            for _ in range(layers)]
    toks[0][3] = 0.5                              # a constant-token image: LayerNorm gives exact zeros
    toks[0][6, 20, 5] = float('nan')              # a NaN patch: the image's statistics become NaN
    toks[0][8, 100, 7] = float('inf')             # an Inf patch: likewise
    return toks


@pytest.mark.parametrize('engine', ENGINES)
def test_pipeline_constant_nan_inf_images(device, engine):
    toks = _poisoned_tokens()
    r_list = [1, 3]
    dev_toks = [t.to(device) for t in toks]
    pools = pipeline.lnamd_pools(dev_toks, r_list)
    scores = pipeline.msm_all(pools, engine=engine).cpu()
    maps, img = pipeline.score_pool(dev_toks, r_list, image_size=64, msm_engine=engine)
    per_r = []
    for ri, r in enumerate(r_list):
        feats = ol.l2_normalise(ol.lnamd_embed(toks, r))
        per_l = []
        for li in range(2):
            ref = om.MSM(feats[:, :, li, :].contiguous())
            _check(ref.numpy(), scores[ri, li].numpy(), f'{engine} r={r} layer {li} scores')
            per_l.append(ref)
        per_r.append(per_l)
    # layer 0 of images 3, 6 and 8 is all NaN, layer 1 finite everywhere
    assert torch.isnan(scores[:, 0, [3, 6, 8]]).all() and torch.isfinite(scores[:, 1]).all()
    ref_maps, ref_img = oe.maps_and_scores(per_r, 64)
    _check(ref_maps.numpy(), maps.cpu().numpy(), f'{engine} maps')
    _check(ref_img.numpy(), img.cpu().numpy(), f'{engine} image scores')
    assert torch.isnan(img.cpu()[[3, 6, 8]]).all() and torch.isfinite(img.cpu()[[0, 1, 2, 4, 5, 7, 9]]).all()


def test_epilogue_nan_stencil(device):
    from musc_hip import _epilogue_hip
    g = torch.Generator().manual_seed(7)
    scores = torch.rand((2, 3, 4, 49), generator=g, dtype=torch.float64)
    scores[1, 2, 0, 24] = float('nan')             # centre of image 0's 7 x 7 grid, one (r, l) map
    scores[0, 0, 3, 0] = float('nan')              # corner of image 3's grid
    maps, img = _epilogue_hip.maps_and_scores(scores.to(device), 50)
    ref_maps, ref_img = oe.maps_and_scores([[scores[r, l] for l in range(3)] for r in range(2)], 50)
    _check(ref_maps.numpy(), maps.cpu().numpy(), 'epilogue maps')
    _check(ref_img.numpy(), img.cpu().numpy(), 'epilogue image scores')


def test_rscin_nan_image_score(device):
    g = torch.Generator().manual_seed(8)
    cls = torch.nn.functional.normalize(torch.randn((12, 32), generator=g), dim=-1)
    raw = torch.rand((12,), generator=g, dtype=torch.float64)
    raw[4] = float('nan')
    got = _RsCIN_hip.RsCIN(raw.to(device), cls.to(device), [1, 2, 3]).cpu().numpy()
    with np.errstate(invalid='ignore'):
        ref = orc.rscin(raw.numpy(), list(cls.numpy()), [1, 2, 3])
    _check(ref, got, 'RsCIN with a NaN image score')
    assert np.isnan(got).all()
