"""End-to-end parity of the fused pipeline: tokens -> LNAMD -> L2 -> MSM -> maps, image scores."""
import numpy as np
import pytest
import torch

from oracle import epilogue as oe
from oracle import lnamd as ol
from oracle import msm as om
from musc_hip import pipeline, synthetic

pytestmark = pytest.mark.gpu
ATOL = 2e-5


def oracle_chain(tokens, r_list, image_size):
    """models/musc.py:227-288 restated with the oracle modules (CPU)."""
    per_r = []
    for r in r_list:
        feats = ol.l2_normalise(ol.lnamd_embed(tokens, r))          # (N, P, L, C)
        per_r.append([om.MSM(feats[:, :, l, :].contiguous()) for l in range(feats.shape[2])])
    return oe.maps_and_scores(per_r, image_size)


def test_config1_plumbing_end_to_end(device):
    tokens = synthetic.plumbing_tokens(8, seed=42)
    maps, img = pipeline.score_pool([tokens.to(device)], r_list=[1], image_size=518)
    ref_maps, ref_img = oracle_chain([tokens], [1], 518)
    err_m = (maps.cpu() - ref_maps).abs().max().item()
    err_i = (img.cpu() - ref_img).abs().max().item()
    print(f'config1 end-to-end: max map err {err_m:.3e}, image score err {err_i:.3e}', flush=True)
    assert err_m <= ATOL and err_i <= ATOL


def test_multi_layer_multi_radius_small(device):
    g = torch.Generator().manual_seed(11)
    tokens = [torch.randn((7, 82, 64), generator=g) + torch.randn((64,), generator=g) for _ in range(3)]
    maps, img = pipeline.score_pool([t.to(device) for t in tokens], r_list=[1, 3, 5], image_size=40)
    ref_maps, ref_img = oracle_chain(tokens, [1, 3, 5], 40)
    assert (maps.cpu() - ref_maps).abs().max().item() <= ATOL
    assert (img.cpu() - ref_img).abs().max().item() <= ATOL


def test_config2_full_size_sampled_images(device):
    # BASELINE config 2 at full size (83 images x 4 layers x 37x37 x 1024, radii 1/3/5): the
    # pipeline (LNAMD raw sums -> in-MSM row normalisation -> 12 MSM calls -> epilogue) against
    # the oracle chain for two query images.  An image's maps and score depend only on its own
    # 12 score rows, and compute_scores_fast restates the reference per query image.
    from musc_hip import _epilogue_hip
    torch.set_num_threads(min(16, torch.get_num_threads()))
    toks = synthetic.pool_tokens(83, 4, seed=42)
    pools = pipeline.lnamd_pools([t.to(device) for t in toks], [1, 3, 5])
    scores = pipeline.msm_all(pools)                                     # (3, 4, 83, 1369) float64
    del pools
    maps, img = _epilogue_hip.maps_and_scores(scores, 518)
    scores, maps, img = scores.cpu(), maps.cpu(), img.cpu()
    picks = (7, 60)
    ref_rows = [[None] * 4 for _ in range(3)]
    for ri, r in enumerate((1, 3, 5)):
        feats = ol.l2_normalise(ol.aggregate_direct(toks, r))            # (83, 1369, 4, 1024)
        for li in range(4):
            z = feats[:, :, li, :].contiguous()
            rows = torch.stack([om.compute_scores_fast(z, i).double() for i in picks], 0)
            err = (scores[ri, li, list(picks)] - rows).abs().max().item()
            print(f'config2 r={r} layer {li}: max score err {err:.3e}', flush=True)
            assert err <= ATOL
            ref_rows[ri][li] = rows
        del feats
    ref_maps, ref_img = oe.maps_and_scores(ref_rows, 518)
    err_m = (maps[list(picks)] - ref_maps).abs().max().item()
    err_i = (img[list(picks)] - ref_img).abs().max().item()
    print(f'config2 sampled maps err {err_m:.3e}, image score err {err_i:.3e}', flush=True)
    assert err_m <= ATOL and err_i <= ATOL
