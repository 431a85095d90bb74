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
