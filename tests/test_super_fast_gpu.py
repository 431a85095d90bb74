"""super_fast profile on the GPU: the reference's known-answer pooling test, the plugin
contract (tools/test_super_fast.py:42-58) and the 28x28 scoring pipeline."""
from types import SimpleNamespace
from unittest.mock import patch

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import epilogue as oe
from oracle import lnamd as ol
from oracle import msm as om
from musc_hip import _lnamd_hip, _super_fast, pipeline

pytestmark = pytest.mark.gpu
ATOL = 2e-5


def test_known_answer_arange(golden, device):
    g = golden('super_fast_pool.npz')
    x = torch.from_numpy(g['x'].astype(np.float32)).reshape(1, 1369, 1, 1).repeat(1, 1, 1, 4).to(device)
    out = _super_fast.adaptive_pool(x, 28).cpu()
    assert out.shape == (1, 784, 1, 4)
    np.testing.assert_allclose(out[0, :, 0, 0].numpy().reshape(28, 28), g['pooled'], rtol=2e-7, atol=0)


def test_plugin_contract_and_factory_lifetime(device):
    # same contract as tools/test_super_fast.py:42-58, with the features on the GPU
    features = torch.arange(2 * 1369 * 8, dtype=torch.float32).reshape(2, 1369, 1, 8).half().to(device)

    class Base:
        cleared = False

        def __call__(self, *args, **kwargs):
            return features

        def clear(self):
            self.cleared = True

    with patch.object(_super_fast, 'RadiusAggregationCache', side_effect=Base):
        first = _super_fast.new_aggregation()
        second = _super_fast.new_aggregation()
    assert first.base is not second.base
    output = first(SimpleNamespace(r=3), [], return_cpu=False)
    expected = F.adaptive_avg_pool2d(features.cpu()[:, :, 0].transpose(1, 2).reshape(2, 8, 37, 37).float(),
                                     (28, 28)).half().flatten(2).transpose(1, 2).unsqueeze(2).contiguous()
    assert torch.equal(output.cpu(), expected)
    assert output.shape == (2, 784, 1, 8)
    first.clear()
    assert first.base.cleared and not second.base.cleared
    with pytest.raises(ValueError):
        first(SimpleNamespace(r=1), [])


def test_super_fast_pipeline_vs_oracle(device):
    g = torch.Generator().manual_seed(13)
    tokens = [torch.randn((8, 1370, 64), generator=g) + torch.randn((64,), generator=g)]
    maps, img = pipeline.score_pool([t.to(device) for t in tokens], r_list=[3], image_size=96, pool_grid=28)
    feats = ol.l2_normalise(ol.super_fast_pool(ol.lnamd_embed(tokens, 3)))      # (N, 784, 1, C)
    ref_maps, ref_img = oe.maps_and_scores([[om.MSM(feats[:, :, 0, :].contiguous())]], 96)
    assert maps.shape == (8, 1, 96, 96)
    assert (maps.cpu() - ref_maps).abs().max().item() <= ATOL
    assert (img.cpu() - ref_img).abs().max().item() <= ATOL
