"""End-to-end (config 5 in miniature): images -> encoder with fused attention -> LNAMD ->
MSM -> epilogue -> RsCIN, against the oracle chain on the same model's math path."""
import numpy as np
import pytest
import torch

from oracle import epilogue as oe
from oracle import lnamd as ol
from oracle import msm as om
from oracle import rscin as orc
from musc_hip import pipeline, synthetic, vit

pytestmark = pytest.mark.gpu


def test_small_category_end_to_end(device):
    torch.manual_seed(0)
    model = vit.CLIPVision(image_size=84, patch_size=14, width=128, layers=4, heads=2, output_dim=32).eval()
    imgs, anomalous = synthetic.images(n=8, size=84, seed=3, anomaly_fraction=0.25)
    assert len(anomalous) == 2
    layers, r_list = (1, 3), (1, 3, 5)
    out = pipeline.run_category(model.to(device), imgs.to(device), feature_layers=layers, r_list=r_list,
                                batch_size=4, k_list=(1, 2, 3), autocast=False)
    # oracle: the same model on the CPU with nn.MultiheadAttention's math path
    cpu_model = model.cpu()
    with torch.no_grad():
        toks, cls = [[], []], []
        for s in range(0, 8, 4):
            pooled, t = cpu_model.encode_image(imgs[s:s + 4], [l + 1 for l in layers])
            cls.append(pooled / pooled.norm(dim=-1, keepdim=True))
            for i in range(2):
                toks[i].append(t[i])
    ref_tokens = [torch.cat(t, 0) for t in toks]
    for a, b in zip(out['tokens'], ref_tokens):
        torch.testing.assert_close(a.cpu(), b, rtol=1e-4, atol=1e-4)
    # downstream from the GPU's own tokens: the scoring gate 2e-5
    per_r = []
    gpu_toks = [t.cpu() for t in out['tokens']]
    for r in r_list:
        feats = ol.l2_normalise(ol.lnamd_embed(gpu_toks, r))
        per_r.append([om.MSM(feats[:, :, l, :].contiguous()) for l in range(2)])
    ref_maps, ref_img = oe.maps_and_scores(per_r, 84)
    assert (out['maps'].cpu() - ref_maps).abs().max().item() <= 2e-5
    assert (out['image_scores'].cpu() - ref_img).abs().max().item() <= 2e-5
    # RsCIN against its definition, fp32 tie-breaks of the top-k choice allowed
    ok, info = orc.check_rscin(out['scores'].cpu().numpy(), ref_img.numpy(), out['class_tokens'].cpu().numpy(),
                               [1, 2, 3], atol=2e-5)
    assert ok, info


def test_category_end_to_end_split_engine(device):
    # a 16 x 16 patch grid (224 px) so that P = 256 meets the split engine's minimum
    torch.manual_seed(1)
    model = vit.CLIPVision(image_size=224, patch_size=14, width=128, layers=4, heads=2, output_dim=32).eval()
    imgs, _ = synthetic.images(n=8, size=224, seed=4, anomaly_fraction=0.25)
    layers, r_list = (1, 3), (1, 3, 5)
    kw = dict(feature_layers=layers, r_list=r_list, batch_size=4, k_list=(1, 2, 3), autocast=False)
    out16 = pipeline.run_category(model.to(device), imgs.to(device), msm_engine='split16', **kw)
    out32 = pipeline.run_category(model.to(device), imgs.to(device), msm_engine='fp32', **kw)
    for a, b in zip(out16['tokens'], out32['tokens']):
        torch.testing.assert_close(a, b, rtol=0, atol=1e-6)  # the encoder does not depend on the engine
    # the split engine's maps against the oracle chain from the same tokens (gate 2e-5)
    per_r = []
    gpu_toks = [t.cpu() for t in out16['tokens']]
    for r in r_list:
        feats = ol.l2_normalise(ol.lnamd_embed(gpu_toks, r))
        per_r.append([om.MSM(feats[:, :, l, :].contiguous()) for l in range(2)])
    ref_maps, ref_img = oe.maps_and_scores(per_r, 224)
    err_m = (out16['maps'].cpu() - ref_maps).abs().max().item()
    err_i = (out16['image_scores'].cpu() - ref_img).abs().max().item()
    print(f'split engine end to end: max map err {err_m:.3e}, image-score err {err_i:.3e}', flush=True)
    assert err_m <= 2e-5 and err_i <= 2e-5
    assert (out16['maps'] - out32['maps']).abs().max().item() <= 2e-5
    np.testing.assert_allclose(out16['scores'].cpu().numpy(), out32['scores'].cpu().numpy(), rtol=0, atol=2e-5)
