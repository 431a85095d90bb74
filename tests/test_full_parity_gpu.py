"""BASELINE configs 2 and 3 at full size, every row of every MSM call, both engines.

The oracle's torch restatement (compute_scores_fast, models/modules/_MSM.py:10-30) runs
on the GPU box's device with full-fp32 matmuls (oracle.msm.MSM_device), one query image
at a time, on the same features the pipeline scores; it is pinned against the C float64
brute force on sampled rows.  The LNAMD features are checked against the oracle's
layer_norm + avg_pool2d restatement (models/modules/_encoder_gpu.py:14-42) on the device,
and the maps and image scores against the oracle epilogue (models/musc.py:259-288)
applied to the oracle's own scores.  Gate: 2e-5 absolute (tools/benchmark_support.py:11).
"""
import numpy as np
import pytest
import torch

import oracle
from musc_hip import _RsCIN_hip, _epilogue_hip, pipeline, synthetic, vit
from musc_hip.agreement import compare_arrays
from oracle import epilogue as oe
from oracle import lnamd as ol
from oracle import msm as om
from oracle import rscin as orc

pytestmark = pytest.mark.gpu
ATOL = 2e-5


@pytest.fixture(autouse=True)
def full_fp32_matmul():
    prev = (torch.backends.cuda.matmul.allow_tf32, torch.get_float32_matmul_precision())
    torch.backends.cuda.matmul.allow_tf32 = False
    torch.set_float32_matmul_precision('highest')
    yield
    torch.backends.cuda.matmul.allow_tf32 = prev[0]
    torch.set_float32_matmul_precision(prev[1])


def _gate(ref, got, what):
    res = compare_arrays(ref, got)
    print(f'{what}: pass={res["pass"]} max abs err {res.get("max_absolute_error")}', flush=True)
    assert res['pass'], (what, res)
    return res['max_absolute_error']


def _pin_device_oracle(z_dev, ref_scores, rows, label):
    """The device oracle's rows against the C float64 brute force over those rows."""
    n, p, _ = z_dev.shape
    a, b = om.rank_window(n)
    f64 = oracle.msm_row_scores_f64_c(z_dev.cpu().numpy(), rows, a, b)
    got = ref_scores.reshape(-1)[torch.as_tensor(rows)].cpu().numpy()
    err = np.abs(got - f64).max()
    print(f'{label}: device oracle vs float64 brute force on {len(rows)} rows: {err:.3e}', flush=True)
    assert err <= ATOL


def _sample_rows(n, p, k, seed):
    rng = np.random.default_rng(seed)
    return np.sort(rng.choice(n * p, size=k, replace=False))


def _full_pool_check(toks_dev, r_list, pool_grid, label):
    n_layers = len(toks_dev)
    pools = pipeline.lnamd_pools(toks_dev, r_list, pool_grid)          # (R, L, N, P, C) raw window sums
    got = {e: pipeline.msm_all(pools, engine=e) for e in ('fp32', 'split16')}
    n, p = pools.shape[2], pools.shape[3]
    ref = torch.empty((len(r_list), n_layers, n, p), dtype=torch.float64, device=pools.device)
    worst = {'features': 0.0, 'fp32': 0.0, 'split16': 0.0}
    for ri, r in enumerate(r_list):
        feats = ol.aggregate_direct(toks_dev, r, device=None)            # (N, P0, L, C) on the device
        if pool_grid is not None:
            feats = ol.super_fast_pool(feats, pool_grid)
        feats = ol.l2_normalise(feats)
        for li in range(n_layers):
            z_ref = feats[:, :, li, :].contiguous()
            z_gpu = pools[ri, li] / pools[ri, li].norm(dim=-1, keepdim=True)
            worst['features'] = max(worst['features'], _gate(z_ref, z_gpu, f'{label} r={r} l={li} features'))
            ref[ri, li] = om.MSM_device(z_ref)
            if ri == 0 and li == 0:
                _pin_device_oracle(z_ref, ref[ri, li], _sample_rows(n, p, 24, 1), label)
            for e in got:
                worst[e] = max(worst[e], _gate(ref[ri, li], got[e][ri, li], f'{label} r={r} l={li} {e} scores'))
        del feats
    ref_cpu = ref.cpu()
    side = int(round(p ** 0.5))
    ref_maps, ref_img = oe.maps_and_scores([[ref_cpu[ri, li] for li in range(n_layers)]
                                            for ri in range(len(r_list))], 518)
    imgs = {}
    for e in got:
        maps, img = _epilogue_hip.maps_and_scores(got[e], 518)
        worst[f'{e} maps'] = _gate(ref_maps, maps.cpu(), f'{label} {e} maps')
        worst[f'{e} image scores'] = _gate(ref_img, img.cpu(), f'{label} {e} image scores')
        imgs[e] = img
    print(f'{label}: worst errors over all {len(r_list) * n_layers} calls x {n} x {p} rows: {worst} '
          f'(grid {side}x{side})', flush=True)
    return ref_maps, ref_img, imgs


def test_config2_every_row_both_engines(device):
    toks = [t.to(device) for t in synthetic.pool_tokens(83, 4, seed=42)]
    _full_pool_check(toks, [1, 3, 5], None, 'config2')


def test_config3_every_row_both_engines(device):
    # super_fast-shaped pool: one layer, r = 3, 37 x 37 adaptively pooled to 28 x 28 (P = 784)
    toks = [t.to(device) for t in synthetic.pool_tokens(83, 1, seed=5)]
    _full_pool_check(toks, [3], 28, 'config3')


# Encoder tokens under fp16 autocast: the fused blocks against the same model's own
# math path (nn.MultiheadAttention, torch LayerNorm/QuickGELU), after 6/12/18/24 of the 24
# blocks.  Both compute in fp16 under autocast but round at different points (the fused
# attention keeps its softmax statistics and probabilities in fp32 up to the P.V product;
# LayerNorm and the residual add are fused), so they drift apart by fp16 rounding steps
# that later blocks carry forward.  Bound: relative Frobenius error per layer.
TOKEN_REL_TOL = 1e-2


def test_config5_end_to_end_both_engines(device):
    # random-init ViT-L/14 at 518 px, 160 seeded uniform images (8 with an
    # intensity-shifted rectangle), batch 4 under fp16 autocast, tokens after blocks
    # 6/12/18/24, LNAMD r = 1/3/5, MSM over all 160 x 159 pairs (ranks [0, 47)), the
    # epilogue and RsCIN k = 1/2/3 (models/musc.py:163-296)
    torch.manual_seed(0)
    model = vit.vit_l14(518).eval().to(device)
    imgs, anomalous = synthetic.images(n=160, size=518, seed=42, anomaly_fraction=0.05)
    assert len(anomalous) == 8
    imgs = imgs.to(device)
    layers = (5, 11, 17, 23)
    out = pipeline.run_category(model, imgs, feature_layers=layers, r_list=(1, 3, 5), batch_size=4,
                                k_list=(1, 2, 3), autocast=True)
    assert all(t.dtype == torch.float16 and t.shape == (160, 1370, 1024) for t in out['tokens'])
    # (a) the first batch's tokens against the model's math path
    with torch.no_grad(), torch.autocast('cuda', dtype=torch.float16):
        _, ref_tokens = model.encode_image(imgs[:4], [l + 1 for l in layers])
    for l, (a, b) in enumerate(zip(out['tokens'], ref_tokens)):
        a, b = a[:4].float(), b.float()
        rel = ((a - b).norm() / b.norm()).item()
        print(f'config5 layer {layers[l]} tokens: relative Frobenius error {rel:.3e}, max abs '
              f'{(a - b).abs().max().item():.3e} (max |ref| {b.abs().max().item():.3e})', flush=True)
        assert rel <= TOKEN_REL_TOL
    del ref_tokens
    # (b) every score row of all 12 calls, both engines, from the GPU's own tokens; maps and
    # image scores through the epilogue
    ref_maps, ref_img, imgs_by_engine = _full_pool_check(out['tokens'], [1, 3, 5], None, 'config5')
    # (c) the pipeline's own outputs (fp32 engine) and RsCIN on the class tokens
    _gate(ref_maps, out['maps'].cpu(), 'config5 run_category maps')
    _gate(ref_img, out['image_scores'].cpu(), 'config5 run_category image scores')
    # RsCIN's top-k neighbour choice is discontinuous: where two similarities are closer
    # than fp32 rounding can settle, the reference's own choice depends on its summation
    # order, so such rows may match either the float64 definition or the fp32
    # restatement (oracle.rscin.check_rscin); every other row must match both
    cls = out['class_tokens'].cpu().numpy()
    for what, got in (('fp32 engine', out['scores']),
                      ('split16 engine', _RsCIN_hip.RsCIN(imgs_by_engine['split16'], out['class_tokens'], [1, 2, 3]))):
        ok, info = orc.check_rscin(got.cpu().numpy(), ref_img.numpy(), cls, [1, 2, 3], atol=ATOL)
        print(f'config5 RsCIN ({what}): pass={ok} {info}', flush=True)
        assert ok, (what, info)
