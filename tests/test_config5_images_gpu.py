"""BASELINE config 5 from images: the product path against the model's own math path.

`pipeline.run_category` (the encoding hook with this build's fused blocks and attention,
LNAMD, MSM, the epilogue and RsCIN; models/musc.py:163-296) runs over the 160 seeded
images of config 5 on the random-init ViT-L/14 at 518 px.  The same model runs through
its own math path (nn.MultiheadAttention with need_weights=True, torch LayerNorm,
conv1, QuickGELU: open_clip/transformer.py:232-248, 555-614) and the oracle chain
(layer_norm + avg_pool2d, L2 normalisation, compute_scores_fast restated on the
device, the epilogue; oracle.msm.MSM_device is pinned against the C float64 brute force
in test_full_parity_gpu.py) scores those tokens.  The reference's harness compares
maps and scores of its two backends at 2e-5 (tools/benchmark.py:316-334,
tools/benchmark_support.py:11).

fp32 (no autocast): both paths round at 2^-24, and the gate is the reference's 2e-5
on the maps, the image scores and RsCIN's refined scores.  RsCIN keeps each row's k
largest class-token similarities, which is discontinuous: a row whose k-th and
(k+1)-th similarities lie closer than twice the largest similarity difference between
the two paths' class tokens may keep either image, so such rows are checked against
the definition on the product path's own inputs instead, and are counted.

fp16 autocast (config 5 as the reference runs it, musc.py:196): every fp16 GEMM output
rounds at 2^-11 relative, so any change of arithmetic order anywhere in the encoder
(a different softmax reduction, LayerNorm reduction or convolution algorithm) flips
roundings that the following blocks carry on; on this random-init encoder the tokens
then differ in most elements by an fp16 step or two and the maps by a few 1e-5.  The
reference's own accelerated encoder (models/modules/_attention_gpu.py:41-81, 141-146:
torch's bmm for both products, its own softmax with fp32 max and sum over the fp16
logits and P = fp16(exp(l - max) / sum)) is that kind of change.  The test restates it
in torch ops (F.softmax replaced while the math path runs, as the reference does),
measures its distance from the math path beside the product's, and gates the product
at twice that distance or 2e-5, whichever is larger (RsCIN likewise, on the rows whose
k nearest class tokens are the same under all three).  It also runs the product path
with its fused attention replaced by the same restatement (the math path's rounding
points: fp16 logits, fp32 max and sum, P = fp16(exp(l - max) / sum), fp16 P.V): the
maps then move by as much as the product's own do, so aligning the attention's
rounding points does not bring the fp16 comparison under 2e-5 either -- the
one-pass LayerNorm's reduction order alone moves them that far on this model.  With
the same model's weight matrices scaled by 1/4, whose blocks damp rounding
differences, the product meets the 2e-5 gate from images (last test).
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from musc_hip import _attention_hip, pipeline, synthetic, vit
from oracle import epilogue as oe
from oracle import lnamd as ol
from oracle import msm as om
from oracle import rscin as orc

pytestmark = pytest.mark.gpu
ATOL = 2e-5
LAYERS = (5, 11, 17, 23)
R_LIST = (1, 3, 5)
K_LIST = (1, 2, 3)
_F_SOFTMAX = F.softmax


@pytest.fixture(scope='module')
def setup(device):
    prev = (torch.backends.cuda.matmul.allow_tf32, torch.get_float32_matmul_precision())
    torch.backends.cuda.matmul.allow_tf32 = False
    torch.set_float32_matmul_precision('highest')
    torch.manual_seed(0)
    model = vit.vit_l14(518).eval().to(device)
    imgs, anomalous = synthetic.images(n=160, size=518, seed=42, anomaly_fraction=0.05)
    assert len(anomalous) == 8
    yield model, imgs.to(device)
    torch.backends.cuda.matmul.allow_tf32 = prev[0]
    torch.set_float32_matmul_precision(prev[1])


def _reference_design_softmax(input, dim=None, _stacklevel=3, dtype=None):
    """The reference's accelerated softmax (_attention_gpu.py:41-81) in torch ops: fp32
    maximum and sum over the fp16 logits, fp32 probabilities exp(l - max) / sum, which
    the following bmm rounds to fp16 under autocast (as it does torch's softmax)."""
    if input.dtype == torch.float16 and dim in (-1, input.ndim - 1) and dtype is None:
        x = input.float()
        e = torch.exp(x - x.amax(-1, keepdim=True))
        return e / e.sum(-1, keepdim=True)
    return _F_SOFTMAX(input, dim=dim, _stacklevel=_stacklevel, dtype=dtype)


def _reference_design_attention_packed(qkv, heads, scale):
    """The fused attention's place in the product path taken by the reference design's
    arithmetic in torch ops: softmax(q k^T * scale) v from the packed (T, B, 3E)
    in-projection, with torch's bmm for both products and _reference_design_softmax."""
    t, b, e3 = qkv.shape
    e = e3 // 3
    q, k, v = (qkv[..., i * e:(i + 1) * e].reshape(t, b * heads, 64).transpose(0, 1) for i in range(3))
    p = _reference_design_softmax(torch.bmm(q * scale, k.transpose(1, 2).contiguous()), dim=-1)
    o = torch.bmm(p.to(v.dtype), v.contiguous())
    return o.transpose(0, 1).reshape(t, b, e)


def _encode_math(model, imgs, autocast, softmax=None):
    """The model's own forward in batches of 4 (musc.py:196-215): tokens per layer and
    L2-normalised class tokens."""
    toks, cls = [[] for _ in LAYERS], []
    if softmax is not None:
        F.softmax = softmax
    try:
        with torch.no_grad(), torch.autocast('cuda', dtype=torch.float16, enabled=autocast):
            for s in range(0, imgs.shape[0], 4):
                pooled, t = model.encode_image(imgs[s:s + 4], [l + 1 for l in LAYERS])
                cls.append((pooled / pooled.norm(dim=-1, keepdim=True)).float())
                for l, x in enumerate(t):
                    toks[l].append(x)
    finally:
        F.softmax = _F_SOFTMAX
    return [torch.cat(t, 0).contiguous() for t in toks], torch.cat(cls, 0)


def _oracle_chain(tokens):
    """Maps and image scores of the oracle chain on `tokens` (musc.py:227-288)."""
    n, p = tokens[0].shape[0], tokens[0].shape[1] - 1
    scores = torch.empty((len(R_LIST), len(LAYERS), n, p), dtype=torch.float64, device=tokens[0].device)
    for ri, r in enumerate(R_LIST):
        feats = ol.l2_normalise(ol.aggregate_direct(tokens, r, device=None))
        for li in range(len(LAYERS)):
            scores[ri, li] = om.MSM_device(feats[:, :, li, :].contiguous())
        del feats
    s = scores.cpu()
    return oe.maps_and_scores([[s[ri, li] for li in range(len(LAYERS))] for ri in range(len(R_LIST))], 518)


def _max_err(a, b):
    a = a.cpu() if isinstance(a, torch.Tensor) else torch.as_tensor(a)
    b = b.cpu() if isinstance(b, torch.Tensor) else torch.as_tensor(b)
    assert a.shape == b.shape and torch.isfinite(a).all() and torch.isfinite(b).all()
    return (a.double() - b.double()).abs().max().item()


def _token_drift(a, b):
    out = []
    for x, y in zip(a, b):
        x, y = x.float(), y.float()
        out.append(f'{((x - y).norm() / y.norm()).item():.2e} rel, {(x != y).float().mean().item():.0%} differ')
    return '; '.join(out)


def _stable_rows(cls_ref, cls_got, k_list):
    """Rows whose k largest similarities are the same set under both class-token sets:
    the k-th and (k+1)-th largest of the reference row differ by more than twice the
    largest similarity difference between the two sets."""
    wr = cls_ref.double() @ cls_ref.double().T
    wg = cls_got.double() @ cls_got.double().T
    delta = (wr - wg).abs().max().item()
    s = torch.sort(wr, dim=1, descending=True).values
    ok = torch.ones(wr.shape[0], dtype=torch.bool, device=wr.device)
    for k in k_list:
        ok &= (s[:, k - 1] - s[:, k]) > 2 * delta
    return ok.cpu().numpy(), delta


def test_config5_fp32_from_images_both_engines(setup):
    model, imgs = setup
    ref_tok, ref_cls = _encode_math(model, imgs, autocast=False)
    ref_maps, ref_img = _oracle_chain(ref_tok)
    out = pipeline.run_category(model, imgs, feature_layers=LAYERS, r_list=R_LIST, batch_size=4, k_list=K_LIST,
                                autocast=False)
    assert all(t.dtype == torch.float32 and t.shape == (160, 1370, 1024) for t in out['tokens'])
    print(f'config5 fp32 tokens vs math path: {_token_drift(out["tokens"], ref_tok)}', flush=True)
    del ref_tok
    split_maps, split_img = pipeline.score_pool(out['tokens'], r_list=R_LIST, image_size=518, msm_engine='split16')
    for what, maps, img in (('fp32 engine', out['maps'], out['image_scores']), ('split16 engine', split_maps, split_img)):
        em, ei = _max_err(maps, ref_maps), _max_err(img, ref_img)
        print(f'config5 fp32 from images ({what}): maps {em:.3e}, image scores {ei:.3e}', flush=True)
        assert em <= ATOL and ei <= ATOL
    # RsCIN (musc.py:290-296) on the pipeline's image scores and class tokens
    got = out['scores'].cpu().numpy().astype(np.float64)
    ref = orc.rscin_bruteforce_f64(ref_img.numpy(), ref_cls.cpu().numpy(), list(K_LIST))
    stable, delta = _stable_rows(ref_cls, out['class_tokens'], K_LIST)
    err = np.abs(got - ref)
    print(f'config5 fp32 RsCIN from images: class-token similarities differ by {delta:.2e}; '
          f'{int(stable.sum())} of {len(stable)} rows keep the same neighbours, worst {err[stable].max():.3e}; '
          f'other rows worst {err[~stable].max() if (~stable).any() else 0.0:.3e}', flush=True)
    assert stable.mean() >= 0.9
    assert np.all(err[stable] <= ATOL)
    ok, info = orc.check_rscin(got, out['image_scores'].cpu().numpy(), out['class_tokens'].cpu().numpy(),
                               list(K_LIST), atol=ATOL)
    assert ok, info


def test_config5_fp16_from_images_within_reference_design_spread(setup, monkeypatch):
    model, imgs = setup
    ref_tok, ref_cls = _encode_math(model, imgs, autocast=True)
    ref_maps, ref_img = _oracle_chain(ref_tok)
    des_tok, des_cls = _encode_math(model, imgs, autocast=True, softmax=_reference_design_softmax)
    print(f'config5 fp16 reference-design tokens vs math path: {_token_drift(des_tok, ref_tok)}', flush=True)
    des_maps, des_img = _oracle_chain(des_tok)
    del des_tok
    spread = (_max_err(des_maps, ref_maps), _max_err(des_img, ref_img))
    print(f'config5 fp16 reference design vs math path: maps {spread[0]:.3e}, image scores {spread[1]:.3e}',
          flush=True)
    out = pipeline.run_category(model, imgs, feature_layers=LAYERS, r_list=R_LIST, batch_size=4, k_list=K_LIST,
                                autocast=True)
    print(f'config5 fp16 product tokens vs math path: {_token_drift(out["tokens"], ref_tok)}', flush=True)
    del ref_tok
    split_maps, split_img = pipeline.score_pool(out['tokens'], r_list=R_LIST, image_size=518, msm_engine='split16')
    gate = (max(ATOL, 2 * spread[0]), max(ATOL, 2 * spread[1]))
    for what, maps, img in (('fp32 engine', out['maps'], out['image_scores']), ('split16 engine', split_maps, split_img)):
        em, ei = _max_err(maps, ref_maps), _max_err(img, ref_img)
        print(f'config5 fp16 from images ({what}): maps {em:.3e}, image scores {ei:.3e} '
              f'(gate {gate[0]:.2e} / {gate[1]:.2e})', flush=True)
        assert em <= gate[0] and ei <= gate[1]
    # RsCIN (musc.py:290-296): on the rows whose k nearest class tokens are the same under
    # the math path, the reference design and the product, the product's refined scores
    # lie within twice the reference design's distance from the math path's (or 2e-5).
    # The random-init encoder's class tokens crowd together: fp16 moves their similarities
    # by ~3e-5, more than the gap between the k-th and (k+1)-th neighbour on most rows, so
    # about a fifth of the rows qualify; the others are checked against the definition on
    # the product's own inputs (check_rscin below).
    ref_rs = orc.rscin_bruteforce_f64(ref_img.numpy(), ref_cls.cpu().numpy(), list(K_LIST))
    des_rs = orc.rscin_bruteforce_f64(des_img.numpy(), des_cls.cpu().numpy(), list(K_LIST))
    got_rs = out['scores'].cpu().numpy().astype(np.float64)
    stable_des, delta_des = _stable_rows(ref_cls, des_cls, K_LIST)
    stable_got, delta_got = _stable_rows(ref_cls, out['class_tokens'], K_LIST)
    both = stable_des & stable_got
    rs_spread = np.abs(des_rs - ref_rs)[both].max() if both.any() else np.nan
    rs_err = np.abs(got_rs - ref_rs)[both].max() if both.any() else np.nan
    print(f'config5 fp16 RsCIN from images: class-token similarities differ by {delta_des:.2e} (reference '
          f'design), {delta_got:.2e} (product); {int(both.sum())} of {len(both)} rows keep the same '
          f'neighbours under both; reference design {rs_spread:.3e}, product {rs_err:.3e}', flush=True)
    assert both.sum() >= 16
    assert rs_err <= max(ATOL, 2 * rs_spread)
    ok, info = orc.check_rscin(got_rs, out['image_scores'].cpu().numpy(), out['class_tokens'].cpu().numpy(),
                               list(K_LIST), atol=ATOL)
    assert ok, info
    del out, split_maps, split_img
    # the product path with the math path's attention rounding points
    monkeypatch.setattr(_attention_hip, 'attention_packed', _reference_design_attention_packed)
    aligned = pipeline.run_category(model, imgs, feature_layers=LAYERS, r_list=R_LIST, batch_size=4,
                                    k_list=K_LIST, autocast=True)
    em, ei = _max_err(aligned['maps'], ref_maps), _max_err(aligned['image_scores'], ref_img)
    print(f'config5 fp16 from images, product path with the reference design attention: maps {em:.3e}, '
          f'image scores {ei:.3e}', flush=True)
    assert em <= gate[0] and ei <= gate[1]


def test_config5_fp16_from_images_at_quarter_weight_scale(setup):
    # The same architecture and images with every weight matrix scaled by 1/4: its blocks
    # damp rounding differences instead of amplifying them (the reference design's own
    # distance from the math path falls from 3.0e-5 to 4.6e-6, near the 4.3e-6 the
    # reference reports for its real-weight encoder, benchmarks/representative/REPORT.md:38),
    # so here the product must meet the reference's 2e-5 gate from images under fp16
    # autocast, both engines.  The scaled encoder's class tokens all but coincide (their
    # neighbour gaps lie below the paths' similarity differences), so RsCIN is checked
    # against the definition on the product's own inputs, and against the math path on
    # the rows whose neighbours are stable, if any
    _, imgs = setup
    torch.manual_seed(0)
    model = vit.vit_l14(518).eval().to(imgs.device)
    with torch.no_grad():
        for prm in model.parameters():
            if prm.ndim >= 2:
                prm.mul_(0.25)
    ref_tok, ref_cls = _encode_math(model, imgs, autocast=True)
    ref_maps, ref_img = _oracle_chain(ref_tok)
    out = pipeline.run_category(model, imgs, feature_layers=LAYERS, r_list=R_LIST, batch_size=4, k_list=K_LIST,
                                autocast=True)
    print(f'config5 fp16 at weight scale 1/4, product tokens vs math path: {_token_drift(out["tokens"], ref_tok)}',
          flush=True)
    del ref_tok
    split_maps, split_img = pipeline.score_pool(out['tokens'], r_list=R_LIST, image_size=518, msm_engine='split16')
    for what, maps, img in (('fp32 engine', out['maps'], out['image_scores']), ('split16 engine', split_maps, split_img)):
        em, ei = _max_err(maps, ref_maps), _max_err(img, ref_img)
        print(f'config5 fp16 at weight scale 1/4 ({what}): maps {em:.3e}, image scores {ei:.3e}', flush=True)
        assert em <= ATOL and ei <= ATOL
    got = out['scores'].cpu().numpy().astype(np.float64)
    ref = orc.rscin_bruteforce_f64(ref_img.numpy(), ref_cls.cpu().numpy(), list(K_LIST))
    stable, delta = _stable_rows(ref_cls, out['class_tokens'], K_LIST)
    err = np.abs(got - ref)
    print(f'config5 fp16 at weight scale 1/4, RsCIN: similarities differ by {delta:.2e}; {int(stable.sum())} of '
          f'{len(stable)} rows keep the same neighbours, worst {err[stable].max() if stable.any() else 0.0:.3e}',
          flush=True)
    assert np.all(err[stable] <= ATOL)
    ok, info = orc.check_rscin(got, out['image_scores'].cpu().numpy(), out['class_tokens'].cpu().numpy(),
                               list(K_LIST), atol=ATOL)
    assert ok, info
