"""Fused scoring pipeline: layer tokens -> anomaly maps + image scores.

Covers the hot path of MuSc.make_category_data (models/musc.py:225-288) for one
division, starting from the encoder's layer tokens:

    for r in r_list:                                   (musc.py:227)
        features = LNAMD_r(tokens); features /= ||features||   (:235-238)
        for l in layers: maps_l = MSM(Z_l, 0, 0.3)     (:250-256)
        maps_r = mean_l maps_l                          (:259)
    maps = mean_r maps_r; upsample bilinear align_corners  (:263-272)
    image score = max(maps)                             (:288)

MI355X layout: the whole pool stays resident in HBM.  One LNAMD launch reads
every layer's tokens once and writes every (radius, layer) pool contiguous,
(R, L, N, P, C) fp32 (5.6 GB at N=83, P=1369), as window sums of (x - mean):
the LayerNorm scale and the 1/r^2 of the box mean cancel in the L2
normalisation, which the MSM applies to each row on the fly
(MUSC_MSM_NORMALIZE_ROWS: its norms pass computes 1/||row|| and the pair
kernel's epilogue scales each dot product), so no pass over the 5.6 GB exists
just to normalise.  The R*L MSM calls reuse one workspace and write into one
(R, L, N, P) float64 score tensor, which the epilogue kernel reduces, upsamples
and maximises.  Everything is asynchronous on torch's current stream.
"""
from __future__ import annotations

import torch

from . import _MSM_hip, _epilogue_hip, _lnamd_hip
from ._RsCIN_hip import RsCIN
from . import _runtime as rt


def lnamd_pools(tokens: list[torch.Tensor], r_list: list[int], pool_grid: int | None = None) -> torch.Tensor:
    """(R, L, N, P, C) fp32 LNAMD window sums of (x - mean), to be scored with normalize_rows.

    Scored with row normalisation these give exactly the features of musc.py:227-243
    (LayerNorm, box mean, L2 normalisation), up to fp32 rounding.  `pool_grid`
    pools every patch grid to pool_grid x pool_grid in the same LNAMD pass (the
    super_fast aggregation, models/modules/_super_fast.py:17-27, ahead of the L2
    normalisation at musc.py:238); P is then pool_grid**2.
    """
    return _lnamd_hip.lnamd(tokens, r_list, raw_sums=True, layout='rlbpc', pool_side=pool_grid)


def msm_all(pools: torch.Tensor, topmin_min: float = 0, topmin_max: float = 0.3,
            pair_events: list | None = None, normalize_rows: bool = True, engine: str = 'fp32',
            rank_events: list | None = None, refine_events: list | None = None) -> torch.Tensor:
    """(R, L, N, P) float64 MSM maps of every (radius, layer) pool.

    Runs the four MSM stages explicitly (prepare, pair minima, cancellation
    refinement, rank) so that a caller can pass `pair_events`, a list that receives one (start, end)
    torch.cuda.Event pair recorded around each pair-minima kernel on the stream
    it runs on (`rank_events` and `refine_events` the same around each rank and
    cancellation-refinement kernel).  `engine` selects how the dot products are
    formed ('fp32' or 'split16', see _MSM_hip).
    """
    rt.require_device_tensor(pools, 'pools')
    if pools.ndim != 5 or pools.dtype != torch.float32 or not pools.is_contiguous():
        raise ValueError('pools must be a contiguous fp32 (R, L, N, P, C) tensor')
    r, l, n, p, c = pools.shape
    a, b = _MSM_hip.rank_window(n, topmin_min, topmin_max)
    if not 0 <= a < b <= n - 1:
        raise ValueError('Require valid nonempty trimmed ranks 0<=a<b<=N-1.')
    _MSM_hip.check_engine(engine, p)
    lib = rt.library()
    flags = rt.MSM_NORMALIZE_ROWS if normalize_rows else 0
    split = engine == 'split16'
    with torch.cuda.device(pools.device):
        scores = torch.empty((r, l, n, p), dtype=torch.float64, device=pools.device)
        ws = rt.workspace(_MSM_hip.workspace_bytes(n, p, c, engine), pools.device)
        s = rt.stream(pools.device)
        for ri in range(r):
            for li in range(l):
                z = pools[ri, li]
                if split:
                    rt.check(lib.musc_msm_split_prepare_f32(z.data_ptr(), n, p, c, flags, ws.data_ptr(), ws.numel(),
                                                            s), 'musc_msm_split_prepare_f32')
                else:
                    rt.check(lib.musc_msm_prepare_f32(z.data_ptr(), n, p, c, flags, ws.data_ptr(), ws.numel(), s),
                             'musc_msm_prepare_f32')
                if pair_events is not None:
                    ev = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                    ev[0].record()
                if split:
                    rt.check(lib.musc_msm_split_pair_minima(n, p, c, ws.data_ptr(), ws.numel(), s),
                             'musc_msm_split_pair_minima')
                else:
                    rt.check(lib.musc_msm_pair_minima_f32(z.data_ptr(), n, p, c, ws.data_ptr(), ws.numel(), s),
                             'musc_msm_pair_minima_f32')
                if pair_events is not None:
                    ev[1].record()
                    pair_events.append(ev)
                if refine_events is not None:
                    fev = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                    fev[0].record()
                rt.check(lib.musc_msm_refine_f32(z.data_ptr(), n, p, c, ws.data_ptr(), ws.numel(), s),
                         'musc_msm_refine_f32')
                if refine_events is not None:
                    fev[1].record()
                    refine_events.append(fev)
                if rank_events is not None:
                    rev = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                    rev[0].record()
                rt.check(lib.musc_msm_rank_f32(n, p, a, b, scores[ri, li].data_ptr(), ws.data_ptr(), ws.numel(), s),
                         'musc_msm_rank_f32')
                if rank_events is not None:
                    rev[1].record()
                    rank_events.append(rev)
    return scores


def score_pool(tokens: list[torch.Tensor], r_list=(1, 3, 5), image_size: int = 518, topmin_min: float = 0,
               topmin_max: float = 0.3, want_maps: bool = True, timing: dict | None = None,
               pool_grid: int | None = None, msm_engine: str = 'fp32'):
    """Tokens (list over layers of (N, 1+P, C) GPU tensors) -> (maps (N,1,S,S) f64, image scores (N,) f64).

    `timing`, if given, receives torch.cuda.Event pairs: timing['lnamd'] (one
    pair around the LNAMD launch), timing['pairs'] (one per MSM pair kernel),
    timing['refine'] (one per refinement kernel) and timing['rank'] (one per MSM
    rank kernel).
    `pool_grid` (the super_fast profile: 28) adaptively pools every patch grid to
    pool_grid x pool_grid before scoring (models/modules/_super_fast.py:17-27).
    `msm_engine` selects the MSM dot-product engine ('fp32' or 'split16').
    """
    lnamd_ev = None
    if timing is not None:
        lnamd_ev = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
        lnamd_ev[0].record()
    pools = lnamd_pools(tokens, list(r_list), pool_grid)
    if timing is not None:
        lnamd_ev[1].record()
        timing.setdefault('lnamd', []).append(lnamd_ev)
    scores = msm_all(pools, topmin_min, topmin_max,
                     pair_events=timing.setdefault('pairs', []) if timing is not None else None, engine=msm_engine,
                     rank_events=timing.setdefault('rank', []) if timing is not None else None,
                     refine_events=timing.setdefault('refine', []) if timing is not None else None)
    del pools
    return _epilogue_hip.maps_and_scores(scores, image_size, want_maps=want_maps)


def run_category(model, images: torch.Tensor, feature_layers=(5, 11, 17, 23), r_list=(1, 3, 5),
                 batch_size: int = 4, image_size: int | None = None, k_list=(1, 2, 3), autocast: bool = True,
                 pool_grid: int | None = None, timing: dict | None = None, msm_engine: str = 'fp32'):
    """One division of MuSc.make_category_data's hot path (models/musc.py:163-296) on the GPU.

    images (N, 3, S, S) normalised GPU tensor -> dict with 'maps' (N, 1, S, S) float64,
    'image_scores' (N,) float64 map maxima, 'scores' (N,) fp32 after RsCIN, 'class_tokens'
    (N, D) fp32.  The encoder runs in batches of `batch_size` under fp16 autocast (as at
    musc.py:196) with the fused attention (musc_hip._encoder_hip); layer tokens stay on
    the GPU; then LNAMD, MSM (engine `msm_engine`), the epilogue and RsCIN run as in
    score_pool.
    """
    from . import _encoder_hip

    n = images.shape[0]
    image_size = image_size or images.shape[-1]
    out_layers = [l + 1 for l in feature_layers]               # musc.py:61
    ev = (lambda: torch.cuda.Event(enable_timing=True)) if timing is not None else None
    if timing is not None:
        e0 = ev(); e0.record()
    _encoder_hip.begin_inference()
    tokens_per_layer = [[] for _ in out_layers]
    cls = []
    with torch.no_grad(), torch.autocast('cuda', dtype=torch.float16, enabled=autocast):
        for start in range(0, n, batch_size):
            pooled, toks = _encoder_hip.encode_image(model, images[start:start + batch_size], out_layers)
            pooled = pooled / pooled.norm(dim=-1, keepdim=True)  # musc.py:215
            cls.append(pooled.float())
            for l, t in enumerate(toks):
                tokens_per_layer[l].append(t)
    tokens = [torch.cat(t, 0).contiguous() for t in tokens_per_layer]
    class_tokens = torch.cat(cls, 0)
    if timing is not None:
        e1 = ev(); e1.record()
    maps, image_scores = score_pool(tokens, r_list=r_list, image_size=image_size, pool_grid=pool_grid,
                                    msm_engine=msm_engine)
    if timing is not None:
        e2 = ev(); e2.record()
    scores = RsCIN(image_scores, class_tokens, list(k_list))
    if timing is not None:
        e3 = ev(); e3.record()
        timing.setdefault('events', []).append((e0, e1, e2, e3))
    return {'maps': maps, 'image_scores': image_scores, 'scores': scores, 'class_tokens': class_tokens,
            'tokens': tokens}
