"""Mutual scoring module on MI355X: the drop-in `scoring` plugin.

Same call contract as the reference's accelerated MSM
(models/modules/_MSM_gpu.py:701-830) and its original (models/modules/_MSM.py:53-59),
as called at models/musc.py:254:

    scores = MSM(Z=Z, device=device, topmin_min=0, topmin_max=0.3)

Z is a (N, P, C) fp32 GPU tensor; the result is a (N, P) float64 GPU tensor on
Z's device.  Invalid input raises ValueError exactly where the reference does
(_MSM_gpu.py:702-711).  The work runs in libmusc_hip (musc_msm_scores_f32) on
torch's current stream; nothing synchronises.

Two engines form the pairwise dot products: 'fp32' (fp32 MFMA, the default) and
'split16' (each fp32 dot product from three fp16 MFMA products, hi.hi + hi.lo +
lo.hi of a hi/lo fp16 split of the normalised rows; error below 2^-22 |a||b|,
needs P >= 256).  Both share the minima, rank and output contract.
"""
from __future__ import annotations

import ctypes

import torch

from . import _runtime as rt


def rank_window(n: int, topmin_min: float = 0, topmin_max: float = 0.3) -> tuple[int, int]:
    """Trimmed rank window [a, b) -- _MSM_gpu.py:705-709 / _MSM.py:19-26."""
    a = int((n - 1) * topmin_min) if topmin_min < 1 else int(topmin_min)
    b = int((n - 1) * topmin_max) if topmin_max < 1 else int(topmin_max)
    a, b = sorted((a, b))
    return a, b


def _validate(Z: torch.Tensor) -> tuple[int, int, int]:
    if not isinstance(Z, torch.Tensor) or Z.ndim != 3 or not Z.is_cuda or Z.dtype != torch.float32:
        raise ValueError('Expected CUDA FP32 features with shape (N,P,C).')
    n, p, c = Z.shape
    if not (n >= 2 and p > 0 and c > 0):
        raise ValueError('Requires N>=2, P>0, C>0.')
    return n, p, c


ENGINES = ('fp32', 'split16')
SPLIT_MIN_P = 256


def check_engine(engine: str, p: int) -> None:
    if engine not in ENGINES:
        raise ValueError(f'Unknown MSM engine {engine!r}; expected one of {ENGINES}.')
    if engine == 'split16' and p < SPLIT_MIN_P:
        raise ValueError(f'The split16 MSM engine needs P >= {SPLIT_MIN_P} patches per image (got {p}).')


def workspace_bytes(n: int, p: int, c: int, engine: str = 'fp32') -> int:
    out = ctypes.c_size_t()
    lib = rt.library()
    if engine == 'split16':
        rt.check(lib.musc_msm_split_workspace_bytes(n, p, c, ctypes.byref(out)), 'musc_msm_split_workspace_bytes')
    else:
        rt.check(lib.musc_msm_workspace_bytes(n, p, c, ctypes.byref(out)), 'musc_msm_workspace_bytes')
    return out.value


def MSM(Z: torch.Tensor, device=None, topmin_min: float = 0, topmin_max: float = 0.3,
        workspace: torch.Tensor | None = None, out: torch.Tensor | None = None,
        normalize_rows: bool = False, engine: str = 'fp32') -> torch.Tensor:
    """(N, P) float64 mutual scores.  `workspace` / `out` let a caller reuse buffers.

    normalize_rows scores Z[i, q] / ||Z[i, q]|| instead of Z[i, q] (the L2
    normalisation of models/musc.py:238, applied inside the kernels).  `engine`
    selects how the dot products are formed ('fp32' or 'split16').
    """
    n, p, c = _validate(Z)
    a, b = rank_window(n, topmin_min, topmin_max)
    if not 0 <= a < b <= n - 1:
        raise ValueError('Require valid nonempty trimmed ranks 0<=a<b<=N-1.')
    check_engine(engine, p)
    lib = rt.library()
    with torch.cuda.device(Z.device):
        z = Z.contiguous()
        need = workspace_bytes(n, p, c, engine)
        ws = workspace if workspace is not None and workspace.numel() >= need else rt.workspace(need, z.device)
        if out is not None:
            if out.shape != (n, p) or out.dtype != torch.float64 or out.device != z.device or not out.is_contiguous():
                raise ValueError('out must be a contiguous (N, P) float64 tensor on the features device')
            scores = out
        else:
            scores = torch.empty((n, p), dtype=torch.float64, device=z.device)
        s = rt.stream(z.device)
        if engine == 'split16':
            flags = rt.MSM_NORMALIZE_ROWS if normalize_rows else 0
            rc = lib.musc_msm_split_scores_f32(z.data_ptr(), n, p, c, a, b, flags, scores.data_ptr(), ws.data_ptr(),
                                               ws.numel(), s)
            rt.check(rc, 'musc_msm_split_scores_f32')
            return scores
        if not normalize_rows:
            rc = lib.musc_msm_scores_f32(z.data_ptr(), n, p, c, a, b, scores.data_ptr(), ws.data_ptr(), ws.numel(), s)
            rt.check(rc, 'musc_msm_scores_f32')
            return scores
        rt.check(lib.musc_msm_prepare_f32(z.data_ptr(), n, p, c, rt.MSM_NORMALIZE_ROWS, ws.data_ptr(), ws.numel(), s),
                 'musc_msm_prepare_f32')
        rt.check(lib.musc_msm_pair_minima_f32(z.data_ptr(), n, p, c, ws.data_ptr(), ws.numel(), s),
                 'musc_msm_pair_minima_f32')
        rt.check(lib.musc_msm_refine_f32(z.data_ptr(), n, p, c, ws.data_ptr(), ws.numel(), s), 'musc_msm_refine_f32')
        rt.check(lib.musc_msm_rank_f32(n, p, a, b, scores.data_ptr(), ws.data_ptr(), ws.numel(), s),
                 'musc_msm_rank_f32')
        return scores


def nearest(Z: torch.Tensor, workspace: torch.Tensor | None = None) -> torch.Tensor:
    """(N*P, N) fp32 per-reference-image nearest distances, +inf on the own image.

    The intermediate of the scoring (`torch.min(torch.cdist(...), -1)[0]` at
    _MSM.py:16-17, the `nearest` tensor of _MSM_gpu.py:717).
    """
    n, p, c = _validate(Z)
    lib = rt.library()
    with torch.cuda.device(Z.device):
        z = Z.contiguous()
        need = workspace_bytes(n, p, c)
        ws = workspace if workspace is not None and workspace.numel() >= need else rt.workspace(need, z.device)
        out = torch.empty((n * p, n), dtype=torch.float32, device=z.device)
        rc = lib.musc_msm_nearest_f32(z.data_ptr(), n, p, c, out.data_ptr(), ws.data_ptr(), ws.numel(),
                                      rt.stream(z.device))
        rt.check(rc, 'musc_msm_nearest_f32')
        return out
