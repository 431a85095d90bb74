"""Score-map epilogue on MI355X (libmusc_hip musc_maps_f64).

Fuses models/musc.py:259-288: float64 mean over layers, then over radii, bilinear
upsampling with align_corners=True to image_size x image_size, and the image
score as the maximum of each map.
"""
from __future__ import annotations

import math

import torch

from . import _runtime as rt


def maps_and_scores(scores: torch.Tensor, image_size: int, want_maps: bool = True):
    """scores (R, L, N, P) float64 GPU tensor -> maps (N, 1, S, S) float64 (or None), image scores (N,)."""
    rt.require_device_tensor(scores, 'scores')
    if scores.ndim != 4 or scores.dtype != torch.float64:
        raise ValueError('scores must be a (R, L, N, P) float64 tensor')
    r, l, n, p = scores.shape
    side = math.isqrt(p)
    if side * side != p:
        raise ValueError('P must be a square grid')
    s = scores.contiguous()
    with torch.cuda.device(s.device):
        maps = torch.empty((n, 1, image_size, image_size), dtype=torch.float64, device=s.device) if want_maps else None
        img = torch.empty((n,), dtype=torch.float64, device=s.device)
        rc = rt.library().musc_maps_f64(s.data_ptr(), r, l, n, side, image_size,
                                        maps.data_ptr() if maps is not None else None, img.data_ptr(),
                                        rt.stream(s.device))
        rt.check(rc, 'musc_maps_f64')
    return maps, img
