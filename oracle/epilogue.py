"""CPU oracle for the score-map epilogue.  TEST INFRASTRUCTURE ONLY.

`maps_and_scores` restates models/musc.py:247-288: the per-layer MSM maps of
one radius are stacked and averaged (float64 torch.mean over layers, :259), the
per-radius results are averaged again (:263), the (N, P) map is viewed as
(N, 1, side, side) and upsampled with F.interpolate(mode='bilinear',
align_corners=True) (:269-272), and the image score is the maximum of each
upsampled map (:288).

`bilinear_align_corners_f64` is an independent float64 loop over the textbook
definition (source coordinate = dst * (in-1)/(out-1)); it pins the interpolate
call, including the closed form that the four corners equal the grid corners.
"""
from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn.functional as F


def maps_and_scores(scores_rl: list[list[torch.Tensor]], image_size: int) -> tuple[torch.Tensor, torch.Tensor]:
    """scores_rl[r][l]: (N, P) float64 -> maps (N, 1, S, S) float64, image scores (N,)."""
    per_radius = []
    for per_layer in scores_rl:
        stack = torch.stack([s.detach().cpu().double() for s in per_layer], 0)
        per_radius.append(torch.mean(stack, 0))
    avg = torch.mean(torch.stack(per_radius, 0), 0)
    n, p = avg.shape
    side = int(np.sqrt(p))
    maps = F.interpolate(avg.view(n, 1, side, side), size=image_size, mode='bilinear', align_corners=True)
    return maps, maps.reshape(n, -1).max(-1)[0]


def bilinear_align_corners_f64(grid: np.ndarray, out: int) -> np.ndarray:
    grid = np.asarray(grid, dtype=np.float64)
    side = grid.shape[0]
    scale = (side - 1) / (out - 1) if out > 1 else 0.0
    res = np.empty((out, out))
    for y in range(out):
        sy = y * scale
        y0 = min(int(math.floor(sy)), side - 1)
        y1 = min(y0 + 1, side - 1)
        ly = sy - y0
        for x in range(out):
            sx = x * scale
            x0 = min(int(math.floor(sx)), side - 1)
            x1 = min(x0 + 1, side - 1)
            lx = sx - x0
            res[y, x] = ((1 - ly) * ((1 - lx) * grid[y0, x0] + lx * grid[y0, x1])
                         + ly * ((1 - lx) * grid[y1, x0] + lx * grid[y1, x1]))
    return res
