"""CPU oracle for the mutual scoring module (MSM).  TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg may import
this module, and only as the checker.  The product path (musc_hip) never calls
it and fails loudly when the HIP library is missing.

Two restatements of the reference algorithm live here:

* `compute_scores_fast` / `MSM` restate the reference's original torch-fp32 backend
  line for line in behaviour (models/modules/_MSM.py:10-30 and :53-59): cdist from
  query image i to every other image's patches, min over each reference image's
  patches, two topk calls selecting ascending ranks [k_min, k_max), fp32 mean,
  then float64.  This is the parity target (2e-5 absolute).
* `msm_bruteforce_f64` is an independent float64 brute force written from the
  mathematical definition with explicit differences (no expanded-norm GEMM, no
  topk).  It pins the torch restatement: tests compare the two on seeded inputs,
  on closed forms (identical images give zero scores, one-dimensional offsets give
  |delta_j - delta_i|) and on invariants (permutations, scaling).

The C restatement in msm_f64.c (built into oracle/_build/libmsm_oracle.so) is the
same float64 brute force, fast enough for the full plumbing configuration.
"""
from __future__ import annotations

import numpy as np
import torch


def rank_window(n: int, topmin_min: float = 0, topmin_max: float = 0.3) -> tuple[int, int]:
    """Ranks [k_min, k_max) of the n-1 per-image minima that are averaged.

    Mirrors models/modules/_MSM.py:19-26: fractions below 1 are scaled by the
    number of reference images (n-1) and truncated; the pair is swapped if
    reversed.
    """
    k_max, k_min = topmin_max, topmin_min
    if k_max < 1:
        k_max = int((n - 1) * k_max)
    if k_min < 1:
        k_min = int((n - 1) * k_min)
    if k_max < k_min:
        k_max, k_min = k_min, k_max
    return int(k_min), int(k_max)


def per_image_minima(Z: torch.Tensor, i: int) -> torch.Tensor:
    """(P, N-1) Euclidean minima of query image i against every other image.

    models/modules/_MSM.py:15-17: Z_ref drops image i, cdist against all remaining
    patches, then the minimum over each reference image's P patches.
    """
    n, p, c = Z.shape
    z_ref = torch.cat((Z[:i], Z[i + 1:]), dim=0)
    d = torch.cdist(Z[i:i + 1], z_ref.reshape(-1, c)).reshape(p, n - 1, p)
    return torch.min(d, -1)[0]


def compute_scores_fast(Z: torch.Tensor, i: int, topmin_min: float = 0, topmin_max: float = 0.3) -> torch.Tensor:
    """Scores (P,) fp32 of query image i (models/modules/_MSM.py:10-30)."""
    m = per_image_minima(Z, i)
    k_min, k_max = rank_window(Z.shape[0], topmin_min, topmin_max)
    vals, _ = torch.topk(m.float(), k_max, largest=False, sorted=True)
    vals, _ = torch.topk(vals.float(), k_max - k_min, largest=True, sorted=True)
    return torch.mean(vals.clone(), dim=1)


def MSM(Z: torch.Tensor, topmin_min: float = 0, topmin_max: float = 0.3) -> torch.Tensor:
    """(N, P) float64 scores (models/modules/_MSM.py:53-59), on the CPU."""
    Z = Z.detach().to('cpu', torch.float32).contiguous()
    rows = [compute_scores_fast(Z, i, topmin_min, topmin_max).double() for i in range(Z.shape[0])]
    return torch.stack(rows, 0)


def MSM_device(Z: torch.Tensor, topmin_min: float = 0, topmin_max: float = 0.3) -> torch.Tensor:
    """(N, P) float64 scores, the same restatement evaluated where Z lives.

    For full-size parity checks on the GPU box: compute_scores_fast's torch calls
    (cdist, min, topk, mean) run on Z's device in fp32, one query image at a time.
    Tests pin this device run against the float64 brute force on sampled rows
    (msm_row_scores_f64_c); matmul TF32/reduced-precision modes must be off.
    """
    Z = Z.detach().float().contiguous()
    return torch.stack([compute_scores_fast(Z, i, topmin_min, topmin_max).double()
                        for i in range(Z.shape[0])], 0)


def nearest(Z: torch.Tensor) -> torch.Tensor:
    """(N*P, N) fp32 per-reference-image minima with +inf on the own image."""
    Z = Z.detach().to('cpu', torch.float32).contiguous()
    n, p, _ = Z.shape
    out = torch.full((n * p, n), float('inf'), dtype=torch.float32)
    for i in range(n):
        m = per_image_minima(Z, i)
        others = [j for j in range(n) if j != i]
        out[i * p:(i + 1) * p, others] = m
    return out


# ---------------------------------------------------------------------------
# Independent float64 brute force (pins the restatement above).
# ---------------------------------------------------------------------------
def nearest_bruteforce_f64(Z: np.ndarray) -> np.ndarray:
    """(N*P, N) float64 minima from explicit differences; +inf on the own image."""
    Z = np.asarray(Z, dtype=np.float64)
    n, p, _ = Z.shape
    out = np.full((n * p, n), np.inf)
    for i in range(n):
        for j in range(n):
            if j == i:
                continue
            diff = Z[i][:, None, :] - Z[j][None, :, :]          # (P, P, C)
            out[i * p:(i + 1) * p, j] = np.sqrt((diff * diff).sum(-1)).min(1)
    return out


def scores_from_nearest_f64(nearest_np: np.ndarray, n: int, p: int, k_min: int, k_max: int) -> np.ndarray:
    """Mean of ascending ranks [k_min, k_max) of each row's n-1 finite minima."""
    out = np.empty(n * p)
    for row in range(n * p):
        vals = np.sort(np.delete(nearest_np[row], row // p))
        out[row] = vals[k_min:k_max].mean()
    return out.reshape(n, p)


def msm_bruteforce_f64(Z: np.ndarray, topmin_min: float = 0, topmin_max: float = 0.3) -> np.ndarray:
    n, p, _ = np.shape(Z)
    k_min, k_max = rank_window(n, topmin_min, topmin_max)
    return scores_from_nearest_f64(nearest_bruteforce_f64(Z), n, p, k_min, k_max)
