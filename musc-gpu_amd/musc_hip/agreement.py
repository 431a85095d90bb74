"""Agreement gate between a reference result and a candidate result.

Same contract as the reference benchmark's gate (tools/benchmark_support.py:11,72-98),
which voids a speed claim unless the accelerated run reproduces the original
backend's maps and scores (tools/benchmark.py:318-334):

  * empty arrays fail ("cannot establish agreement");
  * a shape mismatch fails;
  * any non-finite value, in either array, fails;
  * otherwise the arrays agree when max |reference - candidate| <= 2e-5 (ATOL).

The comparison runs in float64 over chunks of `chunk_images` leading rows, so that
memory-mapped full-pool maps need not be loaded at once; two torch tensors on one GPU
are compared there, in one piece (same tests, same keys).  The returned dict carries
the same keys as the reference's (pass, shape_match, finite, max_absolute_error,
max_relative_error_reference_floor_1e_12, rmse, absolute_tolerance, dtypes).
"""
from __future__ import annotations

import math

import numpy as np

ATOL = 2e-5


def _numpy(x) -> np.ndarray:
    if hasattr(x, 'detach'):  # torch tensor, any device
        x = x.detach().cpu().numpy()
    return np.asarray(x)


def _compare_on_device(ref, cand) -> dict:
    """compare_arrays for two torch tensors on one GPU: the same tests, evaluated there."""
    import torch
    a, b = ref.detach().to(torch.float64), cand.detach().to(torch.float64)
    finite = bool(torch.isfinite(a).all().item() and torch.isfinite(b).all().item())
    out = {'shape_match': True, 'finite': finite, 'absolute_tolerance': ATOL,
           'reference_dtype': str(ref.dtype), 'candidate_dtype': str(cand.dtype)}
    if not finite:
        # the reference skips non-finite chunks; with one chunk per call nothing is left
        out.update({'pass': False, 'max_absolute_error': None,
                    'max_relative_error_reference_floor_1e_12': None, 'rmse': None})
        return out
    d = (a - b).abs()
    worst = float(d.max().item())
    out.update({'pass': worst <= ATOL, 'max_absolute_error': worst,
                'max_relative_error_reference_floor_1e_12': float((d / a.abs().clamp_min(1e-12)).max().item()),
                'rmse': float(d.square().mean().sqrt().item())})
    return out


def compare_arrays(reference, candidate, chunk_images: int = 4) -> dict:
    if (hasattr(reference, 'is_cuda') and hasattr(candidate, 'is_cuda') and reference.is_cuda
            and candidate.is_cuda and reference.device == candidate.device
            and reference.numel() and candidate.numel() and reference.shape == candidate.shape):
        return _compare_on_device(reference, candidate)
    ref, cand = _numpy(reference), _numpy(candidate)
    if ref.size == 0 or cand.size == 0:
        return {'pass': False, 'error': 'Empty predictions cannot establish agreement'}
    if ref.shape != cand.shape:
        return {'pass': False, 'shape_match': False, 'reference_shape': list(ref.shape),
                'candidate_shape': list(cand.shape)}
    worst_abs = worst_rel = 0.0
    sq_sum, count = 0.0, 0
    finite = True
    rows = ref.shape[0] if ref.ndim else 1
    ref2 = ref.reshape(rows, -1)
    cand2 = cand.reshape(rows, -1)
    for start in range(0, rows, chunk_images):
        a = ref2[start:start + chunk_images].astype(np.float64)
        b = cand2[start:start + chunk_images].astype(np.float64)
        if not (np.isfinite(a).all() and np.isfinite(b).all()):
            finite = False
            continue
        if a.size:
            d = np.abs(a - b)
            worst_abs = max(worst_abs, float(d.max()))
            worst_rel = max(worst_rel, float((d / np.maximum(np.abs(a), 1e-12)).max()))
            sq_sum += float(np.square(d).sum())
            count += d.size
    return {'pass': bool(finite and worst_abs <= ATOL), 'shape_match': True, 'finite': finite,
            'max_absolute_error': worst_abs if finite else None,
            'max_relative_error_reference_floor_1e_12': worst_rel if finite else None,
            'rmse': math.sqrt(sq_sum / count) if finite and count else None,
            'absolute_tolerance': ATOL, 'reference_dtype': str(ref.dtype), 'candidate_dtype': str(cand.dtype)}


def nan_aware_match(reference, candidate, atol: float = ATOL) -> dict:
    """For inputs whose reference result legitimately holds NaN (zero-norm or non-finite
    features): the NaN positions must coincide exactly, the +-inf positions and signs
    too, and the remaining finite values must agree within `atol`."""
    ref, cand = _numpy(reference).astype(np.float64), _numpy(candidate).astype(np.float64)
    if ref.shape != cand.shape:
        return {'pass': False, 'shape_match': False}
    nan_r, nan_c = np.isnan(ref), np.isnan(cand)
    inf_ok = bool(np.array_equal(np.isposinf(ref), np.isposinf(cand))
                  and np.array_equal(np.isneginf(ref), np.isneginf(cand)))
    fin = np.isfinite(ref) & np.isfinite(cand)
    err = float(np.abs(ref[fin] - cand[fin]).max()) if fin.any() else 0.0
    same_nan = bool(np.array_equal(nan_r, nan_c))
    return {'pass': same_nan and inf_ok and err <= atol, 'nan_positions_equal': same_nan,
            'inf_positions_equal': inf_ok, 'reference_nan': int(nan_r.sum()), 'candidate_nan': int(nan_c.sum()),
            'max_absolute_error_finite': err}
