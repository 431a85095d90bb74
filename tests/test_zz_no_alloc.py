"""musc_msm_scores_f32_noalloc (the workspace in the library's per-GPU scratch array)
against musc_msm_scores_f32 (workspace from the caller), through the C-ABI.

Two calls in a row, the second on a smaller pool, so the second call runs on scratch
the first one left behind; then a pool too large for the scratch is rejected.  The
two entry points run the same kernels, so the scores must be bit-identical (and
within the 2e-5 gate of the oracle's restatement, which the workspace entry point
meets in test_msm_gpu.py).
"""
import ctypes

import pytest
import torch

from musc_hip import _MSM_hip, synthetic
from musc_hip import _runtime as rt

pytestmark = pytest.mark.gpu


def _with_workspace(z, a, b):
    n, p, c = z.shape
    ws = rt.workspace(_MSM_hip.workspace_bytes(n, p, c), z.device)
    out = torch.empty((n, p), dtype=torch.float64, device=z.device)
    rc = rt.library().musc_msm_scores_f32(z.data_ptr(), n, p, c, a, b, out.data_ptr(), ws.data_ptr(), ws.numel(),
                                          rt.stream(z.device))
    rt.check(rc, 'musc_msm_scores_f32')
    return out


def _no_alloc(z, a, b):
    n, p, c = z.shape
    out = torch.full((n, p), float('nan'), dtype=torch.float64, device=z.device)
    rc = rt.library().musc_msm_scores_f32_noalloc(z.data_ptr(), n, p, c, a, b, out.data_ptr(),
                                                  rt.stream(z.device))
    rt.check(rc, 'musc_msm_scores_f32_noalloc')
    return out


def test_no_alloc_matches_the_workspace_entry_point(device):
    # call 1: config 5's pool shape (N = 160, P = 1369, C = 1024: 136 MiB of workspace);
    # call 2: a smaller pool (stale keys of call 1 lie beyond its minima)
    for (n, p, c), seed in (((160, 1369, 1024), 42), ((20, 300, 256), 7)):
        z = synthetic.msm_features(n, p, c, seed=seed).to(device)
        a, b = _MSM_hip.rank_window(n)
        got = _no_alloc(z, a, b)
        ref = _with_workspace(z, a, b)
        torch.cuda.synchronize()
        err = (got - ref).abs().max().item()
        print(f'no-alloc vs workspace entry point, N={n} P={p} C={c}: max abs diff {err:.3e}', flush=True)
        assert torch.equal(got, ref)


def test_no_alloc_rejects_pools_beyond_the_scratch(device):
    assert rt.library().musc_target_arch() == b'gfx950'
    limit = 256 << 20
    n, p, c = 600, 200, 4            # n * p * n * 4 bytes of minima keys = 288 MB > 256 MiB
    assert _MSM_hip.workspace_bytes(n, p, c) > limit
    z = torch.zeros((n, p, c), device=device)
    out = torch.zeros((n, p), dtype=torch.float64, device=device)
    rc = rt.library().musc_msm_scores_f32_noalloc(z.data_ptr(), n, p, c, 0, 179, out.data_ptr(), rt.stream(device))
    assert rc == rt.MUSC_ERR_SCRATCH_LIMIT
    assert b'no-allocation scratch' in rt.library().musc_strerror(rc)
    assert (out == 0).all()          # nothing was launched
    with pytest.raises(RuntimeError, match='no-allocation scratch'):
        rt.check(rc, 'musc_msm_scores_f32_noalloc')
