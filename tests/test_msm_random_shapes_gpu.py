"""MSM over seeded random shapes, both engines, against the C float64 brute force.

The hand-picked shape lists of test_msm_gpu.py cover the kernels' branches one by one;
this sweep draws pools of 2-12 images, 1-300 patches and 1-160 channels (channel counts
that are and are not multiples of the 16-channel stage, of 4, odd ones), with and without
row normalisation, random rank windows and, in some pools, a duplicated image (exact
zero minima through the cancellation refinement), and checks every score row against
the float64 brute force over the definition (models/modules/_MSM.py:10-30) at the
reference's 2e-5 gate (tools/benchmark_support.py:11).  The split engine runs where it
is defined (P >= 256) and must raise ValueError elsewhere, as its contract says.
Features are drawn at the scale the scoring sees them (unit-norm rows, or rows of norm
~1-3 when not normalised), where fp32 distances carry ~1e-7 relative error.
"""
import numpy as np
import pytest
import torch

import oracle
from musc_hip import _MSM_hip
from oracle import msm as om

pytestmark = pytest.mark.gpu
ATOL = 2e-5


def _case(k):
    rng = np.random.default_rng(1000 + k)
    n = int(rng.integers(2, 13))
    p = int(rng.choice([1, 2, 7, 37, 64, 100, 127, 128, 129, 200, 256, 257, 300]))
    c = int(rng.choice([1, 3, 4, 15, 16, 17, 31, 32, 33, 64, 96, 100, 128, 160]))
    normalize = bool(rng.integers(0, 2))
    a = int(rng.integers(0, n - 1))
    b = int(rng.integers(a + 1, n))
    dup = n >= 3 and rng.random() < 0.4
    if dup and rng.random() < 0.5:
        a, b = 0, 1
    z = rng.standard_normal((n, p, c)).astype(np.float32) + rng.standard_normal(c).astype(np.float32)
    z /= np.sqrt(np.float32(c))
    if not normalize:
        z *= np.float32(rng.uniform(0.5, 2.0))
    if dup:
        z[n - 1] = z[0]
    return n, p, c, normalize, a, b, dup, z


@pytest.mark.parametrize('k', range(40))
def test_random_pool_against_float64(device, k):
    n, p, c, normalize, a, b, dup, z = _case(k)
    zt = torch.from_numpy(z)
    ref_in = (zt / zt.norm(dim=-1, keepdim=True)).numpy() if normalize else z
    # ranks given as counts (>= 1) or 0, so that every window is valid for every n
    lo, hi = (a if a >= 1 else 0), b
    ra, rb = om.rank_window(n, lo, hi)
    assert (ra, rb) == (a, b)
    ref = oracle.msm_row_scores_f64_c(ref_in, np.arange(n * p), a, b).reshape(n, p)
    engines = ['fp32'] + (['split16'] if p >= 256 else [])
    for engine in engines:
        got = _MSM_hip.MSM(zt.to(device), topmin_min=lo, topmin_max=hi, normalize_rows=normalize,
                           engine=engine).cpu().numpy()
        err = np.abs(got - ref).max()
        print(f'case {k}: n={n} p={p} c={c} normalize={normalize} ranks=[{a},{b}) dup={dup} '
              f'{engine}: {err:.2e}', flush=True)
        assert np.isfinite(got).all() and err <= ATOL
        if dup and (a, b) == (0, 1):
            # the first and last images are identical: each one's smallest minimum is
            # exactly 0, and the window holds only it
            assert np.all(got[0] == 0.0) and np.all(got[n - 1] == 0.0)
    if p < 256:
        with pytest.raises(ValueError):
            _MSM_hip.MSM(zt.to(device), topmin_min=lo, topmin_max=hi, normalize_rows=normalize, engine='split16')
