"""MSM on a pool larger than 2 GiB: N = 400 images x 1369 patches x 1024 channels.

The features take 2.24 GB, so 32-bit byte offsets from the start of the pool no longer
reach every row; the pair kernels address each tile's row panels through buffer
resources based at the panels (any pool size), and the rank stage takes its N > 192
path.  The reference tiles any N under its 256 MiB scratch cap
(models/modules/_MSM_gpu.py:11, 731-766).  Checked against the C float64 brute force on
sampled rows and against the oracle's compute_scores_fast (models/modules/_MSM.py:10-30)
run on the device for two whole query images; gate 2e-5 (tools/benchmark_support.py:11).
"""
import numpy as np
import pytest
import torch

import oracle
from musc_hip import _MSM_hip
from oracle import msm as om

pytestmark = pytest.mark.gpu
ATOL = 2e-5
N, P, C = 400, 1369, 1024


@pytest.fixture(scope='module')
def pool(device):
    g = torch.Generator(device=device).manual_seed(400)
    z = torch.randn((N, P, C), generator=g, device=device)
    z = z / z.norm(dim=-1, keepdim=True)
    assert z.numel() * 4 > 2 ** 31
    return z


@pytest.fixture(scope='module')
def reference(pool):
    prev = (torch.backends.cuda.matmul.allow_tf32, torch.get_float32_matmul_precision())
    torch.backends.cuda.matmul.allow_tf32 = False
    torch.set_float32_matmul_precision('highest')
    try:
        a, b = om.rank_window(N)
        rows = np.sort(np.random.default_rng(5).choice(N * P, size=24, replace=False))
        f64 = oracle.msm_row_scores_f64_c(pool.cpu().numpy(), rows, a, b)
        dev = {i: om.compute_scores_fast(pool, i).double().cpu().numpy() for i in (0, N - 1)}
    finally:
        torch.backends.cuda.matmul.allow_tf32 = prev[0]
        torch.set_float32_matmul_precision(prev[1])
    # the device oracle itself against the float64 brute force where their rows meet
    for i, sc in dev.items():
        own = rows[(rows >= i * P) & (rows < (i + 1) * P)]
        for r in own:
            assert abs(sc[r - i * P] - f64[list(rows).index(r)]) <= ATOL
    return rows, f64, dev


@pytest.mark.parametrize('engine', ['fp32', 'split16'])
def test_pool_over_2gib(pool, reference, engine):
    rows, f64, dev = reference
    got = _MSM_hip.MSM(pool, engine=engine)
    assert got.shape == (N, P) and got.dtype == torch.float64
    flat = got.reshape(-1)[torch.as_tensor(rows, device=got.device)].cpu().numpy()
    err = np.abs(flat - f64).max()
    print(f'N={N} {engine}: sampled rows vs float64 brute force {err:.3e}', flush=True)
    assert err <= ATOL
    g = got.cpu().numpy()
    for i, sc in dev.items():
        e = np.abs(g[i] - sc).max()
        print(f'N={N} {engine}: query image {i} vs device oracle {e:.3e}', flush=True)
        assert e <= ATOL
