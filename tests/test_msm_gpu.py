"""MSM parity on the GPU: libmusc_hip vs the oracle (2e-5 absolute, the reference's gate)."""
import numpy as np
import pytest
import torch

import oracle
from oracle import msm as om
from musc_hip import _MSM_hip
from musc_hip import synthetic

pytestmark = pytest.mark.gpu
ATOL = 2e-5  # tools/benchmark_support.py:11


def _gpu(x, device):
    return torch.as_tensor(x).to(device)


@pytest.mark.parametrize('case', ['a', 'b', 'c', 'd'])
def test_golden(golden, device, case):
    g = golden('msm_small.npz')
    z = _gpu(g[f'{case}_z'], device)
    scores = _MSM_hip.MSM(z).cpu().numpy()
    np.testing.assert_allclose(scores, g[f'{case}_scores'], rtol=0, atol=ATOL)
    near = _MSM_hip.nearest(z).cpu().numpy()
    np.testing.assert_allclose(near, g[f'{case}_nearest'], rtol=0, atol=ATOL)


# p >= 128 takes the two-segment register epilogue for tiles straddling an image boundary
# (p = 128: every tile inside one image; 129/130/200/257/300/1369: straddling tiles, padded
# last tile row); p < 128 the LDS epilogue (several images per tile); c % 4 != 0 the masked loads;
# c % 64 != 0 (36, 100, 7, 33, 4, 96, 32) the channel-masked loads, with an odd number of 32-channel
# chunks rounded up by a zero chunk (7, 33, 4, 96, 32); c % 64 == 0 the unmasked whole-chunk loads,
# with the register epilogues (1024, 64 at p >= 128) and with the LDS epilogue (128, 64 at p < 128)
@pytest.mark.parametrize('n,p,c', [(5, 200, 36), (9, 130, 1024), (17, 64, 100), (6, 129, 7), (12, 257, 33),
                                   (40, 3, 4), (7, 128, 64), (5, 300, 1024), (5, 1369, 64), (8, 150, 96),
                                   (6, 140, 32), (30, 60, 128), (12, 100, 64)])
def test_random_shapes_vs_oracles(device, n, p, c):
    torch.manual_seed(n * 1000 + p)
    z = torch.nn.functional.normalize(torch.randn((n, p, c)), dim=-1)
    got = _MSM_hip.MSM(z.to(device)).cpu().numpy()
    ref_t = om.MSM(z).numpy()
    ref_64 = oracle.msm_scores_f64_c(z.numpy(), *om.rank_window(n))
    np.testing.assert_allclose(got, ref_t, rtol=0, atol=ATOL)
    np.testing.assert_allclose(got, ref_64, rtol=0, atol=ATOL)


@pytest.mark.parametrize('n,p,c', [(2, 1, 1), (2, 5, 3), (3, 1, 17), (4, 2, 5), (2, 130, 8)])
def test_minimal_shapes(device, n, p, c):
    # smallest pools (N = 2 needs topmin_max = 1 for a nonempty window), one patch per
    # image, one channel; inputs spread out so no pair is within fp32 cancellation range
    g = torch.Generator().manual_seed(n * 100 + p * 10 + c)
    if c == 1:
        z = torch.linspace(-1.0, 1.0, n * p)[torch.randperm(n * p, generator=g)].reshape(n, p, 1)
    else:
        z = torch.nn.functional.normalize(torch.randn((n, p, c), generator=g), dim=-1)
    got = _MSM_hip.MSM(z.to(device), topmin_min=0, topmin_max=1.0).cpu().numpy()
    ref = oracle.msm_scores_f64_c(z.numpy(), *om.rank_window(n, 0, 1.0))
    np.testing.assert_allclose(got, ref, rtol=0, atol=ATOL)


def test_closed_form_one_dimensional_offsets(device):
    # Z[j] = base + delta_j * u: every patch's nearest patch in image j is the same patch,
    # at |delta_j - delta_i|, so the scores are interval means of sorted |delta_j - delta_i|
    rng = np.random.default_rng(14)
    n, p, c = 11, 150, 64
    base = rng.standard_normal((p, c))
    base /= np.linalg.norm(base, axis=1, keepdims=True)
    u = rng.standard_normal(c)
    u /= np.linalg.norm(u)
    # offsets at least 0.04 apart: the expanded form's ~1e-7 error in d^2 then stays far
    # below the gate in d (it is not a property of the closed form but of fp32 cdist)
    delta = rng.permutation((np.arange(n) + 0.5 * rng.random(n)) * 0.045)
    z = (base[None] + delta[:, None, None] * u[None, None]).astype(np.float32)
    got = _MSM_hip.MSM(torch.from_numpy(z).to(device)).cpu().numpy()
    k_min, k_max = om.rank_window(n)
    for i in range(n):
        d = np.sort([abs(delta[j] - delta[i]) for j in range(n) if j != i])
        np.testing.assert_allclose(got[i], d[k_min:k_max].mean(), rtol=0, atol=ATOL, err_msg=f'image {i}')


def test_rank_windows(device):
    torch.manual_seed(3)
    z = torch.randn((21, 50, 24))
    for lo, hi in ((0.1, 0.5), (0, 1), (0.5, 0.2), (2, 5), (0, 20)):
        got = _MSM_hip.MSM(z.to(device), topmin_min=lo, topmin_max=hi).cpu().numpy()
        ref = om.MSM(z, lo, hi).numpy()
        np.testing.assert_allclose(got, ref, rtol=0, atol=ATOL, err_msg=f'window {lo},{hi}')


def test_nearest_vs_oracle(device):
    torch.manual_seed(4)
    z = torch.nn.functional.normalize(torch.randn((7, 300, 64)), dim=-1)
    got = _MSM_hip.nearest(z.to(device)).cpu().numpy()
    ref = om.nearest(z).numpy()
    assert np.isinf(got[np.isinf(ref)]).all()
    fin = np.isfinite(ref)
    np.testing.assert_allclose(got[fin], ref[fin], rtol=0, atol=ATOL)


def test_config1_plumbing_kernel_level(device):
    # BASELINE config 1 shape: N=8, P=1369, C=1024, seeded N(0,1), L2-normalised
    z = synthetic.msm_features(8, 1369, 1024, seed=42)
    got = _MSM_hip.MSM(z.to(device)).cpu().numpy()
    ref = om.MSM(z).numpy()
    err = np.abs(got - ref).max()
    print(f'config1 kernel-level max abs err {err:.3e}', flush=True)
    assert err <= ATOL


def test_default_pool_sampled_queries(device):
    # BASELINE config 2 shape (N=83, P=1369, C=1024, correlated features); the oracle
    # restates compute_scores_fast per query image, so three query images are checked.
    toks = synthetic.pool_tokens(83, layers=1, seed=42)[0]
    z = toks[:, 1:, :].contiguous()
    got = _MSM_hip.MSM(z.to(device)).cpu().numpy()
    for i in (0, 41, 82):
        ref = om.compute_scores_fast(z, i).double().numpy()
        err = np.abs(got[i] - ref).max()
        print(f'config2 query image {i}: max abs err {err:.3e}', flush=True)
        assert err <= ATOL


def test_full_size_properties(device):
    # BASELINE config 3 shape (N=83, P=784): deterministic, permutation-equivariant, scale-equivariant
    z = synthetic.msm_features(83, 784, 1024, seed=7).to(device)
    a = _MSM_hip.MSM(z)
    b = _MSM_hip.MSM(z)
    assert torch.equal(a, b), 'MSM must be bitwise deterministic'
    perm = torch.randperm(83, generator=torch.Generator().manual_seed(1)).to(device)
    c = _MSM_hip.MSM(z[perm].contiguous())
    assert (c - a[perm]).abs().max().item() <= 1e-6
    pp = torch.randperm(784, generator=torch.Generator().manual_seed(2)).to(device)
    d = _MSM_hip.MSM(z[:, pp].contiguous())
    assert (d - a[:, pp]).abs().max().item() <= 1e-6
    e = _MSM_hip.MSM(z * 2.0)
    assert (e - 2.0 * a).abs().max().item() <= 4e-6
    # sampled oracle check of two query images at this shape
    zc = z.cpu()
    for i in (5, 77):
        ref = om.compute_scores_fast(zc, i).double().numpy()
        assert np.abs(a[i].cpu().numpy() - ref).max() <= ATOL


def test_identical_images_score_near_zero(device):
    base = torch.nn.functional.normalize(torch.randn((1, 64, 32)), dim=-1)
    z = base.repeat(6, 1, 1).to(device)
    got = _MSM_hip.MSM(z).cpu().numpy()
    # exact answer 0: the expanded form ||a||^2 + ||b||^2 - 2 a.b would leave the square
    # root of a few fp32 ulps of ||a||^2 + ||b||^2 (as torch.cdist's matmul path does);
    # the refinement recomputes those minima by explicit differences
    assert np.all(got == 0.0), got.max()


def test_input_validation(device):
    with pytest.raises(ValueError, match='nonempty trimmed ranks'):
        _MSM_hip.MSM(torch.randn((4, 10, 8), device=device))
    with pytest.raises(ValueError, match='CUDA FP32'):
        _MSM_hip.MSM(torch.randn((8, 10, 8), device=device, dtype=torch.float64))
    with pytest.raises(ValueError):
        _MSM_hip.MSM(torch.randn((1, 10, 8), device=device))


def test_normalize_rows_equals_normalised_input(device):
    torch.manual_seed(12)
    z = torch.randn((11, 150, 96)) * 3.0 + 0.7
    got = _MSM_hip.MSM(z.to(device), normalize_rows=True).cpu().numpy()
    ref = om.MSM(torch.nn.functional.normalize(z, dim=-1)).numpy()
    np.testing.assert_allclose(got, ref, rtol=0, atol=ATOL)
    # without the flag the scores are those of the raw rows
    raw = _MSM_hip.MSM(z.to(device)).cpu().numpy()
    np.testing.assert_allclose(raw, om.MSM(z).numpy(), rtol=0, atol=1e-4)


@pytest.mark.parametrize('n', [2, 3, 31, 32, 33, 64, 65, 96, 97, 128, 129, 160, 161, 192, 193, 200, 256, 257,
                               513, 1025])
def test_rank_selection_across_register_sizes(device, n):
    # the rank kernels keep a row's n minima in registers: one lane per row for n <= 192
    # (instantiations of 32/64/96/128/160/192 keys), one wave per row beyond (4/8/16/32 slots
    # per lane up to 256/512/1024/2048 images); every boundary, windows starting above 0, and
    # ties.  Small-integer features make every norm and dot product
    # exact in fp32, so both sides see the same squared distances (integers) and ties are
    # exact: many equal minima, and image 1 duplicates image 0 (zero distances).
    g = torch.Generator().manual_seed(n)
    z = torch.randint(-2, 3, (n, 5, 12), generator=g).float()
    if n >= 3:
        z[1] = z[0]
    zd = z.to(device)
    windows = [(0, 0.3), (0, 1.0 - 1e-9), (0.1, 0.3)] if n >= 11 else [(0, n - 1)]
    for lo, hi in windows:
        a, b = om.rank_window(n, lo, hi)
        if not 0 <= a < b <= n - 1:
            continue
        got = _MSM_hip.MSM(zd, topmin_min=lo, topmin_max=hi).cpu().numpy()
        ref = om.MSM(z, lo, hi).numpy()
        err = np.abs(got - ref).max()
        assert err <= ATOL, (n, lo, hi, err)
