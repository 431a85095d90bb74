"""Split MSM engine (fp32 dot products from three fp16 MFMA products) vs the oracle.

Same gate as the fp32 engine: 2e-5 absolute on scores (tools/benchmark_support.py:11).
The per-(patch, image) minima are also checked directly against the float64 brute force.
"""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from oracle import msm as om
from musc_hip import _MSM_hip, pipeline, synthetic
from musc_hip import _runtime as rt

pytestmark = pytest.mark.gpu
ATOL = 2e-5  # tools/benchmark_support.py:11


def _split(z, **kw):
    return _MSM_hip.MSM(z, engine='split16', **kw)


# p = 256: tiles aligned with images; 257/300/400/1369: tiles straddling an image boundary
# (two-segment epilogue) and a padded last tile row; c % 32 != 0: zero-padded channel blocks
@pytest.mark.parametrize('n,p,c', [(5, 256, 64), (5, 257, 33), (6, 300, 1024), (5, 1369, 100), (9, 400, 7),
                                   (7, 512, 32)])
def test_random_shapes_vs_oracles(device, n, p, c):
    torch.manual_seed(n * 1000 + p)
    z = torch.nn.functional.normalize(torch.randn((n, p, c)), dim=-1)
    got = _split(z.to(device)).cpu().numpy()
    ref_t = om.MSM(z).numpy()
    ref_64 = oracle.msm_scores_f64_c(z.numpy(), *om.rank_window(n))
    np.testing.assert_allclose(got, ref_t, rtol=0, atol=ATOL)
    np.testing.assert_allclose(got, ref_64, rtol=0, atol=ATOL)


def test_two_image_pool(device):
    # N = 2 (window [0, 1) with topmin_max = 1): every patch's score is its distance to the
    # nearest patch of the other image
    torch.manual_seed(5)
    z = torch.nn.functional.normalize(torch.randn((2, 300, 48)), dim=-1)
    got = _split(z.to(device), topmin_min=0, topmin_max=1.0).cpu().numpy()
    ref = oracle.msm_scores_f64_c(z.numpy(), *om.rank_window(2, 0, 1.0))
    np.testing.assert_allclose(got, ref, rtol=0, atol=ATOL)


def test_closed_form_one_dimensional_offsets(device):
    # Z[j] = base + delta_j * u (unnormalised rows): the nearest patch in image j is the
    # same patch, at |delta_j - delta_i|
    rng = np.random.default_rng(15)
    n, p, c = 9, 260, 64
    base = rng.standard_normal((p, c))
    base /= np.linalg.norm(base, axis=1, keepdims=True)
    u = rng.standard_normal(c)
    u /= np.linalg.norm(u)
    # offsets at least 0.04 apart: the expanded form's ~1e-7 error in d^2 then stays far
    # below the gate in d (it is not a property of the closed form but of fp32 cdist)
    delta = rng.permutation((np.arange(n) + 0.5 * rng.random(n)) * 0.045)
    z = (base[None] + delta[:, None, None] * u[None, None]).astype(np.float32)
    got = _split(torch.from_numpy(z).to(device)).cpu().numpy()
    k_min, k_max = om.rank_window(n)
    for i in range(n):
        d = np.sort([abs(delta[j] - delta[i]) for j in range(n) if j != i])
        np.testing.assert_allclose(got[i], d[k_min:k_max].mean(), rtol=0, atol=ATOL, err_msg=f'image {i}')


def _split_minima(z: torch.Tensor, normalize: bool) -> np.ndarray:
    """Squared per-(row, image) minima left by the split pair kernel in its workspace."""
    n, p, c = z.shape
    lib = rt.library()
    ws = rt.workspace(_MSM_hip.workspace_bytes(n, p, c, 'split16'), z.device)
    s = rt.stream(z.device)
    flags = rt.MSM_NORMALIZE_ROWS if normalize else 0
    rt.check(lib.musc_msm_split_prepare_f32(z.data_ptr(), n, p, c, flags, ws.data_ptr(), ws.numel(), s), 'prepare')
    rt.check(lib.musc_msm_split_pair_minima(n, p, c, ws.data_ptr(), ws.numel(), s), 'pairs')
    torch.cuda.synchronize()
    rows = n * p
    off = 2 * ((rows * 4 + 255) // 256 * 256)
    keys = ws[off:off + rows * n * 4].view(torch.int32).cpu().numpy().view(np.uint32)
    # the buffer holds min keys: key - 1 is the squared minimum's bits (0xffffffff: NaN)
    return (keys - np.uint32(1)).view(np.float32).reshape(rows, n)


def test_minima_vs_f64_bruteforce(device):
    torch.manual_seed(21)
    z = torch.nn.functional.normalize(torch.randn((5, 300, 96)), dim=-1)
    got = _split_minima(z.to(device), normalize=False)
    ref = oracle.msm_nearest_f64_c(z.numpy()) ** 2
    fin = np.isfinite(ref)
    assert np.isinf(got[~fin]).all(), 'own-image entries must stay +inf'
    # squared distances of unit vectors: fp32-level agreement (|d^2| <= 4)
    np.testing.assert_allclose(got[fin], ref[fin], rtol=0, atol=2e-6)


# Image boundaries at many offsets inside the 256 x 256 tiles: a pool of n images of p
# rows puts boundaries at k p (k = 1 .. n-1), i.e. at offsets k p mod 256 within a tile.
# p = 264 gives offsets on 8-row group edges; 261 and 269 offsets inside groups, in both
# lane halves (rows lh*4 + e); 383 and 385 offsets next to the 128-row wave edge and the
# 64-row half edge; 300 and 449 mixed.  The straddling tiles are reduced per image segment
# in 64-row halves; every per-(row, image) minimum is checked, so a distance credited to
# the wrong segment shows.  With the rows normalised in the kernel (rows of unequal norms
# in, unit rows scored) the waves take the unit-row reduction, whose variants differ by
# where the boundaries cross the wave; without, the general one.
@pytest.mark.parametrize('normalize', [False, True])
@pytest.mark.parametrize('p', [261, 264, 269, 300, 383, 385, 449])
def test_minima_at_boundary_offsets_vs_f64_bruteforce(device, p, normalize):
    n = 8
    torch.manual_seed(p)
    z = torch.randn((n, p, 48)) + 0.3 * torch.randn((1, 1, 48))
    if normalize:
        z = z * (0.5 + torch.rand((n, p, 1)))
        z64 = z.double().numpy()
        ref_in = (z64 / np.linalg.norm(z64, axis=-1, keepdims=True)).astype(np.float32)
    else:
        z = torch.nn.functional.normalize(z, dim=-1)
        ref_in = z.numpy()
    offs = sorted({(k * p) % 256 for k in range(1, n)})
    got = _split_minima(z.to(device), normalize=normalize)
    ref = oracle.msm_nearest_f64_c(ref_in) ** 2
    fin = np.isfinite(ref)
    print(f'p={p} normalize={normalize}: boundary offsets {offs}', flush=True)
    assert np.isinf(got[~fin]).all(), 'own-image entries must stay +inf'
    np.testing.assert_allclose(got[fin], ref[fin], rtol=0, atol=2e-6)


# The hi/lo split exactly as written -- hi = fp16(fp32(v)), lo = fp16(fp32(v - hi)), v =
# x * 2^10 / ||row|| in fp64, each narrowing rounded to nearest even -- on the prepare
# kernel's three paths (a row in registers: c a multiple of 32 up to 1024; eight channels
# per lane; one), zero padding included.  Integer-valued rows make the fp64 sum of squares
# exact in any order, so the restatement's scale is the kernel's bit for bit; a compiler
# that folds the two narrowing steps into one rounding, or fuses x * scale into the
# subtraction, changes some of these bits.
@pytest.mark.parametrize('c', [1024, 96, 1000, 37])
def test_split_array_rounding_as_written(device, c):
    n, p = 2, 260
    rng = np.random.default_rng(c)
    z = rng.integers(-60, 61, size=(n, p, c)).astype(np.float32)
    z *= np.exp2(rng.integers(-6, 7, size=(n, p, 1))).astype(np.float32)  # exact: powers of two
    zt = torch.from_numpy(z).to(device)
    ws = rt.workspace(_MSM_hip.workspace_bytes(n, p, c, 'split16'), device)
    ws.zero_()
    lib = rt.library()
    rt.check(lib.musc_msm_split_prepare_f32(zt.data_ptr(), n, p, c, 0, ws.data_ptr(), ws.numel(), rt.stream(device)),
             'prepare')
    torch.cuda.synchronize()
    rows, nkb = n * p, (c + 31) // 32 * 2
    hl_bytes = rows * nkb * 64
    off = ws.numel() - (hl_bytes + 255) // 256 * 256
    got = ws[off:off + hl_bytes].cpu().numpy().view(np.uint16).reshape(rows, nkb, 2, 16)
    x = np.zeros((rows, nkb * 16))
    x[:, :c] = z.reshape(rows, c).astype(np.float64)
    acc = (x * x).sum(axis=1)  # exact: integers below 2^53 times powers of four
    sc = np.ldexp(1.0 / np.sqrt(acc), 10)
    v = x * sc[:, None]
    hi = v.astype(np.float32).astype(np.float16)
    lo = (v - hi.astype(np.float64)).astype(np.float32).astype(np.float16)
    want = np.stack([hi.reshape(rows, nkb, 16), lo.reshape(rows, nkb, 16)], axis=2).view(np.uint16)
    bad = np.argwhere(got != want)
    assert len(bad) == 0, f'{len(bad)} of {got.size} split values differ, first (row, block, hi/lo, k) {bad[:4].tolist()}'


def test_config1_plumbing_kernel_level(device):
    z = synthetic.msm_features(8, 1369, 1024, seed=42)
    zd = z.to(device)
    got = _split(zd).cpu().numpy()
    fp32 = _MSM_hip.MSM(zd).cpu().numpy()
    ref = om.MSM(z).numpy()
    err, diff = np.abs(got - ref).max(), np.abs(got - fp32).max()
    print(f'config1 split engine: max abs err vs oracle {err:.3e}, vs fp32 engine {diff:.3e}', flush=True)
    assert err <= ATOL


def test_default_pool_sampled_queries(device):
    toks = synthetic.pool_tokens(83, layers=1, seed=42)[0]
    z = toks[:, 1:, :].contiguous()
    got = _split(z.to(device)).cpu().numpy()
    for i in (0, 41, 82):
        ref = om.compute_scores_fast(z, i).double().numpy()
        err = np.abs(got[i] - ref).max()
        print(f'config2 split engine, query image {i}: max abs err {err:.3e}', flush=True)
        assert err <= ATOL


def test_super_fast_shape_deterministic_and_sampled(device):
    z = synthetic.msm_features(83, 784, 1024, seed=7).to(device)
    a = _split(z)
    b = _split(z)
    assert torch.equal(a, b), 'split engine must be bitwise deterministic'
    perm = torch.randperm(83, generator=torch.Generator().manual_seed(1)).to(device)
    c = _split(z[perm].contiguous())
    assert (c - a[perm]).abs().max().item() <= 1e-6
    zc = z.cpu()
    for i in (5, 77):
        ref = om.compute_scores_fast(zc, i).double().numpy()
        assert np.abs(a[i].cpu().numpy() - ref).max() <= ATOL


def test_normalize_rows_and_raw_rows(device):
    torch.manual_seed(12)
    z = torch.randn((7, 260, 96)) * 3.0 + 0.7
    got = _split(z.to(device), normalize_rows=True).cpu().numpy()
    ref = om.MSM(torch.nn.functional.normalize(z, dim=-1)).numpy()
    np.testing.assert_allclose(got, ref, rtol=0, atol=ATOL)
    # unnormalised rows: the per-row scale carries ||z|| (distances here are ~30)
    raw = _split(z.to(device)).cpu().numpy()
    np.testing.assert_allclose(raw, om.MSM(z).numpy(), rtol=0, atol=1e-4)


def test_identical_images_score_near_zero(device):
    base = torch.nn.functional.normalize(torch.randn((1, 256, 32)), dim=-1)
    got = _split(base.repeat(6, 1, 1).to(device)).cpu().numpy()
    assert got.max() < 1e-3


def test_pipeline_engine_matches_fp32_engine(device):
    toks = [t.to(device) for t in synthetic.pool_tokens(8, layers=2, seed=5)]
    m32, i32 = pipeline.score_pool(toks, r_list=[1, 3], image_size=64)
    m16, i16 = pipeline.score_pool(toks, r_list=[1, 3], image_size=64, msm_engine='split16')
    assert (m16 - m32).abs().max().item() <= ATOL
    assert (i16 - i32).abs().max().item() <= ATOL


def test_engine_validation(device):
    z = torch.randn((6, 100, 16), device=device)
    with pytest.raises(ValueError, match='P >= 256'):
        _split(z)
    with pytest.raises(ValueError, match='Unknown MSM engine'):
        _MSM_hip.MSM(torch.randn((6, 300, 16), device=device), engine='bf16')
    n, p, c = 6, 100, 16
    size = ctypes.c_size_t()
    lib = rt.library()
    rt.check(lib.musc_msm_split_workspace_bytes(n, p, c, ctypes.byref(size)), 'ws')
    ws = rt.workspace(size.value, device)
    rc = lib.musc_msm_split_pair_minima(n, p, c, ws.data_ptr(), ws.numel(), rt.stream(device))
    assert rc == 1003  # MUSC_ERR_UNSUPPORTED: the C-ABI rejects p < 256 itself
