"""Fused encoder-block layers (musc_layernorm_rows, musc_activation) vs torch's own ops,
as the reference's modules call them (open_clip/transformer.py:23-35, 247-248)."""
import pytest
import torch
import torch.nn.functional as F

from musc_hip import _layers_hip
from musc_hip import _runtime as rt

pytestmark = pytest.mark.gpu


def _inputs(device, rows, width, dtype, seed, scale=1.0, offset=0.0):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn((rows, width), generator=g) * scale + offset).to(dtype).to(device)
    w = (1 + 0.1 * torch.randn(width, generator=g)).to(device)
    b = (0.1 * torch.randn(width, generator=g)).to(device)
    return x, w, b


def _assert_fp16_close(got, ref, terms):
    """Within one fp16 rounding step of ref, plus a few fp32 rounding steps of `terms`,
    the magnitudes that cancel in ref: near zero two fp32 evaluations in different
    summation orders may round to fp16 values several ulps of ref apart."""
    ulp = torch.finfo(torch.float16).eps * ref.float().abs().clamp_min(2.0 ** -14)
    bound = ulp + 4 * torch.finfo(torch.float32).eps * terms
    excess = (got.float() - ref.float()).abs() - bound
    worst = int(excess.argmax())
    assert excess.max() <= 0, (f'max excess {excess.max().item():.3e} at {worst}: got '
                               f'{got.flatten()[worst].item()} ref {ref.flatten()[worst].item()}')


def _ln_terms(x, w, b):
    # |x_hat w| + |b| + 8 |w| mean|x| / std: the last term bounds how far an fp32
    # row mean computed in another order moves x_hat (delta_mean * rstd)
    xf = x.float()
    xhat = F.layer_norm(xf, (x.shape[-1],), None, None, 1e-5)
    spread = xf.abs().mean(-1, keepdim=True) / xf.std(-1, unbiased=False, keepdim=True).clamp_min(1e-3)
    return (xhat * w).abs() + b.abs() + 8 * w.abs() * spread


def _torch_cast_back_ln(x, w, b, eps=1e-5):
    # LayerNorm.forward of transformer.py:26-29 under fp16 autocast: fp32 layer_norm, cast back
    return F.layer_norm(x.float(), (x.shape[-1],), w, b, eps).to(x.dtype)


@pytest.mark.parametrize('width', [64, 128, 1000, 1024])
def test_layer_norm_fp32(device, width):
    x, w, b = _inputs(device, 257, width, torch.float32, width, scale=3.0, offset=5.0)
    got = _layers_hip.layer_norm(x, w, b, 1e-5)
    torch.testing.assert_close(got, _torch_cast_back_ln(x, w, b), rtol=1e-5, atol=2e-5)


@pytest.mark.parametrize('width', [128, 1024, 2048])
def test_layer_norm_fp16_within_one_ulp(device, width):
    x, w, b = _inputs(device, 1370 * 2, width, torch.float16, width, scale=2.0, offset=1.0)
    got = _layers_hip.layer_norm(x, w, b, 1e-5)
    ref = _torch_cast_back_ln(x, w, b)
    assert got.dtype == torch.float16
    # fp32 statistics in a different summation order: one fp16 rounding step apart
    _assert_fp16_close(got, ref, _ln_terms(x, w, b))
    assert (got == ref).float().mean() > 0.99


@pytest.mark.parametrize('dtype', [torch.float32, torch.float16])
def test_residual_add_and_layer_norm(device, dtype):
    x, w, b = _inputs(device, 513, 1024, dtype, 11)
    r, _, _ = _inputs(device, 513, 1024, dtype, 12, scale=0.5)
    s, y = _layers_hip.layer_norm(x, w, b, 1e-5, residual=r)
    assert torch.equal(s, x + r)                      # torch's own add, bit for bit
    ref = _torch_cast_back_ln(x + r, w, b)
    if dtype == torch.float32:
        torch.testing.assert_close(y, ref, rtol=1e-5, atol=2e-5)
    else:
        _assert_fp16_close(y, ref, _ln_terms(x + r, w, b))


def test_layer_norm_constant_rows_and_no_affine(device):
    # constant rows: zero variance -> (x - mean) = 0 -> output = bias (eps keeps rstd finite)
    x = torch.full((8, 256), 3.25, device=device)
    w = torch.ones(256, device=device)
    b = torch.linspace(-1, 1, 256, device=device)
    torch.testing.assert_close(_layers_hip.layer_norm(x, w, b, 1e-5), b.expand(8, 256), rtol=0, atol=0)
    x2, _, _ = _inputs(device, 16, 256, torch.float32, 13)
    torch.testing.assert_close(_layers_hip.layer_norm(x2, None, None, 1e-5),
                               F.layer_norm(x2, (256,), None, None, 1e-5), rtol=1e-5, atol=2e-5)


def test_quick_gelu_fp16_matches_torch_ops(device):
    # x * torch.sigmoid(1.702 * x) in fp16 (three roundings), transformer.py:32-35
    g = torch.Generator().manual_seed(14)
    x = (torch.randn((5480, 4096), generator=g) * 3).half().to(device)
    ref = x * torch.sigmoid(1.702 * x)
    got = _layers_hip.activation_(x.clone(), rt.ACT_QUICK_GELU)
    _assert_fp16_close(got, ref, torch.zeros_like(ref, dtype=torch.float32))
    assert (got == ref).float().mean() > 0.999


def _all_finite_fp16(device):
    bits = torch.arange(-32768, 32768, dtype=torch.int32).to(torch.int16)
    x = bits.view(torch.float16)
    return x[torch.isfinite(x)].contiguous().to(device)    # 63488 values, both zeros, subnormals


def test_quick_gelu_fp16_every_input(device):
    # the activation is elementwise, so agreement on every finite fp16 value is agreement
    # on any tensor: bit-identical to torch's three-op fp16 chain (transformer.py:32-35)
    x = _all_finite_fp16(device)
    ref = x * torch.sigmoid(1.702 * x)
    got = _layers_hip.activation_(x.clone(), rt.ACT_QUICK_GELU)
    assert torch.equal(torch.isfinite(got), torch.isfinite(ref))
    fin = torch.isfinite(ref)
    match = (got[fin] == ref[fin]).float().mean().item()
    print(f'QuickGELU fp16: {match:.6f} of {int(fin.sum())} finite inputs bit-identical to torch', flush=True)
    assert torch.equal(got[fin], ref[fin])
    # the non-finite inputs: +inf -> +inf, -inf -> NaN (-inf * 0), NaN -> NaN, as torch
    special = torch.tensor([float('inf'), float('-inf'), float('nan')], dtype=torch.float16, device=device)
    ref_s = special * torch.sigmoid(1.702 * special)
    got_s = _layers_hip.activation_(torch.cat([special, special.new_zeros(5)]), rt.ACT_QUICK_GELU)[:3]
    assert torch.equal(torch.isnan(got_s), torch.isnan(ref_s))
    assert torch.equal(got_s[~torch.isnan(ref_s)], ref_s[~torch.isnan(ref_s)])


def test_gelu_fp16_every_input(device):
    x = _all_finite_fp16(device)
    ref = F.gelu(x)
    got = _layers_hip.activation_(x.clone(), rt.ACT_GELU)
    assert torch.equal(torch.isfinite(got), torch.isfinite(ref))
    fin = torch.isfinite(ref)
    _assert_fp16_close(got[fin], ref[fin], x[fin].float().abs())


@pytest.mark.parametrize('mode', [0, 1])
def test_activation_fp32(device, mode):
    g = torch.Generator().manual_seed(15 + mode)
    x = (torch.randn((1000, 512), generator=g) * 3).to(device)
    ref = x * torch.sigmoid(1.702 * x) if mode == rt.ACT_QUICK_GELU else F.gelu(x)
    got = _layers_hip.activation_(x.clone(), mode)
    torch.testing.assert_close(got, ref, rtol=1e-6, atol=1e-6)


def test_activation_gelu_fp16(device):
    g = torch.Generator().manual_seed(17)
    x = (torch.randn((256, 1024), generator=g) * 3).half().to(device)
    ref = F.gelu(x)
    got = _layers_hip.activation_(x.clone(), rt.ACT_GELU)
    _assert_fp16_close(got, ref, x.float().abs())
