"""Fused attention parity on the GPU vs torch softmax(q k^T * scale) v (CPU fp32, or float64 for config 4)."""
import pytest
import torch

from musc_hip import _attention_hip, synthetic

pytestmark = pytest.mark.gpu


def reference(q, k, v, scale):
    q, k, v = (x.detach().cpu().float() for x in (q, k, v))
    return torch.softmax((q * scale) @ k.transpose(1, 2), -1) @ v


@pytest.mark.parametrize('bh,t', [(4, 1), (3, 33), (2, 77), (8, 1370)])
def test_fp32(device, bh, t):
    g = torch.Generator().manual_seed(bh * 10000 + t)
    q, k, v = (torch.randn((bh, t, 64), generator=g) * 0.64 for _ in range(3))
    out = _attention_hip.attention(q.to(device), k.to(device), v.to(device), 0.125).cpu()
    ref = reference(q, k, v, 0.125)
    torch.testing.assert_close(out, ref, rtol=1e-4, atol=2e-5)


def test_fp16_storage(device):
    g = torch.Generator().manual_seed(1)
    q, k, v = (torch.randn((8, 1370, 64), generator=g).half() for _ in range(3))
    out = _attention_hip.attention(q.to(device), k.to(device), v.to(device), 0.125).cpu()
    assert out.dtype == torch.float16
    ref = reference(q, k, v, 0.125)
    torch.testing.assert_close(out.float(), ref, rtol=2e-3, atol=2e-3)


@pytest.mark.parametrize('bh,t', [(4, 1), (3, 31), (3, 33), (2, 64), (2, 65), (2, 77), (2, 97), (2, 129), (2, 161)])
def test_fp16_ragged(device, bh, t):
    # every tail of the fp16 kernel's three-stage key pipeline (1 to 6 key blocks, ragged
    # last block) against the CPU fp32 reference of the same fp16 inputs
    g = torch.Generator().manual_seed(bh * 10000 + t + 7)
    q, k, v = (torch.randn((bh, t, 64), generator=g).half() * 0.64 for _ in range(3))
    out = _attention_hip.attention(q.to(device), k.to(device), v.to(device), 0.125).cpu()
    torch.testing.assert_close(out.float(), reference(q, k, v, 0.125), rtol=2e-3, atol=2e-3)


@pytest.mark.parametrize('dtype', [torch.float32, torch.float16])
@pytest.mark.parametrize('t,slope', [(700, 0.1), (1370, 0.05), (300, 0.6)])
def test_growing_logits(device, dtype, t, slope):
    # logits rising along the keys: the running maximum is raised every few blocks, so
    # the accumulator rescaling (and, in the fp16 kernel, the rescaling of probabilities
    # whose P V product is still pending) runs many times per query
    g = torch.Generator().manual_seed(t)
    q = torch.zeros((2, t, 64))
    k = torch.randn((2, t, 64), generator=g) * 0.1
    q[:, :, 0] = 1.0
    k[:, :, 0] += slope * torch.arange(t).float()
    v = torch.randn((2, t, 64), generator=g)
    q, k, v = q.to(dtype), k.to(dtype), v.to(dtype)
    out = _attention_hip.attention(q.to(device), k.to(device), v.to(device), 1.0).cpu().float()
    tol = 1e-4 if dtype == torch.float32 else 1e-2
    torch.testing.assert_close(out, reference(q, k, v, 1.0), rtol=tol, atol=tol)


@pytest.mark.parametrize('dtype', [torch.float32, torch.float16])
def test_huge_logits(device, dtype):
    # logits near 2400 (about 3460 in log2 units): past the range in which the fp16 kernel
    # keeps its running maximum an integer and folds it into the logits MFMA, so it issues
    # the logits unshifted and re-bases every block
    g = torch.Generator().manual_seed(17)
    t = 160
    q = torch.zeros((2, t, 64))
    q[:, :, 0] = 60.0
    k = torch.randn((2, t, 64), generator=g) * 0.1
    k[:, :, 0] += 40.0 + 0.05 * torch.randn((2, t), generator=g)
    v = torch.randn((2, t, 64), generator=g)
    q, k, v = q.to(dtype), k.to(dtype), v.to(dtype)
    out = _attention_hip.attention(q.to(device), k.to(device), v.to(device), 1.0).cpu().double()
    q64, k64, v64 = (x.double() for x in (q, k, v))
    ref = torch.softmax(q64 @ k64.transpose(1, 2), -1) @ v64
    tol = 1e-4 if dtype == torch.float32 else 1e-2
    assert torch.isfinite(out).all()
    torch.testing.assert_close(out, ref, rtol=tol, atol=tol)


@pytest.mark.parametrize('dtype', [torch.float32, torch.float16])
def test_sharp_logits_select_one_row_dtypes(device, dtype):
    t = 100
    q = torch.zeros((1, t, 64))
    k = torch.zeros((1, t, 64))
    q[0, :, 0] = 50.0
    k[0, 37, 0] = 1.0
    v = torch.randn((1, t, 64))
    out = _attention_hip.attention(q.to(dtype).to(device), k.to(dtype).to(device), v.to(dtype).to(device), 1.0)
    expect = v[0, 37].to(dtype).float().expand(t, 64)
    torch.testing.assert_close(out.cpu().float()[0], expect, rtol=0, atol=1e-5 if dtype == torch.float32 else 1e-3)


def test_sharp_logits_select_one_row(device):
    t = 100
    q = torch.zeros((1, t, 64))
    k = torch.zeros((1, t, 64))
    q[0, :, 0] = 50.0
    k[0, 37, 0] = 1.0
    v = torch.randn((1, t, 64))
    out = _attention_hip.attention(q.to(device), k.to(device), v.to(device), 1.0).cpu()
    torch.testing.assert_close(out[0], v[0, 37].expand(t, 64), rtol=0, atol=1e-5)


@pytest.mark.parametrize('dtype', [torch.float32, torch.float16])
def test_config4_all_blocks(device, dtype):
    # Config 4: B=4, T=1370, 16 heads of 64; q, k, v = N(0,1) tokens @ N(0, 0.02^2) weights,
    # every one of the 24 blocks against softmax(q k^T / 8) v in float64 (on the GPU, from
    # the same stored inputs).
    tol = 2e-5 if dtype == torch.float32 else 2e-4
    for blk, (q, k, v) in enumerate(synthetic.attention_blocks(24, device=device)):
        q, k, v = q.to(dtype), k.to(dtype), v.to(dtype)
        out = _attention_hip.attention(q, k, v, 0.125)
        q64, k64, v64 = q.double(), k.double(), v.double()
        ref = torch.softmax(torch.bmm(q64 * 0.125, k64.transpose(1, 2).contiguous()), -1)
        ref = torch.bmm(ref, v64)
        err = (out.double() - ref).abs().max().item()
        print(f'block {blk}: max |err| {err:.3e}', flush=True)
        assert err <= tol + tol * ref.abs().max().item(), (blk, err)
