"""Fused attention over seeded random sequence lengths, both storage types and both layouts.

The fixed lists of test_attention_gpu.py and test_encoder_gpu.py pin the kernels' key
pipelines at chosen lengths; this sweep draws 24 lengths from 1 to 2100 (half of them next
to a multiple of the 32-key block, where the last block is ragged or full, with odd and
even block counts) and a number of heads, runs the contiguous and the packed (T, B, 3E)
entries and the block-12 head-averaged weights, and checks them against float64
softmax(q k^T * scale) v of the same (fp16-rounded, for fp16) inputs
(open_clip/transformer.py:232-234): the packed output must equal the contiguous one
bit for bit, the weights' rows must sum to 1.
"""
import numpy as np
import pytest
import torch

from musc_hip import _attention_hip

pytestmark = pytest.mark.gpu


def _lengths():
    rng = np.random.default_rng(77)
    out = []
    for i in range(24):
        if i % 2:
            t = int(rng.integers(1, 66)) * 32 + int(rng.choice([-1, 0, 1]))
        else:
            t = int(rng.integers(1, 2101))
        out.append(max(1, min(t, 2100)))
    return out


@pytest.mark.parametrize('t', _lengths())
@pytest.mark.parametrize('dtype', [torch.float32, torch.float16])
def test_random_length(device, dtype, t):
    g = torch.Generator().manual_seed(t * 3 + (dtype == torch.float16))
    b, h = 2, int(torch.randint(1, 4, (1,), generator=g))
    e = 64 * h
    qkv = (torch.randn((t, b, 3 * e), generator=g) * 0.6).to(dtype).to(device)
    parts = qkv.reshape(t, b, 3, h, 64)
    q, k, v = (parts[:, :, i].reshape(t, b * h, 64).transpose(0, 1).contiguous() for i in range(3))
    out = _attention_hip.attention(q, k, v, 0.125)
    q64, k64, v64 = q.double(), k.double(), v.double()
    p64 = torch.softmax(torch.bmm(q64 * 0.125, k64.transpose(1, 2).contiguous()), -1)
    ref = torch.bmm(p64, v64)
    err = (out.double() - ref).abs().max().item()
    tol = 2e-5 + 2e-5 * ref.abs().max().item() if dtype == torch.float32 else 2e-3
    print(f't={t} heads={h} {dtype}: {err:.2e} (tol {tol:.1e})', flush=True)
    assert err <= tol
    packed = _attention_hip.attention_packed(qkv, h, 0.125)
    assert torch.equal(packed, out.transpose(0, 1).reshape(t, b, e))
    w = _attention_hip.attention_weights_packed(qkv, h, 0.125)
    w_ref = p64.reshape(b, h, t, t).mean(1)
    werr = (w.double() - w_ref).abs().max().item()
    print(f'    weights: {werr:.2e}', flush=True)
    # fp32 logits from either storage type: the weights are fp32 arithmetic throughout
    assert w.shape == (b, t, t) and werr <= 1e-6
    torch.testing.assert_close(w.double().sum(-1), torch.ones((b, t), dtype=torch.float64, device=w.device),
                               rtol=0, atol=2e-5)
