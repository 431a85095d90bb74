"""Encoding plugin on the GPU: encode_image with the fused attention vs the same model's
own nn.MultiheadAttention math path."""
import pytest
import torch

from musc_hip import _attention_hip, _encoder_hip, vit

pytestmark = pytest.mark.gpu


def small_model(device, layers=4):
    torch.manual_seed(0)
    m = vit.CLIPVision(image_size=56, patch_size=14, width=128, layers=layers, heads=2, output_dim=32)
    return m.to(device).eval()


def test_fp32_tokens_match_math_path(device):
    model = small_model(device)
    image = torch.rand((2, 3, 56, 56), generator=torch.Generator().manual_seed(1)).to(device)
    with torch.no_grad():
        ref_pooled, ref_tokens = model.encode_image(image, [2, 4])
        _encoder_hip.begin_inference()
        pooled, tokens = _encoder_hip.encode_image(model, image, [2, 4])
    assert len(tokens) == 2 and tokens[0].shape == (2, 17, 128)
    torch.testing.assert_close(pooled, ref_pooled, rtol=1e-4, atol=1e-5)
    for a, b in zip(tokens, ref_tokens):
        torch.testing.assert_close(a, b, rtol=1e-4, atol=1e-5)
    stats = _encoder_hip.research_diagnostics()
    assert stats['fused_attention_calls'] == 4 and stats['weight_blocks'] == 1
    # the original forwards are restored
    for blk in model.visual.transformer.resblocks:
        assert 'forward' not in blk.attn.__dict__


def test_autocast_fp16(device):
    model = small_model(device)
    image = torch.rand((2, 3, 56, 56), generator=torch.Generator().manual_seed(2)).to(device)
    with torch.no_grad(), torch.autocast('cuda', dtype=torch.float16):
        ref_pooled, ref_tokens = model.encode_image(image, [4])
        pooled, tokens = _encoder_hip.encode_image(model, image, [4])
    assert tokens[0].dtype == torch.float16
    torch.testing.assert_close(tokens[0].float(), ref_tokens[0].float(), rtol=2e-2, atol=2e-2)


def test_vit_l14_full_size_block_tokens(device):
    # ViT-L/14 at 518 px: 1370 tokens, 16 heads of 64; compare block-6 tokens (fp32)
    torch.manual_seed(3)
    model = vit.vit_l14(518).to(device).eval()
    image = torch.rand((1, 3, 518, 518), generator=torch.Generator().manual_seed(4)).to(device)
    with torch.no_grad():
        _, ref = model.encode_image(image, [6])
        _, got = _encoder_hip.encode_image(model, image, [6])
    assert got[0].shape == (1, 1370, 1024)
    torch.testing.assert_close(got[0], ref[0], rtol=1e-3, atol=1e-3)


@pytest.mark.parametrize('t', [1, 31, 300, 1370])
@pytest.mark.parametrize('dtype', [torch.float32, torch.float16])
def test_attention_weights_kernel(device, t, dtype):
    # vs the float64 head-averaged softmax of the same (rounded) inputs; rows sum to 1
    g = torch.Generator().manual_seed(5 + t)
    b, h = 2, 16
    q, k = ((torch.randn((b * h, t, 64), generator=g) * 0.5).to(dtype) for _ in range(2))
    got = _attention_hip.attention_weights(q.to(device), k.to(device), h, 0.125).cpu()
    q64, k64 = q.double(), k.double()
    ref = torch.softmax((q64 @ k64.transpose(1, 2)) * 0.125, -1).reshape(b, h, t, t).mean(1)
    assert got.dtype == torch.float32 and got.shape == (b, t, t)
    torch.testing.assert_close(got.double(), ref, rtol=2e-5, atol=1e-7)
    torch.testing.assert_close(got.double().sum(-1), torch.ones((b, t), dtype=torch.float64), rtol=0, atol=2e-5)
