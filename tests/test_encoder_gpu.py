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


@pytest.mark.parametrize('patch_gemm', [False, True])
def test_fp32_tokens_match_math_path(device, monkeypatch, patch_gemm):
    monkeypatch.setattr(_encoder_hip, 'PATCH_EMBED_GEMM', patch_gemm)
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
    assert stats['fused_blocks'] == 4 and stats['fused_attention_calls'] == 4 and stats['weight_blocks'] == 1
    assert stats['fused_layer_norms'] == 2 and stats['fallback_calls'] == 0        # ln_pre, ln_post
    assert stats['patch_embeds'] == (1 if patch_gemm else 0)
    # the original forwards are restored
    for blk in model.visual.transformer.resblocks:
        assert 'forward' not in blk.__dict__ and 'forward' not in blk.attn.__dict__
    assert 'forward' not in model.visual.ln_pre.__dict__ and 'forward' not in model.visual.ln_post.__dict__
    assert 'forward' not in model.visual.conv1.__dict__


@pytest.mark.parametrize('hw', [(56, 56), (518, 518), (31, 44)])
@pytest.mark.parametrize('autocast', [False, True])
def test_patch_embedding_gemm_matches_conv(device, hw, autocast):
    # conv1 with kernel == stride as patches @ W^T; (31, 44): the rows and columns past
    # the last whole patch are dropped, as the convolution drops them
    torch.manual_seed(5)
    conv = torch.nn.Conv2d(3, 96, kernel_size=14, stride=14, bias=False).to(device)
    biased = torch.nn.Conv2d(3, 96, kernel_size=14, stride=14, bias=True).to(device)
    x = torch.rand((3, 3) + hw, generator=torch.Generator().manual_seed(6)).to(device)
    for m in (conv, biased):
        assert _encoder_hip._patch_conv(m)
        hook = _encoder_hip._patch_embed_forward(m, m.forward)
        with torch.no_grad(), torch.autocast('cuda', dtype=torch.float16, enabled=autocast):
            ref, got = m(x), hook(x)
        assert got.shape == ref.shape and got.dtype == ref.dtype
        tol = dict(rtol=2e-3, atol=2e-3) if autocast else dict(rtol=1e-5, atol=1e-5)
        torch.testing.assert_close(got.float(), ref.float(), **tol)
    assert not _encoder_hip._patch_conv(torch.nn.Conv2d(3, 8, kernel_size=14, stride=7))
    assert not _encoder_hip._patch_conv(torch.nn.Conv2d(3, 8, kernel_size=14, stride=14, padding=1))


def test_autocast_fp16(device):
    model = small_model(device)
    image = torch.rand((2, 3, 56, 56), generator=torch.Generator().manual_seed(2)).to(device)
    with torch.no_grad(), torch.autocast('cuda', dtype=torch.float16):
        ref_pooled, ref_tokens = model.encode_image(image, [4])
        pooled, tokens = _encoder_hip.encode_image(model, image, [4])
    assert tokens[0].dtype == torch.float16
    torch.testing.assert_close(tokens[0].float(), ref_tokens[0].float(), rtol=2e-2, atol=2e-2)
    torch.testing.assert_close(pooled.float(), ref_pooled.float(), rtol=2e-2, atol=2e-2)


def test_attention_level_hook_for_other_blocks(device):
    # a block whose activation the fused block path does not cover (tanh GELU) keeps its
    # own forward; only its nn.MultiheadAttention is replaced
    model = small_model(device, layers=2)
    for blk in model.visual.transformer.resblocks:
        blk.mlp.gelu = torch.nn.GELU(approximate='tanh')
    image = torch.rand((2, 3, 56, 56), generator=torch.Generator().manual_seed(7)).to(device)
    with torch.no_grad():
        ref_pooled, ref_tokens = model.encode_image(image, [2])
        _encoder_hip.begin_inference()
        pooled, tokens = _encoder_hip.encode_image(model, image, [2])
    torch.testing.assert_close(tokens[0], ref_tokens[0], rtol=1e-4, atol=1e-5)
    stats = _encoder_hip.research_diagnostics()
    assert stats['fused_blocks'] == 0 and stats['fused_attention_calls'] == 2
    for blk in model.visual.transformer.resblocks:
        assert 'forward' not in blk.__dict__ and 'forward' not in blk.attn.__dict__


def test_masked_call_falls_back(device):
    model = small_model(device, layers=1)
    blk = model.visual.transformer.resblocks[0]
    x = torch.randn((17, 2, 128), generator=torch.Generator().manual_seed(8)).to(device)
    mask = torch.zeros((17, 17), device=device)
    mask[:, 3] = float('-inf')
    with torch.no_grad():
        ref, _ = blk(x, attn_mask=mask)
        fused = _encoder_hip._fused_block_forward(blk, blk.forward, 0, False)
        _encoder_hip.begin_inference()
        got, _ = fused(x, attn_mask=mask)
    torch.testing.assert_close(got, ref, rtol=0, atol=0)
    assert _encoder_hip.research_diagnostics()['fallback_calls'] == 1


@pytest.mark.parametrize('dtype', [torch.float32, torch.float16])
@pytest.mark.parametrize('t', [1, 33, 150, 300, 1370])
def test_packed_attention_matches_contiguous(device, dtype, t):
    # the strided kernels read (T, B, 3E) in place; same arithmetic as the contiguous entry
    g = torch.Generator().manual_seed(9)
    b, h = 3, 4
    e = 64 * h
    qkv = (torch.randn((t, b, 3 * e), generator=g) * 0.5).to(dtype).to(device)
    parts = qkv.reshape(t, b, 3, h, 64)
    q, k, v = (parts[:, :, i].reshape(t, b * h, 64).transpose(0, 1).contiguous() for i in range(3))
    ref = _attention_hip.attention(q, k, v, 0.125).transpose(0, 1).reshape(t, b, e)
    got = _attention_hip.attention_packed(qkv, h, 0.125)
    assert got.shape == (t, b, e) and got.dtype == dtype
    assert torch.equal(got, ref)
    w_ref = _attention_hip.attention_weights(q, k, h, 0.125)
    w_got = _attention_hip.attention_weights_packed(qkv, h, 0.125)
    assert torch.equal(w_got, w_ref)


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
