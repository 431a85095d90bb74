"""The data path and the encoder-block layers over seeded random shapes.

Preprocessing: 16 draws of source sizes (1-1500 per axis, any aspect) and output sizes
(down to 1/15 of the source per axis, the kernel's tap range, up to 3x), through
musc_preprocess_u8 with mean 0 and std 1, so that the resized bytes are recovered
exactly and compared with PIL.Image.resize(BICUBIC) itself (the reference's transform,
open_clip/transform.py:118-133 on PIL images).  LayerNorm: 16 draws of row counts,
widths (the multiples of 4 up to 1024 in fp32, of 8 up to 2048 in fp16 that the kernel
takes), with and without the affine parameters and the fused residual add, against
torch's layer_norm as transformer.py:23-29 calls it, to the tolerances of
test_layers_gpu.py.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from musc_hip import _layers_hip, _preprocess
from test_layers_gpu import _assert_fp16_close, _ln_terms

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize('k', range(16))
def test_random_resize_equals_pillow(device, k):
    from PIL import Image
    rng = np.random.default_rng(3000 + k)
    h, w = int(rng.integers(1, 1501)), int(rng.integers(1, 1501))
    oh = int(rng.integers(max(1, -(-h // 15)), min(3 * h, 700) + 1))
    ow = int(rng.integers(max(1, -(-w // 15)), min(3 * w, 700) + 1))
    b = int(rng.integers(1, 3))
    imgs = rng.integers(0, 256, (b, h, w, 3), dtype=np.uint8)
    imgs[:, : h // 3] = (np.arange(w)[None, None, :, None] * 13 % 256).astype(np.uint8)   # edges that clip
    got = _preprocess.preprocess_u8(torch.from_numpy(imgs).to(device), (oh, ow), (0.0, 0.0, 0.0),
                                    (1.0, 1.0, 1.0)).cpu()
    u8 = torch.round(got * 255).to(torch.uint8).permute(0, 2, 3, 1).numpy()
    print(f'resize {k}: ({h}, {w}) -> ({oh}, {ow}) x{b}', flush=True)
    for i in range(b):
        ref = np.asarray(Image.fromarray(imgs[i], 'RGB').resize((ow, oh), Image.BICUBIC))
        np.testing.assert_array_equal(u8[i], ref)


@pytest.mark.parametrize('k', range(16))
def test_random_layer_norm(device, k):
    rng = np.random.default_rng(4000 + k)
    fp16 = bool(rng.integers(0, 2))
    dtype = torch.float16 if fp16 else torch.float32
    per, top = (8, 2048) if fp16 else (4, 1024)
    width = int(rng.integers(1, top // per + 1)) * per
    rows = int(rng.integers(1, 3000))
    affine, residual = bool(rng.integers(0, 2)), bool(rng.integers(0, 2))
    g = torch.Generator().manual_seed(k)
    x = (torch.randn((rows, width), generator=g) * float(rng.uniform(0.2, 4)) + float(rng.uniform(-3, 3)))
    x = x.to(dtype).to(device)
    w = (1 + 0.1 * torch.randn(width, generator=g)).to(device) if affine else None
    b = (0.1 * torch.randn(width, generator=g)).to(device) if affine else None
    assert _layers_hip.supports_layer_norm(width, dtype)
    if residual:
        r = (torch.randn((rows, width), generator=g) * 0.5).to(dtype).to(device)
        s, y = _layers_hip.layer_norm(x, w, b, 1e-5, residual=r)
        assert torch.equal(s, x + r)
        x = x + r
    else:
        y = _layers_hip.layer_norm(x, w, b, 1e-5)
    ref = F.layer_norm(x.float(), (width,), w, b, 1e-5).to(dtype)
    print(f'layer_norm {k}: rows={rows} width={width} {dtype} affine={affine} residual={residual}', flush=True)
    if fp16:
        ones = torch.ones(width, device=device)
        _assert_fp16_close(y, ref, _ln_terms(x, w if affine else ones, b if affine else 0 * ones))
    else:
        torch.testing.assert_close(y, ref, rtol=1e-5, atol=2e-5)
