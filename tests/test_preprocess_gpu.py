"""GPU image preprocessing (musc_preprocess_u8) vs the CPU evaluation transform: bit-exact.

The oracle (oracle.preprocess) restates Pillow's bicubic resampling and torch's float32
ToTensor / Normalize and is itself pinned against PIL.Image.resize in test_oracle.py;
here the kernels are compared with it, and with Pillow's bytes directly.
"""
import numpy as np
import pytest
import torch

from oracle import preprocess as op
from musc_hip import _loader, _preprocess

pytestmark = pytest.mark.gpu

# fused band kernel (both axes resampled, in_w % 4 == 0), one case per tap count it is built
# for: 5 (224 -> 518), 7 (600), 9 (1024, 900, 700x840), 11 (1100), 13 (100x80 -> 37x41), 15 (1700);
# two passes through HBM: in_w % 4 != 0 (1022, 7x5, 3x3), one axis kept (33x517, 517x33, 518)
# or more than 15 taps (3000x8 -> 300x5)
CASES = [((1024, 1024), 518), ((900, 900), 518), ((224, 224), 518), ((518, 518), 518), ((700, 840), 518),
         ((100, 80), (37, 41)), ((33, 517), (33, 518)), ((517, 33), (518, 33)), ((7, 5), (300, 2)), ((3, 3), 1),
         ((1022, 1022), 518), ((3000, 8), (300, 5)), ((600, 600), 518), ((1100, 1100), 518),
         ((1700, 1700), 518)]


def _images(b, h, w, seed):
    rng = np.random.default_rng(seed)
    img = rng.integers(0, 256, (b, h, w, 3), dtype=np.uint8)
    img[:, : h // 2] = (np.arange(w)[None, None, :, None] * 7 % 256).astype(np.uint8)   # edges that clip
    return img


@pytest.mark.parametrize('src,size', CASES)
def test_matches_the_cpu_transform_bit_for_bit(device, src, size):
    h, w = src
    b = 2 if h * w > 200000 else 3
    imgs = _images(b, h, w, h + w)
    got = _preprocess.preprocess_u8(torch.from_numpy(imgs).to(device), size).cpu()
    oh, ow = (size, size) if isinstance(size, int) else size
    ref = torch.stack([op.to_tensor_normalize(op.resize_bicubic_u8(im, oh, ow)) for im in imgs], 0)
    assert got.shape == (b, 3, oh, ow)
    diff = (got - ref).abs().max().item()
    print(f'{src} -> {(oh, ow)}: max |gpu - cpu| {diff:.3e}', flush=True)
    assert torch.equal(got, ref)


def test_resized_bytes_equal_pillow(device):
    from PIL import Image
    imgs = _images(2, 640, 480, 7)
    # mean 0, std 1: the output is u / 255, from which the resized byte is recovered exactly
    got = _preprocess.preprocess_u8(torch.from_numpy(imgs).to(device), (300, 222), (0.0, 0.0, 0.0),
                                    (1.0, 1.0, 1.0)).cpu()
    u8 = torch.round(got * 255).to(torch.uint8).permute(0, 2, 3, 1).numpy()
    for i in range(2):
        ref = np.asarray(Image.fromarray(imgs[i], 'RGB').resize((222, 300), Image.BICUBIC))
        np.testing.assert_array_equal(u8[i], ref)


def test_unaligned_view_is_handled(device):
    imgs = _images(2, 64, 48, 9)
    flat = torch.zeros(imgs.size + 1, dtype=torch.uint8)
    flat[1:] = torch.from_numpy(imgs.reshape(-1))
    view = flat.to(device)[1:].view(2, 64, 48, 3)          # storage offset 1: not 4-byte aligned
    assert view.data_ptr() % 4 != 0
    got = _preprocess.preprocess_u8(view, 30).cpu()
    ref = torch.stack([op.clip_preprocess(im, 30) for im in imgs], 0)
    assert torch.equal(got, ref)


def test_single_image_and_out_argument(device):
    img = torch.from_numpy(_images(1, 50, 60, 1)[0]).to(device)
    one = _preprocess.preprocess_u8(img, 20)
    assert one.shape == (3, 20, 20)
    out = torch.empty((1, 3, 20, 20), device=device)
    again = _preprocess.preprocess_u8(img.unsqueeze(0), 20, out=out)
    assert again.data_ptr() == out.data_ptr() and torch.equal(again[0], one)
    with pytest.raises(ValueError):
        _preprocess.preprocess_u8(img.float(), 20)
    with pytest.raises(RuntimeError, match='implemented range'):   # beyond 64 taps (reduction above 15.5x)
        _preprocess.preprocess_u8(torch.zeros((1, 2000, 2000, 3), dtype=torch.uint8, device=device), 100)


def test_device_batches_end_to_end(device, tmp_path):
    # PNG files (RGB, grayscale, a second size) through the threaded loader, pinned uint8
    # batches, H2D and the kernels, against PIL decode + the CPU transform
    from PIL import Image
    rng = np.random.default_rng(5)
    arrays = [rng.integers(0, 256, (120, 90, 3), dtype=np.uint8) for _ in range(5)]
    arrays.append(np.repeat(rng.integers(0, 256, (120, 90), dtype=np.uint8)[:, :, None], 3, axis=2))
    arrays.append(rng.integers(0, 256, (64, 64, 3), dtype=np.uint8))
    paths = []
    for i, a in enumerate(arrays):
        p = str(tmp_path / f'{i}.png')
        if i == 5:
            Image.fromarray(a[:, :, 0], 'L').save(p)
        else:
            Image.fromarray(a, 'RGB').save(p)
        paths.append(p)
    seen = []
    for batch, names in _loader.device_batches(paths, size=70, batch_size=3, device=device):
        assert batch.device.type == 'cuda' and batch.shape[1:] == (3, 70, 70)
        for img, name in zip(batch.cpu(), names):
            idx = paths.index(name)
            assert torch.equal(img, op.clip_preprocess(arrays[idx], 70)), name
            seen.append(idx)
    assert seen == list(range(len(paths)))
