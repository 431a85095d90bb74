"""CPU oracle for the image preprocessing of the data path.  TEST INFRASTRUCTURE ONLY.

The reference feeds the encoder with open_clip's evaluation transform
(models/backbone/open_clip/transform.py:118-133, built at factory.py:362 and handed
to the datasets as `clip_transformer`, models/musc.py:80,88-96), applied per image
in the dataset item (datasets/mvtec.py:101-103, after PIL's `.convert("RGB")`):

    Resize((S, S), BICUBIC) -> CenterCrop((S, S)) -> convert('RGB') -> ToTensor()
    -> Normalize(OPENAI_DATASET_MEAN, OPENAI_DATASET_STD)

torchvision's Resize on a PIL image calls `PIL.Image.resize((S, S), BICUBIC)`, so the
arithmetic of the resize lives in Pillow (third-party; the reference pins
Pillow==11.1.0, requirements.txt:13).  `resize_bicubic_u8` restates Pillow's published
8-bit resampling algorithm (libImaging/Resample.c):

  * per axis, coefficients from the bicubic kernel (a = -0.5, support 2) stretched by
    max(in/out, 1) (antialiasing when reducing), window [xmin, xmin + n) around
    center = (x + 0.5) * in/out with xmin = int(center - support + 0.5) and xmax =
    int(center + support + 0.5) clipped to the image, normalised to sum 1, then turned
    into 22-bit fixed point (rounded half away from zero);
  * a horizontal pass over the source rows the vertical pass will read, writing uint8
    (accumulator starts at 2^21, result clipped to [0, 255] after >> 22), then a
    vertical pass over that intermediate the same way;
  * a pass is skipped when its axis keeps its size; an unchanged image is copied.

ToTensor is `uint8 -> float32 / 255` and Normalize `(x - mean) / std` in float32
(torch CPU arithmetic, as torchvision runs them in the dataset worker).  The
restatement is pinned bit for bit against PIL.Image.resize itself in
tests/test_oracle.py (Pillow is installed in this container; the reference's own
tests hold no fixtures for this path).
"""
from __future__ import annotations

import math

import numpy as np
import torch

PRECISION_BITS = 32 - 8 - 2
OPENAI_DATASET_MEAN = (0.48145466, 0.4578275, 0.40821073)   # open_clip/constants.py:1
OPENAI_DATASET_STD = (0.26862954, 0.26130258, 0.27577711)    # open_clip/constants.py:2


def _bicubic(x: float) -> float:
    a = -0.5
    if x < 0.0:
        x = -x
    if x < 1.0:
        return ((a + 2.0) * x - (a + 3.0)) * x * x + 1
    if x < 2.0:
        return (((x - 5) * x + 8) * x - 4) * a
    return 0.0


def coefficients(in_size: int, out_size: int) -> tuple[np.ndarray, np.ndarray, int]:
    """(bounds (out, 2) int: xmin, count), fixed-point coefficients (out, ksize) int64, ksize."""
    scale = float(in_size) / out_size
    filterscale = max(scale, 1.0)
    support = 2.0 * filterscale
    ksize = int(math.ceil(support)) * 2 + 1
    bounds = np.zeros((out_size, 2), dtype=np.int64)
    kk = np.zeros((out_size, ksize), dtype=np.int64)
    ss = 1.0 / filterscale
    for xx in range(out_size):
        center = 0.0 + (xx + 0.5) * scale
        xmin = int(center - support + 0.5)
        if xmin < 0:
            xmin = 0
        xmax = int(center + support + 0.5)
        if xmax > in_size:
            xmax = in_size
        xmax -= xmin
        w = [_bicubic((x + xmin - center + 0.5) * ss) for x in range(xmax)]
        ww = 0.0
        for v in w:
            ww += v
        for x in range(xmax):
            k = w[x] / ww if ww != 0.0 else w[x]
            kk[xx, x] = int(-0.5 + k * (1 << PRECISION_BITS)) if k < 0 else int(0.5 + k * (1 << PRECISION_BITS))
        bounds[xx] = (xmin, xmax)
    return bounds, kk, ksize


def _clip8(acc: np.ndarray) -> np.ndarray:
    out = np.right_shift(acc, PRECISION_BITS)
    out = np.where(acc >= (1 << PRECISION_BITS << 8), 255, out)
    out = np.where(acc <= 0, 0, out)
    return out.astype(np.uint8)


def _pass(src: np.ndarray, bounds: np.ndarray, kk: np.ndarray, axis: int) -> np.ndarray:
    """Resample uint8 src (H, W, 3) along axis 1 (horizontal) or 0 (vertical)."""
    n_out = bounds.shape[0]
    s = src.astype(np.int64)
    if axis == 1:
        acc = np.full((src.shape[0], n_out, src.shape[2]), 1 << (PRECISION_BITS - 1), dtype=np.int64)
        for xx in range(n_out):
            xmin, cnt = bounds[xx]
            acc[:, xx, :] += (s[:, xmin:xmin + cnt, :] * kk[xx, :cnt][None, :, None]).sum(axis=1)
    else:
        acc = np.full((n_out, src.shape[1], src.shape[2]), 1 << (PRECISION_BITS - 1), dtype=np.int64)
        for yy in range(n_out):
            ymin, cnt = bounds[yy]
            acc[yy] += (s[ymin:ymin + cnt] * kk[yy, :cnt][:, None, None]).sum(axis=0)
    return _clip8(acc)


def resize_bicubic_u8(img: np.ndarray, out_h: int, out_w: int) -> np.ndarray:
    """uint8 (H, W, 3) -> uint8 (out_h, out_w, 3), as PIL.Image.resize((out_w, out_h), BICUBIC)."""
    h, w = img.shape[:2]
    need_h, need_v = out_w != w, out_h != h
    if not need_h and not need_v:
        return img.copy()
    bh, kh, _ = coefficients(w, out_w)
    bv, kv, _ = coefficients(h, out_h)
    first = int(bv[0, 0])
    last = int(bv[out_h - 1, 0] + bv[out_h - 1, 1])
    cur = img
    if need_h:
        cur = _pass(img[first:last], bh, kh, axis=1)
        bv = bv.copy()
        bv[:, 0] -= first
    if need_v:
        cur = _pass(cur, bv, kv, axis=0)
    return cur


def to_tensor_normalize(img: np.ndarray, mean=OPENAI_DATASET_MEAN, std=OPENAI_DATASET_STD) -> torch.Tensor:
    """uint8 (H, W, 3) -> float32 (3, H, W): ToTensor then Normalize, torch CPU arithmetic."""
    t = torch.from_numpy(np.ascontiguousarray(img)).permute(2, 0, 1).contiguous()
    t = t.to(dtype=torch.float32).div(255)
    m = torch.as_tensor(mean, dtype=torch.float32).view(-1, 1, 1)
    s = torch.as_tensor(std, dtype=torch.float32).view(-1, 1, 1)
    return t.sub(m).div(s)


def clip_preprocess(img: np.ndarray, size: int, mean=OPENAI_DATASET_MEAN, std=OPENAI_DATASET_STD) -> torch.Tensor:
    """The whole evaluation transform on one RGB uint8 (H, W, 3) image -> (3, size, size)."""
    resized = resize_bicubic_u8(img, size, size)
    # CenterCrop((size, size)) of a size x size image is the identity
    return to_tensor_normalize(resized, mean, std)
