"""The reference's evaluation transform on MI355X (libmusc_hip musc_preprocess_u8).

models/backbone/open_clip/transform.py:118-133 (the `preprocess` handed to the datasets
at models/musc.py:80,88-96) runs per image on the CPU inside the dataset item:
Resize((S, S), BICUBIC) on the PIL image, CenterCrop, ToTensor, Normalize with the
OpenAI CLIP mean and std.  Here the decoded uint8 RGB images go to the GPU as bytes
(a quarter of the float32 volume) and one entry point produces the normalised float32
batch, bit-identical to Pillow's 8-bit bicubic resampling followed by torch's float32
ToTensor and Normalize.
"""
from __future__ import annotations

import ctypes

import torch

from . import _runtime as rt

OPENAI_DATASET_MEAN = (0.48145466, 0.4578275, 0.40821073)   # open_clip/constants.py:1
OPENAI_DATASET_STD = (0.26862954, 0.26130258, 0.27577711)    # open_clip/constants.py:2


def workspace_bytes(batch: int, in_h: int, in_w: int, out_h: int, out_w: int) -> int:
    out = ctypes.c_size_t()
    rt.check(rt.library().musc_preprocess_workspace_bytes(batch, in_h, in_w, out_h, out_w, ctypes.byref(out)),
             'musc_preprocess_workspace_bytes')
    return out.value


def _size(size) -> tuple[int, int]:
    if isinstance(size, int):
        return size, size
    h, w = size
    return int(h), int(w)


def preprocess_u8(images: torch.Tensor, size=518, mean=OPENAI_DATASET_MEAN, std=OPENAI_DATASET_STD,
                  out: torch.Tensor | None = None) -> torch.Tensor:
    """(B, H, W, 3) or (H, W, 3) uint8 RGB GPU tensor -> (B, 3, S, S) / (3, S, S) float32.

    `size` is an int (square output, as Resize((S, S))) or (out_h, out_w).  The result
    equals ToTensor()(Resize(size, BICUBIC)(image)) normalised with `mean` / `std`.
    """
    rt.require_device_tensor(images, 'images')
    single = images.ndim == 3
    x = images.unsqueeze(0) if single else images
    if x.ndim != 4 or x.shape[-1] != 3 or x.dtype != torch.uint8:
        raise ValueError('images must be uint8 (B, H, W, 3) or (H, W, 3) RGB')
    if len(mean) != 3 or len(std) != 3:
        raise ValueError('mean and std need one value per channel')
    b, h, w, _ = x.shape
    oh, ow = _size(size)
    x = x.contiguous()
    if x.data_ptr() % 16:
        x = x.clone()             # the fused kernel reads 4-byte words; a fresh allocation is aligned
    lib = rt.library()
    with torch.cuda.device(x.device):
        if out is None:
            out = torch.empty((b, 3, oh, ow), dtype=torch.float32, device=x.device)
        elif out.shape != (b, 3, oh, ow) or out.dtype != torch.float32 or not out.is_contiguous() \
                or out.device != x.device:
            raise ValueError('out must be a contiguous float32 (B, 3, out_h, out_w) tensor on the images device')
        ws = rt.workspace(workspace_bytes(b, h, w, oh, ow), x.device)
        m = (ctypes.c_float * 3)(*[float(v) for v in mean])
        s = (ctypes.c_float * 3)(*[float(v) for v in std])
        rc = lib.musc_preprocess_u8(x.data_ptr(), b, h, w, oh, ow, ctypes.cast(m, ctypes.c_void_p),
                                    ctypes.cast(s, ctypes.c_void_p), out.data_ptr(), ws.data_ptr(), ws.numel(),
                                    rt.stream(x.device))
        rt.check(rc, 'musc_preprocess_u8')
    return out[0] if single else out
