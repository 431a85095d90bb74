"""Fused ViT block attention on MI355X (libmusc_hip musc_attention_fwd).

softmax(q k^T * scale) v for (B*H, T, 64) fp32 or fp16 tensors, one pass with an
online softmax: the (B*H, T, T) logits of the reference's math path
(models/backbone/open_clip/transformer.py:232-234, softmax fused at
models/modules/_attention_gpu.py:41-81) never reach HBM.
"""
from __future__ import annotations

import torch

from . import _runtime as rt


def attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float) -> torch.Tensor:
    for name, x in (('q', q), ('k', k), ('v', v)):
        rt.require_device_tensor(x, name)
    if not (q.shape == k.shape == v.shape) or q.ndim != 3:
        raise ValueError('q, k, v must share one (B*H, T, D) shape')
    if not (q.dtype == k.dtype == v.dtype) or q.dtype not in (torch.float32, torch.float16):
        raise ValueError('q, k, v must all be float32 or all float16')
    bh, t, d = q.shape
    q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
    with torch.cuda.device(q.device):
        out = torch.empty_like(q)
        rc = rt.library().musc_attention_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
                                             rt.DTYPE_F32 if q.dtype == torch.float32 else rt.DTYPE_F16,
                                             bh, t, d, float(scale), rt.stream(q.device))
        rt.check(rc, 'musc_attention_fwd')
    return out
