"""Fused ViT block attention on MI355X (libmusc_hip musc_attention_fwd).

softmax(q k^T * scale) v for (B*H, T, 64) fp32 or fp16 tensors, one pass with an
online softmax: the (B*H, T, T) logits of the reference's math path
(models/backbone/open_clip/transformer.py:232-234, softmax fused at
models/modules/_attention_gpu.py:41-81) never reach HBM.
"""
from __future__ import annotations

import ctypes

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


def attention_weights(q: torch.Tensor, k: torch.Tensor, heads: int, scale: float) -> torch.Tensor:
    """Head-averaged softmax(q k^T * scale): (B*H, T, 64) q, k -> (B, T, T) fp32."""
    for name, x in (('q', q), ('k', k)):
        rt.require_device_tensor(x, name)
    if q.shape != k.shape or q.ndim != 3 or q.dtype != k.dtype or q.dtype not in (torch.float32, torch.float16):
        raise ValueError('q and k must share one (B*H, T, D) float32/float16 shape')
    bh, t, d = q.shape
    if heads < 1 or bh % heads:
        raise ValueError('leading dimension must be batch * heads')
    q, k = q.contiguous(), k.contiguous()
    lib = rt.library()
    need = ctypes.c_size_t()
    rt.check(lib.musc_attention_weights_workspace_bytes(bh // heads, heads, t, ctypes.byref(need)),
             'musc_attention_weights_workspace_bytes')
    with torch.cuda.device(q.device):
        out = torch.empty((bh // heads, t, t), dtype=torch.float32, device=q.device)
        ws = torch.empty(need.value, dtype=torch.uint8, device=q.device)
        rc = lib.musc_attention_weights(q.data_ptr(), k.data_ptr(),
                                        rt.DTYPE_F32 if q.dtype == torch.float32 else rt.DTYPE_F16,
                                        bh // heads, heads, t, d, float(scale), out.data_ptr(),
                                        ws.data_ptr(), need.value, rt.stream(q.device))
        rt.check(rc, 'musc_attention_weights')
    return out
