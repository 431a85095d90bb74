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


def _packed_layout(qkv: torch.Tensor, heads: int):
    """(T, B, 3E) in-projection output -> pointers of q, k, v and their head strides."""
    rt.require_device_tensor(qkv, 'qkv')
    if qkv.ndim != 3 or qkv.dtype not in (torch.float32, torch.float16) or not qkv.is_contiguous():
        raise ValueError('qkv must be a contiguous (T, B, 3*heads*64) float32/float16 tensor')
    t, b, e3 = qkv.shape
    e = heads * 64
    if heads < 1 or e3 != 3 * e:
        raise ValueError(f'qkv last dimension {e3} is not 3 * heads * 64 = {3 * e}')
    elt = qkv.element_size()
    base = qkv.data_ptr()
    return t, b, e, (base, base + e * elt, base + 2 * e * elt), (3 * e, 64, b * 3 * e)


def attention_packed(qkv: torch.Tensor, heads: int, scale: float) -> torch.Tensor:
    """softmax(q k^T * scale) v straight from nn.MultiheadAttention's packed in-projection
    output (T, B, 3*E), E = heads*64, into the (T, B, E) layout the out-projection takes."""
    t, b, e, (qp, kp, vp), (sb, sh, st) = _packed_layout(qkv, heads)
    with torch.cuda.device(qkv.device):
        out = torch.empty((t, b, e), dtype=qkv.dtype, device=qkv.device)
        rc = rt.library().musc_attention_fwd_strided(
            qp, kp, vp, out.data_ptr(), rt.DTYPE_F32 if qkv.dtype == torch.float32 else rt.DTYPE_F16,
            b, heads, t, 64, sb, sh, st, e, 64, b * e, float(scale), rt.stream(qkv.device))
        rt.check(rc, 'musc_attention_fwd_strided')
    return out


def attention_weights_packed(qkv: torch.Tensor, heads: int, scale: float) -> torch.Tensor:
    """Head-averaged softmax(q k^T * scale), (B, T, T) fp32, from the packed (T, B, 3*E) tensor."""
    t, b, e, (qp, kp, _), (sb, sh, st) = _packed_layout(qkv, heads)
    lib = rt.library()
    need = ctypes.c_size_t()
    rt.check(lib.musc_attention_weights_workspace_bytes(b, heads, t, ctypes.byref(need)),
             'musc_attention_weights_workspace_bytes')
    with torch.cuda.device(qkv.device):
        out = torch.empty((b, t, t), dtype=torch.float32, device=qkv.device)
        ws = torch.empty(need.value, dtype=torch.uint8, device=qkv.device)
        rc = lib.musc_attention_weights_strided(qp, kp, rt.DTYPE_F32 if qkv.dtype == torch.float32 else rt.DTYPE_F16,
                                                b, heads, t, 64, sb, sh, st, float(scale), out.data_ptr(),
                                                ws.data_ptr(), need.value, rt.stream(qkv.device))
        rt.check(rc, 'musc_attention_weights_strided')
    return out
