"""Fused encoder-block layers on MI355X (libmusc_hip musc_layernorm_rows, musc_activation).

Reference: models/backbone/open_clip/transformer.py:23-29 (LayerNorm that casts back
to the input dtype), :32-35 (QuickGELU), :247-248 (residual adds around ln_2),
model.py:84-87 (QuickGELU for OpenAI weights, nn.GELU otherwise).  Each call is one
pass over the activations where torch's autocast path makes three (cast, normalise,
cast back; or 1.702 x, sigmoid, product).
"""
from __future__ import annotations

import torch

from . import _runtime as rt

_DTYPES = {torch.float32: rt.DTYPE_F32, torch.float16: rt.DTYPE_F16}


def _affine(p, width: int, device):
    if p is None:
        return None
    if p.numel() != width:
        raise ValueError('LayerNorm affine parameter does not match the row width')
    return p.detach().to(device=device, dtype=torch.float32).contiguous()


def layer_norm(x: torch.Tensor, weight, bias, eps: float, residual: torch.Tensor | None = None):
    """LayerNorm over the last dimension, fp32 statistics, output in x's dtype.

    With `residual`, returns (s, layer_norm(s)) where s = x + residual rounded to x's
    dtype (one pass for the residual add and the norm); otherwise layer_norm(x)."""
    rt.require_device_tensor(x, 'x')
    if x.dtype not in _DTYPES:
        raise ValueError('x must be float32 or float16')
    if residual is not None:
        rt.require_device_tensor(residual, 'residual')
        if residual.shape != x.shape or residual.dtype != x.dtype:
            raise ValueError('residual must match x in shape and dtype')
        residual = residual.contiguous()
    x = x.contiguous()
    width = x.shape[-1]
    rows = x.numel() // width if width else 0
    w, b = _affine(weight, width, x.device), _affine(bias, width, x.device)
    with torch.cuda.device(x.device):
        y = torch.empty_like(x)
        s = torch.empty_like(x) if residual is not None else None
        rc = rt.library().musc_layernorm_rows(
            x.data_ptr(), residual.data_ptr() if residual is not None else None,
            s.data_ptr() if s is not None else None, w.data_ptr() if w is not None else None,
            b.data_ptr() if b is not None else None, _DTYPES[x.dtype], rows, width, float(eps), y.data_ptr(),
            rt.stream(x.device))
        rt.check(rc, 'musc_layernorm_rows')
    return (s, y) if residual is not None else y


def supports_layer_norm(width: int, dtype: torch.dtype) -> bool:
    per = 8 if dtype == torch.float16 else 4
    return dtype in _DTYPES and width % per == 0 and (width // per + 63) // 64 <= 4


def activation_(x: torch.Tensor, mode: int) -> torch.Tensor:
    """In place: QuickGELU (mode rt.ACT_QUICK_GELU) or erf-GELU (rt.ACT_GELU)."""
    rt.require_device_tensor(x, 'x')
    if x.dtype not in _DTYPES or not x.is_contiguous():
        raise ValueError('x must be a contiguous float32 or float16 tensor')
    with torch.cuda.device(x.device):
        rc = rt.library().musc_activation(x.data_ptr(), x.data_ptr(), _DTYPES[x.dtype], int(mode), x.numel(),
                                          rt.stream(x.device))
        rt.check(rc, 'musc_activation')
    return x
