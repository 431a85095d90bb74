"""RsCIN image-score refinement on MI355X (libmusc_hip musc_rscin_f32).

Same call contract as models/modules/_RsCIN.py:23-32 (used at models/musc.py:290-296):
`RsCIN(scores_old, cls_tokens=None, k_list=[0])` returns `scores_old` unchanged when
there are no class tokens or 0 is in k_list, otherwise the refined fp32 scores.
Inputs may be numpy (as at the reference call site; they are copied to the GPU
and the result copied back as numpy) or GPU tensors (result stays on the GPU).
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import _runtime as rt


def RsCIN(scores_old, cls_tokens=None, k_list=(0,)):
    k_list = list(k_list)
    if cls_tokens is None or 0 in k_list:
        return scores_old
    as_numpy = not isinstance(scores_old, torch.Tensor)
    if as_numpy:
        dev = torch.device('cuda', torch.cuda.current_device())
        scores = torch.as_tensor(np.asarray(scores_old, dtype=np.float64)).to(dev)
        cls = torch.as_tensor(np.asarray(cls_tokens, dtype=np.float32)).to(dev)
    else:
        scores = scores_old.to(torch.float64)
        cls = cls_tokens if isinstance(cls_tokens, torch.Tensor) else torch.as_tensor(
            np.asarray(cls_tokens, dtype=np.float32), device=scores.device)
        cls = cls.to(scores.device, torch.float32)
    rt.require_device_tensor(scores, 'scores')
    scores, cls = scores.contiguous(), cls.contiguous()
    n, d = cls.shape
    if scores.shape != (n,):
        raise ValueError('one score per class token is required')
    with torch.cuda.device(scores.device):
        out = torch.empty((n,), dtype=torch.float32, device=scores.device)
        ks = (ctypes.c_int * len(k_list))(*[int(k) for k in k_list])
        rc = rt.library().musc_rscin_f32(cls.data_ptr(), scores.data_ptr(), n, d, ctypes.cast(ks, ctypes.c_void_p),
                                         len(k_list), out.data_ptr(), rt.stream(scores.device))
        rt.check(rc, 'musc_rscin_f32')
    return out.cpu().numpy() if as_numpy else out
