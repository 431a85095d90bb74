"""LNAMD aggregation on MI355X (libmusc_hip musc_lnamd_f32).

`lnamd(tokens, radii, ...)` is the multi-radius primitive: one read of the
layer tokens produces every requested radius.  The reference computes one radius
per call (models/modules/_LNAMD.py:72-129, models/modules/_encoder_gpu.py:14-42);
`aggregate_features` below keeps that per-radius plugin contract on top of it.

`LNAMD` mirrors the attributes of the reference module that the aggregation
plugin reads (`r`, `patch_maker.stride`, `LNA.output_dim`,
`LNA.preprocessing_modules`; _encoder_gpu.py:18-21).  Its `_embed` runs the HIP
kernel; there is no torch/CPU implementation in this package.
"""
from __future__ import annotations

import ctypes
import math
from types import SimpleNamespace

import torch

from . import _runtime as rt

_LAYOUTS = {'rbplc': rt.LAYOUT_RBPLC, 'rlbpc': rt.LAYOUT_RLBPC}


def workspace_bytes(batch: int, n_layers: int) -> int:
    out = ctypes.c_size_t()
    rt.check(rt.library().musc_lnamd_workspace_bytes(batch, n_layers, ctypes.byref(out)), 'musc_lnamd_workspace_bytes')
    return out.value


def _check_tokens(tokens: list[torch.Tensor]) -> tuple[int, int, int, torch.dtype]:
    if not tokens:
        raise ValueError('LNAMD needs at least one layer of tokens')
    first = tokens[0]
    if first.ndim != 3:
        raise ValueError('tokens must be (B, T, C)')
    for t in tokens:
        rt.require_device_tensor(t, 'tokens')
        if t.shape != first.shape or t.dtype != first.dtype or t.device != first.device:
            raise ValueError('all layers must share shape, dtype and device')
    if first.dtype not in (torch.float32, torch.float16):
        raise ValueError('tokens must be float32 or float16')
    b, t, c = first.shape
    return b, t, c, first.dtype


def lnamd(tokens: list[torch.Tensor], radii: list[int], *, l2norm: bool = False, layout: str = 'rbplc',
          has_cls: bool = True, eps: float = 1e-5, stats_workspace: torch.Tensor | None = None,
          stats_ready: bool = False, raw_sums: bool = False, pool_side: int | None = None) -> torch.Tensor:
    """LayerNorm over (C, H, W) + r x r zero-padded box mean for every radius.

    tokens  list of L tensors (B, T, C) (T = 1 + side*side when has_cls).
    Returns fp32:
      layout 'rbplc' -> (R, B, P, L, C)  (each [r] is the plugin's (B, P, L, C) return)
      layout 'rlbpc' -> (R, L, B, P, C)  (each [r, l] is a contiguous MSM pool)
    l2norm   also divides every patch by its L2 norm (models/musc.py:238).
    raw_sums writes the window sums of (x - mean) without the LayerNorm scale and
             the 1/r^2 (the input of an L2-normalising consumer, where they cancel).
    stats_workspace / stats_ready  reuse LayerNorm statistics computed by an
             earlier call on the same tokens (another radius).
    pool_side  adaptively average-pool the side x side grid of outputs to
             pool_side x pool_side in the same pass (F.adaptive_avg_pool2d windows;
             the super_fast 37 -> 28 step); P becomes pool_side**2.  With raw_sums
             the pooled values are plain sums (no division by the window count).
    """
    b, t, c, dtype = _check_tokens(tokens)
    side = math.isqrt(t - int(has_cls))
    if side * side != t - int(has_cls):
        raise ValueError('token count must be a square grid (plus the class token)')
    radii = [int(r) for r in radii]
    n_layers = len(tokens)
    if pool_side is not None and not (1 <= int(pool_side) <= side):
        raise ValueError(f'pool_side must lie in [1, {side}]')
    if pool_side is not None and l2norm and int(pool_side) != side:
        raise ValueError('pooling and the fused L2 normalisation cannot be combined')
    p = side * side if pool_side is None else int(pool_side) ** 2
    dev = tokens[0].device
    shape = (len(radii), b, p, n_layers, c) if layout == 'rbplc' else (len(radii), n_layers, b, p, c)
    toks = [x.contiguous() for x in tokens]
    with torch.cuda.device(dev):
        out = torch.empty(shape, dtype=torch.float32, device=dev)
        need = workspace_bytes(b, n_layers)
        ws = stats_workspace if stats_workspace is not None else rt.workspace(need, dev)
        if ws.numel() < need:
            raise ValueError('stats workspace too small')
        ptrs = (ctypes.c_void_p * n_layers)(*[x.data_ptr() for x in toks])
        rad = (ctypes.c_int * len(radii))(*radii)
        flags = ((rt.LNAMD_L2NORM if l2norm else 0) | (rt.LNAMD_STATS_READY if stats_ready else 0)
                 | (rt.LNAMD_RAW_SUMS if raw_sums else 0))
        in_dtype = rt.DTYPE_F32 if dtype == torch.float32 else rt.DTYPE_F16
        if pool_side is None:
            rc = rt.library().musc_lnamd_f32(ctypes.cast(ptrs, ctypes.c_void_p), n_layers, in_dtype,
                                             b, t, c, int(has_cls), ctypes.cast(rad, ctypes.c_void_p), len(radii),
                                             float(eps), flags, out.data_ptr(), _LAYOUTS[layout], ws.data_ptr(),
                                             ws.numel(), rt.stream(dev))
            rt.check(rc, 'musc_lnamd_f32')
        else:
            rc = rt.library().musc_lnamd_pooled_f32(ctypes.cast(ptrs, ctypes.c_void_p), n_layers, in_dtype,
                                                    b, t, c, int(has_cls), ctypes.cast(rad, ctypes.c_void_p),
                                                    len(radii), float(eps), flags, int(pool_side), out.data_ptr(),
                                                    _LAYOUTS[layout], ws.data_ptr(), ws.numel(), rt.stream(dev))
            rt.check(rc, 'musc_lnamd_pooled_f32')
    return out


# Limits of musc_lnamd_f32 itself (include/musc_hip.h): fp32/fp16 tokens on a ROCm
# device, 4 <= C <= 4096 with C % 4 == 0, at most 16 layers, a grid side of 1..1024.
MAX_LAYERS = 16
MAX_CHANNELS = 4096
MAX_SIDE = 1024


def supported(layer, features: list[torch.Tensor]) -> bool:
    """The reference's fast-path predicate (_encoder_gpu.py:18-21, _aggregation_cache.py:19-23),
    narrowed by the kernel's own limits, so that every input the kernel would reject
    takes layer._embed as in the reference instead of raising."""
    first = features[0]
    batch, length, channels = first.shape
    side = math.isqrt(length - 1)
    if (side * side != length - 1 or layer.patch_maker.stride != 1
            or layer.r not in (1, 3, 5) or layer.LNA.output_dim != channels
            or len(features) != len(layer.LNA.preprocessing_modules)
            or any(t.shape != first.shape or t.dtype != first.dtype or t.device != first.device
                   for t in features)):
        return False
    return (first.dtype in (torch.float32, torch.float16) and first.is_cuda and torch.version.hip is not None
            and batch >= 1 and 4 <= channels <= MAX_CHANNELS and channels % 4 == 0
            and 1 <= len(features) <= MAX_LAYERS and 1 <= side <= MAX_SIDE)


class LNAMD:
    """Descriptor with the reference LNAMD module's attributes (_LNAMD.py:63-70)."""

    def __init__(self, device=None, feature_dim: int = 1024, feature_layer=(1, 2, 3, 4), r: int = 3,
                 patchstride: int = 1):
        self.device = device
        self.r = r
        self.patch_maker = SimpleNamespace(patchsize=r, stride=patchstride)
        self.LNA = SimpleNamespace(output_dim=feature_dim,
                                   preprocessing_modules=[None] * len(list(feature_layer)))

    def _embed(self, features: list[torch.Tensor], return_cpu: bool = True) -> torch.Tensor:
        if self.patch_maker.stride != 1:
            raise ValueError('musc_hip LNAMD supports patch stride 1 only')
        out = lnamd(features, [self.r], layout='rbplc')[0]
        return out.cpu() if return_cpu else out


def aggregate_features(layer, features: list[torch.Tensor], return_cpu: bool = True) -> torch.Tensor:
    """Aggregation plugin: (B, P, L, C) fp32 for radius layer.r (_encoder_gpu.py:14-42)."""
    if not supported(layer, features):
        return layer._embed(features, return_cpu=return_cpu)
    out = lnamd(features, [layer.r], layout='rbplc')[0]
    return out.cpu() if return_cpu else out
