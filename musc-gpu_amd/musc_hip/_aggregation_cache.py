"""Per-division reuse of LayerNorm statistics across radii.

Mirrors models/modules/_aggregation_cache.py:8-58: the aggregation object is
created per category (`new_aggregation()`), called once per (radius, batch) and
cleared after each division (models/musc.py:274-275).  The reference memoises
the LayerNorm'd spatial tensor; here the HIP kernel re-reads the tokens anyway,
so only the per-(image, layer) {mean, rstd} statistics are kept (a few bytes per
image) and later radii skip the statistics pass (MUSC_LNAMD_STATS_READY).
Entries are keyed like the reference's: tensor identity, version counter,
data pointer, shape, stride, dtype and device; inference-mode tensors (no
version counter) are recomputed, never memoised.
"""
from __future__ import annotations

import torch

from . import _lnamd_hip as lh
from . import _runtime as rt


def _key(token: torch.Tensor):
    try:
        version = token._version
    except RuntimeError:
        return None
    return (id(token), version, token.data_ptr(), tuple(token.shape), tuple(token.stride()), token.dtype,
            token.device)


class RadiusAggregationCache:
    def __init__(self):
        self._stats = {}

    def clear(self):
        self._stats.clear()

    def __call__(self, layer, features: list[torch.Tensor], return_cpu: bool = True) -> torch.Tensor:
        if not lh.supported(layer, features):
            return layer._embed(features, return_cpu=return_cpu)
        keys = [_key(t) for t in features]
        key = tuple(keys) if all(k is not None for k in keys) else None
        entry = self._stats.get(key) if key is not None else None
        if entry is not None and all(a is b for a, b in zip(entry[0], features)):
            ws, ready = entry[1], True
        else:
            b = features[0].shape[0]
            ws, ready = rt.workspace(lh.workspace_bytes(b, len(features)), features[0].device), False
            if key is not None:
                self._stats[key] = (list(features), ws)
        out = lh.lnamd(features, [layer.r], layout='rbplc', stats_workspace=ws, stats_ready=ready)[0]
        return out.cpu() if return_cpu else out
