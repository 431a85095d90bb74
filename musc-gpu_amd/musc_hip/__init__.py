"""musc_hip -- MI355X (gfx950) implementation of MuSc's data-parallel hot path.

Host-side mirror of the reference's plugin interface (DylanMartinLSC/musc-gpu,
models/modules/): every compute call goes to libmusc_hip.so (C-ABI in
include/musc_hip.h); nothing here computes on the CPU.

  _backend.select_backend / configure_backend   the inference_backend selector
  _MSM_hip.MSM                                  the `scoring` plugin
  _lnamd_hip.aggregate_features, LNAMD          the `aggregation` plugin (+ multi-radius lnamd)
  _aggregation_cache.RadiusAggregationCache     per-division statistics reuse
  _epilogue_hip.maps_and_scores                 layer/radius means, upsampling, image scores
  pipeline.score_pool                           tokens -> maps + image scores, fused
"""
from ._backend import configure_backend, select_backend  # noqa: F401

__version__ = '0.1.0'
