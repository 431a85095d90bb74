"""Backend selection: the reference's `inference_backend` plugin boundary.

Same signatures and return contract as models/modules/_backend.py:5-33:
`select_backend(requested, device_type, platform=None) -> (selected, reason)`
raises ValueError for unknown names and returns ('original', reason) when the
accelerated path is unavailable; `configure_backend(cfg, device_type)` returns
cfg itself or a deep-copied super_fast preset.

The accelerated path here is libmusc_hip on a ROCm GPU, so the reference's
Windows/NVRTC gate (:12-13) becomes "torch is a ROCm build, libmusc_hip.so loads
and the current device has the architecture its kernels are compiled for".
`platform` is accepted for signature compatibility and ignored.
"""
from __future__ import annotations

from copy import deepcopy

BACKENDS = ('original', 'gpu', 'super_fast')


def select_backend(requested, device_type, platform=None):
    if requested not in BACKENDS:
        raise ValueError('inference_backend must be original, gpu or super_fast')
    if requested == 'original':
        return 'original', None
    if device_type != 'cuda':
        return 'original', 'CUDA is unavailable'
    import torch
    if torch.version.hip is None:
        return 'original', 'the accelerated runtime requires a ROCm build of PyTorch'
    from . import _runtime
    ok, reason = _runtime.device_supported()
    if not ok:
        return 'original', reason
    return requested, None


def configure_backend(cfg, device_type, platform=None):
    """Apply the opt-in super_fast preset only when its accelerated path is available."""
    requested = cfg['models'].get('inference_backend', 'original')
    selected, _ = select_backend(requested, device_type, platform)
    if selected != 'super_fast':
        return cfg
    models = cfg['models']
    datasets = cfg['datasets']
    if (models['backbone_name'] != 'ViT-L-14-336' or models['pretrained'] != 'openai'
            or datasets['img_resize'] != 518 or models['batch_size'] != 4
            or datasets['divide_num'] != 1):
        raise ValueError('super_fast requires ViT-L-14-336/openai, img_resize=518, '
                         'batch_size=4 and divide_num=1; use gpu for other configurations')
    result = deepcopy(cfg)
    result['models']['feature_layers'] = [5]
    result['models']['r_list'] = [3]
    return result
