"""Backend selection: the reference's `inference_backend` plugin boundary.

Same signatures and return contract as models/modules/_backend.py:5-33:
`select_backend(requested, device_type, platform=None) -> (selected, reason)`
raises ValueError for unknown names and returns ('original', reason) when the
accelerated path is unavailable; `configure_backend(cfg, device_type)` returns
cfg itself or a deep-copied super_fast preset.

The accelerated path here is libmusc_hip on a ROCm GPU, so the reference's
Windows/NVRTC gate (:12-13) becomes "torch is a ROCm build, libmusc_hip.so loads,
a device is visible and it has the architecture the kernels are compiled for".
Like the reference's selector (:1, "no model loading or CUDA calls"), this one
starts no GPU runtime: the architecture is compared here only when torch has
already initialised HIP; otherwise the first launch on each device compares it
(musc_hip._runtime.stream) and raises RuntimeError on a mismatch.
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
    ok, reason = _runtime.available()
    if ok:
        if torch.cuda.is_initialized():
            ok, reason = _runtime.device_supported()
        elif torch.cuda.device_count() == 0:      # counts devices without starting HIP
            ok, reason = False, 'no ROCm device is visible'
    if not ok:
        return 'original', reason
    return requested, None


# The one configuration the super_fast preset was validated on, as (section, key, value), and
# the settings the preset replaces (models/modules/_backend.py:24-33).
_SUPER_FAST_REQUIRES = (
    ('models', 'backbone_name', 'ViT-L-14-336'),
    ('models', 'pretrained', 'openai'),
    ('datasets', 'img_resize', 518),
    ('models', 'batch_size', 4),
    ('datasets', 'divide_num', 1),
)
_SUPER_FAST_PRESET = (('models', 'feature_layers', [5]), ('models', 'r_list', [3]))
_SUPER_FAST_MISMATCH = ('super_fast requires ViT-L-14-336/openai, img_resize=518, '
                        'batch_size=4 and divide_num=1; use gpu for other configurations')


def configure_backend(cfg, device_type, platform=None):
    """Apply the opt-in super_fast preset only when its accelerated path is available.

    Returns `cfg` itself unless super_fast is selected; then checks every required setting
    (ValueError with the reference's message on a mismatch) and returns a deep copy with the
    preset's layer and aggregation-degree lists, leaving `cfg` untouched.
    """
    requested = cfg['models'].get('inference_backend', 'original')
    if select_backend(requested, device_type, platform)[0] != 'super_fast':
        return cfg
    if any(cfg[section][key] != value for section, key, value in _SUPER_FAST_REQUIRES):
        raise ValueError(_SUPER_FAST_MISMATCH)
    result = deepcopy(cfg)
    for section, key, value in _SUPER_FAST_PRESET:
        result[section][key] = list(value)
    return result
