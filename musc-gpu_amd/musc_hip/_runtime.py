"""ctypes binding of libmusc_hip.so (the C-ABI declared in include/musc_hip.h).

Plays the role of the reference's native bridge models/modules/_cuda_runtime.py:
  * `library()` loads the prebuilt gfx950 library once (the reference compiles
    CUDA C with NVRTC at first use, :58-92; here the code object is built ahead
    of time by musc_hip/build.py).
  * `check(rc, op)` turns a nonzero return code into RuntimeError with the
    library's message, as `_check` does for CUresult (:47-55).
  * `stream(device)` is torch's current HIP stream, the stream the reference
    launches on (:95-100).

There is no fallback: if the library is missing or fails to load, every entry
point raises.  torch is imported first so that the HIP runtime torch ships
(libamdhip64.so.7) is the one the library binds to.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), 'libmusc_hip.so')

MUSC_OK = 0
MUSC_ERR_INVALID_ARG = 1001
MUSC_ERR_WORKSPACE = 1002
MUSC_ERR_UNSUPPORTED = 1003
MUSC_ERR_SCRATCH_LIMIT = 1004

DTYPE_F32 = 0
DTYPE_F16 = 1
ACT_QUICK_GELU = 0
ACT_GELU = 1
LAYOUT_RBPLC = 0
LAYOUT_RLBPC = 1
LNAMD_L2NORM = 1
LNAMD_STATS_READY = 2
LNAMD_RAW_SUMS = 4
MSM_NORMALIZE_ROWS = 1

# Every symbol include/musc_hip.h declares, with its ctypes signature.
_vp, _i, _f, _sz, _ll = ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_size_t, ctypes.c_longlong
SIGNATURES = {
    'musc_strerror': (ctypes.c_char_p, [_i]),
    'musc_version': (_i, []),
    'musc_target_arch': (ctypes.c_char_p, []),
    'musc_msm_workspace_bytes': (_i, [_i, _i, _i, ctypes.POINTER(_sz)]),
    'musc_msm_scores_f32': (_i, [_vp, _i, _i, _i, _i, _i, _vp, _vp, _sz, _vp]),
    'musc_msm_scores_f32_noalloc': (_i, [_vp, _i, _i, _i, _i, _i, _vp, _vp]),
    'musc_msm_nearest_f32': (_i, [_vp, _i, _i, _i, _vp, _vp, _sz, _vp]),
    'musc_msm_prepare_f32': (_i, [_vp, _i, _i, _i, _i, _vp, _sz, _vp]),
    'musc_msm_pair_minima_f32': (_i, [_vp, _i, _i, _i, _vp, _sz, _vp]),
    'musc_msm_refine_f32': (_i, [_vp, _i, _i, _i, _vp, _sz, _vp]),
    'musc_msm_rank_f32': (_i, [_i, _i, _i, _i, _vp, _vp, _sz, _vp]),
    'musc_msm_split_workspace_bytes': (_i, [_i, _i, _i, ctypes.POINTER(_sz)]),
    'musc_msm_split_prepare_f32': (_i, [_vp, _i, _i, _i, _i, _vp, _sz, _vp]),
    'musc_msm_split_pair_minima': (_i, [_i, _i, _i, _vp, _sz, _vp]),
    'musc_msm_split_scores_f32': (_i, [_vp, _i, _i, _i, _i, _i, _i, _vp, _vp, _sz, _vp]),
    'musc_lnamd_workspace_bytes': (_i, [_i, _i, ctypes.POINTER(_sz)]),
    'musc_lnamd_f32': (_i, [_vp, _i, _i, _i, _i, _i, _i, _vp, _i, _f, _i, _vp, _i, _vp, _sz, _vp]),
    'musc_lnamd_pooled_f32': (_i, [_vp, _i, _i, _i, _i, _i, _i, _vp, _i, _f, _i, _i, _vp, _i, _vp, _sz, _vp]),
    'musc_maps_f64': (_i, [_vp, _i, _i, _i, _i, _i, _vp, _vp, _vp]),
    'musc_adaptive_pool_f32': (_i, [_vp, _i, _i, _i, _i, _vp, _vp]),
    'musc_rscin_f32': (_i, [_vp, _vp, _i, _i, _vp, _i, _vp, _vp]),
    'musc_preprocess_workspace_bytes': (_i, [_i, _i, _i, _i, _i, ctypes.POINTER(_sz)]),
    'musc_preprocess_u8': (_i, [_vp, _i, _i, _i, _i, _i, _vp, _vp, _vp, _vp, _sz, _vp]),
    'musc_attention_fwd': (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _f, _vp]),
    'musc_attention_weights_workspace_bytes': (_i, [_i, _i, _i, ctypes.POINTER(_sz)]),
    'musc_attention_weights': (_i, [_vp, _vp, _i, _i, _i, _i, _i, _f, _vp, _vp, _sz, _vp]),
    'musc_attention_fwd_strided': (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _ll, _ll, _ll, _ll, _ll, _ll, _f, _vp]),
    'musc_attention_weights_strided': (_i, [_vp, _vp, _i, _i, _i, _i, _i, _ll, _ll, _ll, _f, _vp, _vp, _sz, _vp]),
    'musc_layernorm_rows': (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _f, _vp, _vp]),
    'musc_activation': (_i, [_vp, _vp, _i, _i, _ll, _vp]),
    'musc_calibrate_mfma_f32': (_i, [_vp, _i, _i, ctypes.POINTER(ctypes.c_double), _vp]),
    'musc_calibrate_mfma_f16': (_i, [_vp, _i, _i, ctypes.POINTER(ctypes.c_double), _vp]),
}

_lock = threading.Lock()
_lib = None
_load_error: str | None = None


class LibraryUnavailable(RuntimeError):
    """libmusc_hip.so is missing or cannot be loaded; there is no fallback path."""


def library() -> ctypes.CDLL:
    global _lib, _load_error
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            _load_error = f'{LIB_PATH} not found; build it with musc-gpu_amd/musc_hip/build.py'
            raise LibraryUnavailable(_load_error)
        try:
            lib = ctypes.CDLL(LIB_PATH)
        except OSError as exc:  # wrong arch / missing HIP runtime
            _load_error = f'cannot load {LIB_PATH}: {exc}'
            raise LibraryUnavailable(_load_error) from exc
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
        return _lib


def available() -> tuple[bool, str | None]:
    """(True, None) if the library loads, else (False, reason)."""
    try:
        library()
        return True, None
    except LibraryUnavailable as exc:
        return False, str(exc)


def target_arch() -> str:
    """The architecture libmusc_hip.so's kernels are compiled for (e.g. 'gfx950')."""
    return library().musc_target_arch().decode()


def device_supported(device=None) -> tuple[bool, str | None]:
    """(True, None) if the kernels can run on `device` (default: the current one).

    Compares the device's architecture name (gcnArchName up to the first ':') with
    the library's target; a mismatch would otherwise surface as an invalid-device-
    function error at the first launch.
    """
    ok, reason = available()
    if not ok:
        return False, reason
    if not torch.cuda.is_available():
        return False, 'no ROCm device is visible'
    index = torch.cuda.current_device() if device is None else torch.device(device).index
    if index is None:
        index = torch.cuda.current_device()
    arch = str(getattr(torch.cuda.get_device_properties(index), 'gcnArchName', '')).split(':')[0]
    want = target_arch()
    if arch != want:
        return False, f'libmusc_hip.so is built for {want}; device {index} is {arch or "of unknown architecture"}'
    return True, None


def strerror(rc: int) -> str:
    return library().musc_strerror(rc).decode()


def check(rc: int, op: str) -> None:
    if rc == MUSC_OK:
        return
    msg = f'{op}: {strerror(rc)} (code {rc})'
    if rc in (MUSC_ERR_INVALID_ARG,):
        raise ValueError(msg)
    raise RuntimeError(msg)


_supported_devices: set[int] = set()


def stream(device: torch.device | int | None = None) -> int:
    """torch's current stream on `device`, as the handle the C-ABI takes.  The first call
    for a device checks its architecture against the library's (device_supported) and
    raises RuntimeError on a mismatch: every launch of this package passes through here,
    so a device the selector did not examine (it makes no GPU calls before the HIP
    runtime is up) fails loudly at its first launch instead of faulting."""
    s = torch.cuda.current_stream(device)
    index = s.device_index
    if index not in _supported_devices:
        ok, reason = device_supported(index)
        if not ok:
            raise RuntimeError(reason)
        _supported_devices.add(index)
    return s.cuda_stream


def require_device_tensor(t: torch.Tensor, name: str) -> None:
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise ValueError(f'{name} must be a GPU tensor')
    if torch.version.hip is None:
        raise RuntimeError('musc_hip requires a ROCm build of PyTorch')


def workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    """Caller-owned workspace from torch's caching allocator (256-byte aligned)."""
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)
