"""CPU oracle for MuSc's hot path -- TEST INFRASTRUCTURE ONLY.

Restatements of the reference algorithm (DylanMartinLSC/musc-gpu) used as the
checker by tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg.
Nothing in the product package (musc-gpu_amd/musc_hip) imports this package.

Modules
  msm.py       torch-fp32 restatement of models/modules/_MSM.py + float64 brute force
  msm_f64.c    float64 brute force in C (oracle/_build/libmsm_oracle.so)
  lnamd.py     LNAMD._embed restatement, layer_norm+avg_pool2d identity, brute force
  epilogue.py  models/musc.py:247-288 restatement + float64 bilinear brute force
  attention.py float64 softmax attention
"""
import ctypes
import os

_LIB = None


def c_oracle():
    """ctypes handle of the C brute force (built by oracle/build.py)."""
    global _LIB
    if _LIB is None:
        path = os.path.join(os.path.dirname(os.path.abspath(__file__)), '_build', 'libmsm_oracle.so')
        if not os.path.exists(path):
            from oracle.build import build
            build()
        lib = ctypes.CDLL(path)
        fp, ip, dp = ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p
        lib.msm_nearest_f64.argtypes = [fp, ip, ip, ip, dp]
        lib.msm_scores_f64.argtypes = [fp, ip, ip, ip, ip, ip, dp]
        lib.msm_scores_from_nearest_f64.argtypes = [dp, ip, ip, ip, ip, dp]
        lib.msm_nearest_rows_f64.argtypes = [fp, ip, ip, ip, dp, ip, dp]
        _LIB = lib
    return _LIB


def msm_scores_f64_c(z, a, b):
    """float64 scores (N, P) of a float32 numpy array z (N, P, C) via the C brute force."""
    import numpy as np
    z = np.ascontiguousarray(z, dtype=np.float32)
    n, p, c = z.shape
    out = np.empty((n, p), dtype=np.float64)
    rc = c_oracle().msm_scores_f64(z.ctypes.data, n, p, c, a, b, out.ctypes.data)
    if rc:
        raise RuntimeError(f'msm_scores_f64 failed with code {rc}')
    return out


def msm_nearest_f64_c(z):
    import numpy as np
    z = np.ascontiguousarray(z, dtype=np.float32)
    n, p, c = z.shape
    out = np.empty((n * p, n), dtype=np.float64)
    rc = c_oracle().msm_nearest_f64(z.ctypes.data, n, p, c, out.ctypes.data)
    if rc:
        raise RuntimeError(f'msm_nearest_f64 failed with code {rc}')
    return out


def msm_row_scores_f64_c(z, rows, a, b):
    """float64 scores of selected global rows (i*p + q) of a float32 numpy array z (N, P, C),
    from the C brute force over those rows only: (len(rows),) float64."""
    import numpy as np
    z = np.ascontiguousarray(z, dtype=np.float32)
    n, p, c = z.shape
    idx = np.ascontiguousarray(rows, dtype=np.int64)
    near = np.empty((len(idx), n), dtype=np.float64)
    rc = c_oracle().msm_nearest_rows_f64(z.ctypes.data, n, p, c, idx.ctypes.data, len(idx), near.ctypes.data)
    if rc:
        raise RuntimeError(f'msm_nearest_rows_f64 failed with code {rc}')
    out = np.empty(len(idx))
    for k, row in enumerate(idx):
        vals = np.sort(np.delete(near[k], int(row) // p))        # NaN sorts last, as in torch.topk
        out[k] = vals[a:b].mean()
    return out
