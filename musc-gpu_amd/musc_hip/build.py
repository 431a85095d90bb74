"""Build libmusc_hip.so for gfx950 from musc-gpu_amd/csrc/*.hip.

    python musc-gpu_amd/musc_hip/build.py [-v]

Every .hip file under csrc/ is compiled to its own object (in parallel), then
linked into musc-gpu_amd/musc_hip/libmusc_hip.so, the product library.  The HBM
measurement probes under measure/ are linked into their own library,
musc-gpu_amd/measure/libmusc_measure.so, which only kernels_bench.py loads.  Both
are built in-tree so that they travel with the source tree to the GPU host.
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(ROOT, 'csrc')
MEASURE = os.path.join(ROOT, 'measure')
BUILD = os.path.join(ROOT, '_build')
LIB = os.path.join(PKG, 'libmusc_hip.so')
MEASURE_LIB = os.path.join(MEASURE, 'libmusc_measure.so')
ARCH = os.environ.get('MUSC_OFFLOAD_ARCH', 'gfx950')
HIPCC = os.environ.get('HIPCC', '/opt/rocm/bin/hipcc')

# Packed FP32 instructions are disabled for all device code (they are emitted by
# the compiler from ordinary float code otherwise).
DEVICE_FLAGS = ['-Xclang', '-target-feature', '-Xclang', '-packed-fp32-ops']
COMMON = ['-O3', '-std=c++17', '-fPIC', f'--offload-arch={ARCH}', f'-DMUSC_TARGET_ARCH="{ARCH}"', '-Wall',
          '-Wno-unused-function', '-Wno-unused-variable', '-Wno-unused-but-set-variable'] + DEVICE_FLAGS


# Per-file device flags.  attention.hip: the online softmax rescales the MFMA
# accumulators with VALU instructions, so they must live in VGPRs; left to its
# heuristics the compiler puts them in AGPRs and moves every value back and forth
# (157 v_accvgpr moves per 32-key block in the fp16 kernel).
FILE_FLAGS = {'attention.hip': ['-mllvm', '-amdgpu-mfma-vgpr-form']}


def _compile(src: str, verbose: bool) -> str:
    obj = os.path.join(BUILD, os.path.basename(src) + '.o')
    cmd = [HIPCC] + COMMON + FILE_FLAGS.get(os.path.basename(src), []) + ['-c', src, '-o', obj]
    if verbose:
        print(' '.join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = 'packed-fp32-ops'
    err = '\n'.join(line for line in res.stderr.splitlines() if noise not in line)
    if res.returncode != 0:
        raise RuntimeError(f'hipcc failed for {src}:\n{err}')
    if err.strip() and verbose:
        print(err, flush=True)
    return obj


def _link(objs: list[str], lib: str, verbose: bool) -> None:
    tmp = lib + '.tmp'
    cmd = [HIPCC, '-shared', '-fPIC', f'--offload-arch={ARCH}', '-o', tmp] + objs
    if verbose:
        print(' '.join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, lib)


def build(verbose: bool = False) -> str:
    """Build libmusc_hip.so and libmusc_measure.so; returns the product library's path."""
    os.makedirs(BUILD, exist_ok=True)
    sources = sorted(glob.glob(os.path.join(CSRC, '*.hip')))
    probes = sorted(glob.glob(os.path.join(MEASURE, '*.hip')))
    if not sources:
        raise RuntimeError(f'no HIP sources under {CSRC}')
    with cf.ThreadPoolExecutor(max_workers=min(8, len(sources) + len(probes))) as ex:
        objs = list(ex.map(lambda s: _compile(s, verbose), sources + probes))
    _link(objs[:len(sources)], LIB, verbose)
    if probes:
        _link(objs[len(sources):], MEASURE_LIB, verbose)
    return LIB


if __name__ == '__main__':
    print(build(verbose='-v' in sys.argv))
