"""The C-ABI from plain C: tests/capi_c/msm_from_c.c links libmusc_hip.so and the HIP
runtime (no Python, no torch), checks musc_msm_scores_f32 against a float64 brute force, the
four MSM stages called one by one and the no-allocation entry point against it bit for bit,
the split engine's P >= 256 rejection and the epilogue at identity size."""
import os
import subprocess

import pytest

from conftest import ROOT

pytestmark = pytest.mark.gpu


def test_msm_scores_from_c(tmp_path):
    src = os.path.join(ROOT, 'tests', 'capi_c', 'msm_from_c.c')
    libdir = os.path.join(ROOT, 'musc-gpu_amd', 'musc_hip')
    exe = str(tmp_path / 'msm_from_c')
    subprocess.run(['gcc', '-O2', '-std=c11', '-D__HIP_PLATFORM_AMD__', '-I', os.path.join(ROOT, 'include'),
                    '-I', '/opt/rocm/include', src, '-o', exe, '-L', libdir, '-l:libmusc_hip.so',
                    f'-Wl,-rpath,{libdir}', '-L', '/opt/rocm/lib', '-lamdhip64', '-Wl,-rpath,/opt/rocm/lib', '-lm'],
                   check=True, capture_output=True, text=True)
    res = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    print(res.stdout, res.stderr, flush=True)
    assert res.returncode == 0, res.stdout + res.stderr
    assert res.stdout.startswith('max_abs_err ')
