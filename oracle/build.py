"""Build the C restatement of the oracle (test infrastructure only).

    python oracle/build.py            -> oracle/_build/libmsm_oracle.so

Plain gcc, no -march flags, so the library runs on any x86-64 host (the GPU
box's CPU may differ from the build container's).
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
OUT_DIR = os.path.join(HERE, '_build')
LIB = os.path.join(OUT_DIR, 'libmsm_oracle.so')


def build(verbose: bool = False) -> str:
    os.makedirs(OUT_DIR, exist_ok=True)
    cmd = ['gcc', '-O3', '-fopenmp', '-ffp-contract=off', '-shared', '-fPIC',
           os.path.join(HERE, 'msm_f64.c'), '-o', LIB + '.tmp', '-lm']
    if verbose:
        print(' '.join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(LIB + '.tmp', LIB)
    return LIB


if __name__ == '__main__':
    print(build(verbose='-v' in sys.argv))
