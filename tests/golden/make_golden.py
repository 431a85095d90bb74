"""Write the small golden fixtures under tests/golden/ (run from the repo root).

    python tests/golden/make_golden.py

Every expected output comes from the float64 brute forces of the oracle
(explicit differences and loops, no torch), so the fixtures pin the torch-fp32
restatements and the HIP kernels independently of torch's own arithmetic.
The reference repository ships no golden vectors for this path; its one
numeric known-answer test (tools/test_super_fast.py:42-58, adaptive pooling of
an arange input 37x37 -> 28x28) is reproduced as `super_fast_pool.npz`.
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import epilogue as oe  # noqa: E402
from oracle import lnamd as ol  # noqa: E402
from oracle import msm as om  # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))


def unit_rows(x):
    return (x / np.linalg.norm(x, axis=-1, keepdims=True)).astype(np.float32)


def main():
    rng = np.random.default_rng(20240601)
    cases = {}
    for name, (n, p, c) in {'a': (6, 9, 8), 'b': (11, 30, 16), 'c': (7, 1, 5), 'd': (13, 20, 36)}.items():
        z = unit_rows(rng.standard_normal((n, p, c)))
        k_min, k_max = om.rank_window(n)
        cases[f'{name}_z'] = z
        cases[f'{name}_nearest'] = om.nearest_bruteforce_f64(z)
        cases[f'{name}_scores'] = om.msm_bruteforce_f64(z)
        cases[f'{name}_window'] = np.array([k_min, k_max])
    np.savez_compressed(os.path.join(OUT, 'msm_small.npz'), **cases)

    lcases = {}
    tokens = rng.standard_normal((2, 26, 8)).astype(np.float32)  # 1 class token + 5x5 grid
    tokens[:, 1:, :] += rng.standard_normal((1, 1, 8)).astype(np.float32)
    lcases['tokens'] = tokens
    for r in (1, 3, 5):
        lcases[f'r{r}'] = ol.lnamd_bruteforce_f64(tokens, r)
    np.savez_compressed(os.path.join(OUT, 'lnamd_small.npz'), **lcases)

    grid = rng.random((5, 5))
    np.savez_compressed(os.path.join(OUT, 'bilinear_small.npz'), grid=grid,
                        up13=oe.bilinear_align_corners_f64(grid, 13), up37=oe.bilinear_align_corners_f64(grid, 37))

    x = np.arange(37 * 37, dtype=np.float64).reshape(37, 37)
    np.savez_compressed(os.path.join(OUT, 'super_fast_pool.npz'), x=x,
                        pooled=ol.adaptive_pool_bruteforce_f64(x, 28))


if __name__ == '__main__':
    main()
    print('golden fixtures written to', OUT)
