"""The C-ABI library loads and exports what include/musc_hip.h declares (CPU only).

Only argument-validation paths are called here: each returns its error code
before any HIP call, so no GPU is touched.
"""
import ctypes
import os
import re

import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, 'include', 'musc_hip.h')


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r'/\*.*?\*/', '', text, flags=re.S)
    return sorted(set(re.findall(r'\b(musc_\w+)\s*\(', text)))


@pytest.fixture(scope='module')
def lib():
    from musc_hip import _runtime
    return _runtime.library()


def test_every_declared_symbol_is_exported(lib):
    names = declared_functions()
    assert 'musc_msm_scores_f32' in names and 'musc_lnamd_f32' in names
    for name in names:
        assert hasattr(lib, name), f'{name} declared in musc_hip.h but not exported'
    from musc_hip import _runtime
    assert set(names) == set(_runtime.SIGNATURES), 'ctypes signatures out of sync with the header'


def test_measurement_probes_live_in_their_own_library(lib):
    # the HBM probes are working tools: libmusc_measure.so exports what musc_measure.h
    # declares, and the product library exports none of it
    from musc_hip import build
    text = re.sub(r'/\*.*?\*/', '', open(os.path.join(ROOT, 'musc-gpu_amd', 'measure', 'musc_measure.h')).read(),
                  flags=re.S)
    names = sorted(set(re.findall(r'\b(musc_\w+)\s*\(', text)))
    assert names == ['musc_measure_hbm_stream', 'musc_measure_lnamd_pattern']
    probes = ctypes.CDLL(build.MEASURE_LIB)
    for name in names:
        assert hasattr(probes, name) and not hasattr(lib, name)
    assert not hasattr(lib, 'musc_calibrate_hbm_stream') and not hasattr(lib, 'musc_calibrate_lnamd_pattern')


def test_version_and_strerror(lib):
    assert lib.musc_version() >= 100
    assert b'invalid argument' in lib.musc_strerror(1001)
    assert b'workspace' in lib.musc_strerror(1002)
    assert b'implemented range' in lib.musc_strerror(1003)
    assert lib.musc_strerror(0) == b'success'


def test_msm_workspace_bytes(lib):
    out = ctypes.c_size_t()
    assert lib.musc_msm_workspace_bytes(83, 1369, 1024, ctypes.byref(out)) == 0
    rows = 83 * 1369
    align = lambda x: (x + 255) // 256 * 256  # noqa: E731
    # norms | epilogue scales | minima keys | refinement scales | per-image norm maxima
    assert out.value == 3 * align(rows * 4) + align(rows * 83 * 4) + align(83 * 4)
    assert lib.musc_msm_workspace_bytes(1, 10, 10, ctypes.byref(out)) == 1001


def test_msm_split_workspace_and_argument_errors(lib):
    align = lambda x: (x + 255) // 256 * 256  # noqa: E731
    out, base = ctypes.c_size_t(), ctypes.c_size_t()
    assert lib.musc_msm_split_workspace_bytes(83, 1369, 1024, ctypes.byref(out)) == 0
    assert lib.musc_msm_workspace_bytes(83, 1369, 1024, ctypes.byref(base)) == 0
    # the fp32 engine's workspace, then hi[16] | lo[16] fp16 (64 bytes) per row and 16-channel
    # block, the blocks padded to an even count (the pair kernel takes two stages per iteration)
    assert out.value == base.value + align(83 * 1369 * (1024 // 16) * 64)
    assert lib.musc_msm_split_workspace_bytes(5, 300, 33, ctypes.byref(out)) == 0
    assert lib.musc_msm_workspace_bytes(5, 300, 33, ctypes.byref(base)) == 0
    assert out.value == base.value + align(5 * 300 * 4 * 64)  # 33 channels -> 4 zero-padded blocks
    assert lib.musc_msm_split_workspace_bytes(1, 300, 16, ctypes.byref(out)) == 1001
    fake = ctypes.c_void_p(256)  # never dereferenced: validation fails first
    big = ctypes.c_size_t(1 << 40)
    assert lib.musc_msm_split_scores_f32(fake, 8, 300, 16, 2, 2, 0, fake, fake, big, None) == 1001  # empty window
    assert lib.musc_msm_split_scores_f32(fake, 8, 300, 16, 0, 2, 4, fake, fake, big, None) == 1001  # unknown flag
    assert lib.musc_msm_split_scores_f32(fake, 8, 100, 16, 0, 2, 0, fake, fake, big, None) == 1003  # p < 256
    assert lib.musc_msm_split_scores_f32(fake, 8, 300, 16, 0, 2, 0, fake, fake, ctypes.c_size_t(16), None) == 1002
    assert lib.musc_msm_split_prepare_f32(None, 8, 300, 16, 0, fake, big, None) == 1001
    assert lib.musc_msm_split_pair_minima(8, 300, 16, fake, ctypes.c_size_t(16), None) == 1002


def test_msm_argument_errors_before_any_launch(lib):
    fake = ctypes.c_void_p(256)  # never dereferenced: validation fails first
    big = ctypes.c_size_t(1 << 40)
    # empty rank window
    assert lib.musc_msm_scores_f32(fake, 8, 10, 16, 2, 2, fake, fake, big, None) == 1001
    # rank_hi beyond n-1
    assert lib.musc_msm_scores_f32(fake, 8, 10, 16, 0, 8, fake, fake, big, None) == 1001
    # n < 2
    assert lib.musc_msm_scores_f32(fake, 1, 10, 16, 0, 1, fake, fake, big, None) == 1001
    # workspace too small
    assert lib.musc_msm_scores_f32(fake, 8, 10, 16, 0, 2, fake, fake, 16, None) == 1002
    # null features
    assert lib.musc_msm_scores_f32(None, 8, 10, 16, 0, 2, fake, fake, big, None) == 1001
    # more images than the rank kernel stages
    assert lib.musc_msm_scores_f32(fake, 5000, 1, 16, 0, 2, fake, fake, big, None) == 1003


def test_msm_workspace_must_be_256_byte_aligned(lib):
    # every MSM entry point that takes a workspace rejects one that does not start on a
    # 256-byte boundary (its arrays are read with 16-byte loads and merged with atomics)
    fake, off = ctypes.c_void_p(256), ctypes.c_void_p(256 + 4)
    big = ctypes.c_size_t(1 << 40)
    assert lib.musc_msm_scores_f32(fake, 8, 10, 16, 0, 2, fake, off, big, None) == 1001
    assert lib.musc_msm_prepare_f32(fake, 8, 10, 16, 0, off, big, None) == 1001
    assert lib.musc_msm_pair_minima_f32(fake, 8, 10, 16, off, big, None) == 1001
    assert lib.musc_msm_refine_f32(fake, 8, 10, 16, off, big, None) == 1001
    assert lib.musc_msm_rank_f32(8, 10, 0, 2, fake, off, big, None) == 1001
    assert lib.musc_msm_nearest_f32(fake, 8, 10, 16, fake, off, big, None) == 1001
    assert lib.musc_msm_split_scores_f32(fake, 8, 300, 16, 0, 2, 0, fake, off, big, None) == 1001
    assert lib.musc_msm_split_prepare_f32(fake, 8, 300, 16, 0, off, big, None) == 1001
    assert lib.musc_msm_split_pair_minima(8, 300, 16, off, big, None) == 1001
    # the refinement validates like the other stages
    assert lib.musc_msm_refine_f32(None, 8, 10, 16, fake, big, None) == 1001
    assert lib.musc_msm_refine_f32(fake, 8, 10, 16, fake, ctypes.c_size_t(16), None) == 1002


def test_lnamd_argument_errors(lib):
    fake = ctypes.c_void_p(256)
    ptrs = (ctypes.c_void_p * 1)(256)
    radii = (ctypes.c_int * 1)(3)
    even = (ctypes.c_int * 1)(2)
    big = ctypes.c_size_t(1 << 40)
    out = ctypes.c_size_t()
    assert lib.musc_lnamd_workspace_bytes(4, 4, ctypes.byref(out)) == 0 and out.value > 0
    # non-square grid
    assert lib.musc_lnamd_f32(ptrs, 1, 0, 2, 27, 8, 1, radii, 1, 1e-5, 0, fake, 0, fake, big, None) == 1001
    # even radius
    assert lib.musc_lnamd_f32(ptrs, 1, 0, 2, 26, 8, 1, even, 1, 1e-5, 0, fake, 0, fake, big, None) == 1001
    # channels not a multiple of 4
    assert lib.musc_lnamd_f32(ptrs, 1, 0, 2, 26, 6, 1, radii, 1, 1e-5, 0, fake, 0, fake, big, None) == 1003
    # unknown flag
    assert lib.musc_lnamd_f32(ptrs, 1, 0, 2, 26, 8, 1, radii, 1, 1e-5, 8, fake, 0, fake, big, None) == 1001
    # workspace too small
    assert lib.musc_lnamd_f32(ptrs, 1, 0, 2, 26, 8, 1, radii, 1, 1e-5, 0, fake, 0, fake, 8, None) == 1002


def test_maps_and_attention_argument_errors(lib):
    fake = ctypes.c_void_p(256)
    assert lib.musc_maps_f64(fake, 1, 1, 2, 5, 13, None, None, None) == 1001
    assert lib.musc_maps_f64(fake, 1, 1, 2, 500, 13, fake, None, None) == 1003
    assert lib.musc_attention_fwd(fake, fake, fake, fake, 0, 4, 10, 32, 0.125, None) == 1003
    assert lib.musc_attention_fwd(fake, fake, fake, fake, 7, 4, 10, 64, 0.125, None) == 1001
    # a K/V row stride whose 32-row block spans 2 GiB or more exceeds the 32-bit buffer
    # extent (31 * 18e6 * 4 and 31 * 36e6 * 2 bytes are both above 2^31); only strides
    # that are rejected are passed here, so nothing is launched
    for dtype, st in ((0, 18_000_000), (1, 36_000_000)):
        assert (31 * st + 64) * (4 if dtype == 0 else 2) > 2**31
        assert lib.musc_attention_fwd_strided(fake, fake, fake, fake, dtype, 1, 1, 10, 64, 0, 0, st, 0, 0, 64,
                                              0.125, None) == 1003


def test_preprocess_workspace_and_argument_errors(lib):
    out = ctypes.c_size_t()
    assert lib.musc_preprocess_workspace_bytes(4, 1024, 1024, 518, 518, ctypes.byref(out)) == 0
    align = lambda x: (x + 255) // 256 * 256  # noqa: E731
    # two tables of 518 bounds + 518 coefficient rows; 9 taps are stored 12 wide (the widths
    # the kernels are instantiated for: 4, 8, 12, 16, 24, 32, 48, 64)
    tables = 2 * (align(518 * 8) + align(518 * 12 * 4))
    assert out.value == tables                          # fused kernel: the intermediate stays in LDS
    assert lib.musc_preprocess_workspace_bytes(4, 1022, 1022, 518, 518, ctypes.byref(out)) == 0
    assert out.value == tables + align(4 * 1022 * 518 * 3)   # in_w % 4 != 0: two passes through HBM
    assert lib.musc_preprocess_workspace_bytes(2, 518, 518, 518, 518, ctypes.byref(out)) == 0
    assert out.value == 2 * (align(518 * 8) + align(518 * 4 * 4))     # nothing resampled: no intermediate
    assert lib.musc_preprocess_workspace_bytes(0, 10, 10, 5, 5, ctypes.byref(out)) == 1001
    assert lib.musc_preprocess_workspace_bytes(1, 2000, 2000, 100, 100, ctypes.byref(out)) == 1003  # 20x: > 64 taps
    fake = ctypes.c_void_p(256)
    m = (ctypes.c_float * 3)(0.5, 0.5, 0.5)
    s0 = (ctypes.c_float * 3)(1.0, 0.0, 1.0)
    big = ctypes.c_size_t(1 << 40)
    assert lib.musc_preprocess_u8(None, 1, 10, 10, 5, 5, m, m, fake, fake, big, None) == 1001
    assert lib.musc_preprocess_u8(fake, 1, 10, 10, 5, 5, m, s0, fake, fake, big, None) == 1001   # zero std
    assert lib.musc_preprocess_u8(fake, 1, 10, 10, 5, 5, m, m, fake, fake, ctypes.c_size_t(8), None) == 1002
