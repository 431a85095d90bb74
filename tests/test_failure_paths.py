"""Failure handling on the CPU: a missing or unloadable library fails loudly, the
backend selector reports the reason (models/modules/_backend.py:10-13 contract), and
library error codes become Python exceptions (models/modules/_cuda_runtime.py:47-55)."""
import importlib

import pytest
import torch


@pytest.fixture
def fresh_runtime(monkeypatch, tmp_path):
    from musc_hip import _runtime
    monkeypatch.setattr(_runtime, '_lib', None)
    yield _runtime


def test_missing_library_raises_and_selector_reports(fresh_runtime, monkeypatch, tmp_path):
    rt = fresh_runtime
    monkeypatch.setattr(rt, 'LIB_PATH', str(tmp_path / 'libmusc_hip.so'))
    with pytest.raises(rt.LibraryUnavailable, match='not found'):
        rt.library()
    ok, reason = rt.available()
    assert not ok and 'not found' in reason
    from musc_hip._backend import select_backend
    monkeypatch.setattr(torch.version, 'hip', '7.0')
    sel, why = select_backend('gpu', 'cuda')
    assert sel == 'original' and 'not found' in why


def test_unloadable_library_raises(fresh_runtime, monkeypatch, tmp_path):
    rt = fresh_runtime
    bad = tmp_path / 'libmusc_hip.so'
    bad.write_bytes(b'not an ELF file')
    monkeypatch.setattr(rt, 'LIB_PATH', str(bad))
    with pytest.raises(rt.LibraryUnavailable, match='cannot load'):
        rt.library()


def test_error_codes_map_to_exceptions():
    from musc_hip import _runtime as rt
    rt.check(0, 'ok')
    with pytest.raises(ValueError, match='invalid argument'):
        rt.check(rt.MUSC_ERR_INVALID_ARG, 'op')
    with pytest.raises(RuntimeError, match='workspace'):
        rt.check(rt.MUSC_ERR_WORKSPACE, 'op')
    with pytest.raises(RuntimeError, match='implemented range'):
        rt.check(rt.MUSC_ERR_UNSUPPORTED, 'op')


def test_product_entry_points_reject_cpu_tensors():
    # no silent CPU path: every entry point wants device tensors
    from musc_hip import _MSM_hip, _attention_hip, _epilogue_hip, _lnamd_hip
    with pytest.raises(ValueError):
        _MSM_hip.MSM(torch.zeros((8, 4, 4)))
    with pytest.raises(ValueError):
        _lnamd_hip.lnamd([torch.zeros((2, 26, 8))], [3])
    with pytest.raises(ValueError):
        _attention_hip.attention(*(torch.zeros((1, 4, 64)) for _ in range(3)), 0.125)
    with pytest.raises(ValueError):
        _epilogue_hip.maps_and_scores(torch.zeros((1, 1, 2, 25), dtype=torch.float64), 13)
    from musc_hip import _layers_hip, _super_fast, pipeline
    with pytest.raises(ValueError):
        pipeline.msm_all(torch.zeros((1, 1, 8, 4, 4)))
    with pytest.raises(ValueError):
        _super_fast.adaptive_pool(torch.zeros((2, 1369, 1, 8)))
    with pytest.raises(ValueError):
        _layers_hip.activation_(torch.zeros((4, 8)), 0)


def test_bench_refuses_several_gpus():
    import subprocess
    import sys
    from conftest import ROOT
    res = subprocess.run([sys.executable, 'bench.py', '--gpus', '2'], cwd=ROOT, capture_output=True, text=True,
                         timeout=120)
    assert res.returncode == 2 and 'one GPU only' in res.stderr
