"""bench.py's host-side pieces (CPU only): the roofline traffic figure belongs to the kernel
that is built now."""
import importlib.util
import os

from conftest import ROOT


def _bench():
    spec = importlib.util.spec_from_file_location('bench', os.path.join(ROOT, 'bench.py'))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_traffic_profile_matches_the_pair_kernel_sources():
    # profiles/msm_lnamd_hbm_traffic_config2.md records the digest of what msm_pair_min_kernel
    # was compiled from when its HBM traffic was measured; a change to those files needs a new
    # measurement, or bench.py would report traffic: null
    bench = _bench()
    t = bench.profiled_traffic('pool')
    assert t['bytes'] is not None, t
    assert 1e10 < t['bytes'] < 1e12
    assert bench.profiled_traffic('plumbing')['bytes'] is None


def test_traffic_is_withheld_for_other_sources(monkeypatch):
    bench = _bench()
    monkeypatch.setattr(bench, 'pair_kernel_source_digest', lambda: '0' * 64)
    t = bench.profiled_traffic('pool')
    assert t['bytes'] is None and 'stale' in t
