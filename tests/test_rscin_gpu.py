"""RsCIN on the GPU vs the oracle restatement of models/modules/_RsCIN.py."""
import numpy as np
import pytest
import torch

from oracle import rscin as orc
from musc_hip._RsCIN_hip import RsCIN

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize('n,d,ks', [(83, 768, [1, 2, 3]), (160, 768, [1, 8, 9]), (7, 16, [2])])
def test_matches_oracle(device, n, d, ks):
    rng = np.random.default_rng(n)
    cls = rng.standard_normal((n, d)).astype(np.float32)
    cls /= np.linalg.norm(cls, axis=1, keepdims=True)
    raw = rng.random(n) * 2.0 + 0.5
    got = RsCIN(raw, list(cls), ks)
    assert isinstance(got, np.ndarray) and got.dtype == np.float32
    np.testing.assert_allclose(got, orc.rscin(raw, list(cls), ks), rtol=0, atol=2e-6)
    # tensors in -> tensor out on the device
    t = RsCIN(torch.from_numpy(raw).to(device), torch.from_numpy(cls).to(device), ks)
    assert t.is_cuda
    np.testing.assert_allclose(t.cpu().numpy(), got, rtol=0, atol=0)


def test_passthrough(device):
    raw = np.arange(5.0)
    assert RsCIN(raw, None, [1]) is raw
    assert RsCIN(raw, [np.ones(4, np.float32)] * 5, [0, 1]) is raw
