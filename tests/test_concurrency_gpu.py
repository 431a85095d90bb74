"""The C-ABI keeps no state: calls from several host threads, each on its own stream,
give the same bits as sequential calls (the thread-safety contract of the boundary)."""
import threading

import pytest
import torch

from musc_hip import _attention_hip, _epilogue_hip, pipeline

pytestmark = pytest.mark.gpu


def _work(tokens, q, k, v, engine='fp32'):
    pools = pipeline.lnamd_pools(tokens, [1, 3])
    scores = pipeline.msm_all(pools, engine=engine)
    maps, img = _epilogue_hip.maps_and_scores(scores, 40)
    att = _attention_hip.attention(q, k, v, 0.125)
    return maps, img, att


def _inputs(seed, device, side=7):
    g = torch.Generator().manual_seed(seed)
    tokens = [torch.randn((6, 1 + side * side, 48), generator=g).to(device) for _ in range(2)]
    q, k, v = (torch.randn((4, 300, 64), generator=g).to(device) for _ in range(3))
    return tokens, q, k, v


# the split engine needs P >= 256: 17 x 17 grids (P = 289, tiles straddling image boundaries)
@pytest.mark.parametrize('engine,side', [('fp32', 7), ('split16', 17)])
def test_threads_on_separate_streams_match_sequential(device, engine, side):
    inputs = [_inputs(s, device, side) + (engine,) for s in (11, 12)]
    expected = [_work(*x) for x in inputs]
    torch.cuda.synchronize()
    results = [[None] * 8, [None] * 8]
    errors = []

    def run(i):
        try:
            stream = torch.cuda.Stream()
            with torch.cuda.stream(stream):
                for rep in range(8):
                    results[i][rep] = _work(*inputs[i])
            stream.synchronize()
        except Exception as exc:  # surfaced below with its thread
            errors.append((i, exc))

    threads = [threading.Thread(target=run, args=(i,)) for i in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert not any(t.is_alive() for t in threads), 'a worker thread did not finish'
    assert not errors, errors
    torch.cuda.synchronize()
    for i in range(2):
        for rep in range(8):
            for got, ref in zip(results[i][rep], expected[i]):
                assert torch.equal(got, ref), (i, rep)
