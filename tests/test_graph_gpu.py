"""HIP graph capture of the scoring path (LNAMD -> MSM -> epilogue).

The entry points clear their buffers with fill kernels (no hipMemsetAsync), launch only
on the caller's stream and never synchronise, so a caller can capture the whole path
with torch.cuda.graph (hipGraph on ROCm) and replay it.  Every replay, with new inputs
copied into the captured buffers and eager work plus synchronisations in between, must
equal the eager result bit for bit.
"""
import pytest
import torch

from musc_hip import _epilogue_hip, pipeline

pytestmark = pytest.mark.gpu


def _tokens(seed, n, side, c, layers, device):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn((n, 1 + side * side, c), generator=g).to(device) for _ in range(layers)]


def _path(tokens, engine, image_size):
    pools = pipeline.lnamd_pools(tokens, [1, 3, 5])
    scores = pipeline.msm_all(pools, engine=engine)
    return _epilogue_hip.maps_and_scores(scores, image_size)


@pytest.mark.parametrize('engine,side,c', [('fp32', 7, 40), ('split16', 16, 32)])
def test_captured_scoring_replays_match_eager(device, engine, side, c):
    n, layers, size = 6, 2, 48
    static = _tokens(1, n, side, c, layers, device)
    side_stream = torch.cuda.Stream()
    side_stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side_stream):          # eager warm-up before capture
        _path(static, engine, size)
    torch.cuda.current_stream().wait_stream(side_stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        maps_g, img_g = _path(static, engine, size)
    for rep, seed in enumerate((1, 2, 3, 2)):
        new = _tokens(seed, n, side, c, layers, device)
        for dst, src in zip(static, new):
            dst.copy_(src)
        graph.replay()
        torch.cuda.synchronize()
        maps_e, img_e = _path(new, engine, size)   # eager work between the replays
        torch.cuda.synchronize()
        print(f'{engine} replay {rep} (seed {seed}): max |graph - eager| '
              f'{(maps_g - maps_e).abs().max().item():.3e}', flush=True)
        assert torch.equal(maps_g, maps_e), rep
        assert torch.equal(img_g, img_e), rep
    del graph
