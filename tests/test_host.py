"""Host-side logic of the plugin mirror (CPU only, no kernel launches)."""
from copy import deepcopy
from types import SimpleNamespace

import pytest
import torch

from musc_hip import _MSM_hip, _lnamd_hip
from musc_hip._backend import configure_backend, select_backend


CFG = {'models': dict(inference_backend='super_fast', backbone_name='ViT-L-14-336', pretrained='openai',
                      batch_size=4, feature_layers=[5, 11, 17, 23], r_list=[1, 3, 5]),
       'datasets': dict(img_resize=518, divide_num=1)}


def test_select_backend_contract():
    # models/modules/_backend.py:5-14 semantics
    with pytest.raises(ValueError):
        select_backend('fast', 'cuda')
    assert select_backend('original', 'cuda') == ('original', None)
    assert select_backend('gpu', 'cpu') == ('original', 'CUDA is unavailable')
    assert select_backend('super_fast', 'cpu')[0] == 'original'


def _fake_device(monkeypatch, arch):
    """A visible ROCm device of architecture `arch` (gcnArchName as HIP reports it)."""
    monkeypatch.setattr(torch.version, 'hip', torch.version.hip or '7.0')
    monkeypatch.setattr(torch.cuda, 'is_available', lambda: True)
    monkeypatch.setattr(torch.cuda, 'is_initialized', lambda: True)
    monkeypatch.setattr(torch.cuda, 'current_device', lambda: 0)
    monkeypatch.setattr(torch.cuda, 'get_device_properties', lambda i: SimpleNamespace(gcnArchName=arch))


@pytest.fixture
def gfx950(monkeypatch):
    _fake_device(monkeypatch, 'gfx950:sramecc+:xnack-')


def test_select_backend_on_rocm_build(gfx950):
    assert select_backend('gpu', 'cuda') == ('gpu', None)
    assert select_backend('super_fast', 'cuda') == ('super_fast', None)


def test_select_backend_wrong_architecture_falls_back(monkeypatch):
    # the reference answers ('original', reason) whenever its accelerated runtime cannot
    # run (models/modules/_backend.py:10-13); a device the kernels are not built for is such a case
    from musc_hip import _runtime
    assert _runtime.target_arch() == 'gfx950'
    _fake_device(monkeypatch, 'gfx942:sramecc+:xnack-')
    sel, reason = select_backend('gpu', 'cuda')
    assert sel == 'original' and 'gfx942' in reason and 'gfx950' in reason
    cfg = deepcopy(CFG)
    assert configure_backend(cfg, 'cuda') is cfg        # super_fast preset not applied either


def test_select_backend_no_visible_device(monkeypatch):
    monkeypatch.setattr(torch.version, 'hip', torch.version.hip or '7.0')
    monkeypatch.setattr(torch.cuda, 'is_available', lambda: False)
    monkeypatch.setattr(torch.cuda, 'device_count', lambda: 0)
    for initialised in (False, True):
        monkeypatch.setattr(torch.cuda, 'is_initialized', lambda: initialised)
        sel, reason = select_backend('gpu', 'cuda')
        assert sel == 'original' and 'no ROCm device' in reason


def _no_gpu_calls(monkeypatch):
    def fail(*a, **k):
        raise AssertionError('the selector must not start the GPU runtime')
    for name in ('is_available', 'current_device', 'get_device_properties', 'current_stream', 'init'):
        monkeypatch.setattr(torch.cuda, name, fail)


def test_select_backend_makes_no_gpu_calls_before_hip_starts(monkeypatch):
    # models/modules/_backend.py:1: "no model loading or CUDA calls"; with the runtime not
    # yet initialised only the device count is read (it starts no HIP context)
    monkeypatch.setattr(torch.version, 'hip', torch.version.hip or '7.0')
    monkeypatch.setattr(torch.cuda, 'is_initialized', lambda: False)
    monkeypatch.setattr(torch.cuda, 'device_count', lambda: 1)
    _no_gpu_calls(monkeypatch)
    assert select_backend('gpu', 'cuda') == ('gpu', None)
    cfg = deepcopy(CFG)
    assert configure_backend(cfg, 'cuda')['models']['r_list'] == [3]


def test_first_launch_checks_the_architecture(monkeypatch):
    # the architecture the selector skipped is compared at the first launch on a device
    from musc_hip import _runtime
    _fake_device(monkeypatch, 'gfx942:sramecc+:xnack-')
    monkeypatch.setattr(torch.cuda, 'current_stream',
                        lambda d=None: SimpleNamespace(device_index=0, cuda_stream=0))
    monkeypatch.setattr(_runtime, '_supported_devices', set())
    with pytest.raises(RuntimeError, match='gfx942'):
        _runtime.stream(0)
    _fake_device(monkeypatch, 'gfx950:sramecc+:xnack-')
    assert _runtime.stream(0) == 0 and _runtime._supported_devices == {0}


def test_configure_backend_preset_isolated(gfx950):
    # tools/test_super_fast.py:16-24 analogue
    original = deepcopy(CFG)
    changed = configure_backend(CFG, 'cuda')
    if torch.version.hip is None:
        pytest.skip('needs a ROCm torch build to select super_fast')
    assert changed['models']['feature_layers'] == [5] and changed['models']['r_list'] == [3]
    assert CFG == original
    changed['datasets']['divide_num'] = 2
    assert CFG['datasets']['divide_num'] == 1


def test_configure_backend_fallback_and_rejection(gfx950):
    assert configure_backend(CFG, 'cpu') is CFG
    for requested in ('original', 'gpu'):
        cfg = deepcopy(CFG)
        cfg['models']['inference_backend'] = requested
        assert configure_backend(cfg, 'cuda') is cfg
    if torch.version.hip is None:
        return
    for group, key, value in [('models', 'backbone_name', 'ViT-B-32'), ('models', 'batch_size', 8),
                              ('datasets', 'img_resize', 336), ('datasets', 'divide_num', 2)]:
        changed = deepcopy(CFG)
        changed[group][key] = value
        with pytest.raises(ValueError, match='super_fast requires'):
            configure_backend(changed, 'cuda')


def test_msm_rank_window_and_validation():
    assert _MSM_hip.rank_window(83) == (0, 24)
    assert _MSM_hip.rank_window(8) == (0, 2)
    with pytest.raises(ValueError, match='CUDA FP32'):
        _MSM_hip.MSM(torch.zeros((8, 4, 4)))          # CPU tensor: rejected before any launch
    with pytest.raises(ValueError, match='CUDA FP32'):
        _MSM_hip.MSM(torch.zeros((8, 4)))


def test_msm_engine_selection():
    _MSM_hip.check_engine('fp32', 1)
    _MSM_hip.check_engine('split16', _MSM_hip.SPLIT_MIN_P)
    with pytest.raises(ValueError, match='Unknown MSM engine'):
        _MSM_hip.check_engine('bf16', 1369)
    with pytest.raises(ValueError, match='P >= 256'):
        _MSM_hip.check_engine('split16', _MSM_hip.SPLIT_MIN_P - 1)


def _dev(shape, dtype=torch.float32):
    """Stands for a device tensor: what the predicate reads (shape, dtype, device, is_cuda)."""
    return SimpleNamespace(shape=torch.Size(shape), dtype=dtype, device=torch.device('cuda', 0), is_cuda=True)


def test_aggregation_predicate(monkeypatch):
    monkeypatch.setattr(torch.version, 'hip', torch.version.hip or '7.0')
    layer = _lnamd_hip.LNAMD(feature_dim=8, feature_layer=[1, 2], r=3)
    feats = [_dev((2, 26, 8)), _dev((2, 26, 8))]
    assert _lnamd_hip.supported(layer, feats)
    assert not _lnamd_hip.supported(layer, feats[:1])                       # layer count mismatch
    assert not _lnamd_hip.supported(layer, [_dev((2, 27, 8))] * 2)          # not square
    layer7 = _lnamd_hip.LNAMD(feature_dim=8, feature_layer=[1, 2], r=7)
    assert not _lnamd_hip.supported(layer7, feats)                          # r outside {1,3,5}
    stride2 = SimpleNamespace(r=3, patch_maker=SimpleNamespace(stride=2),
                              LNA=SimpleNamespace(output_dim=8, preprocessing_modules=[0, 0]))
    assert not _lnamd_hip.supported(stride2, feats)
    assert not _lnamd_hip.supported(layer, [torch.zeros((2, 26, 8))] * 2)   # host tensors


@pytest.mark.parametrize('case', ['c_not_mult_4', 'c_too_large', 'too_many_layers', 'bf16', 'fp64', 'no_grid'])
def test_aggregation_predicate_kernel_limits_fall_back(case, monkeypatch):
    # inputs musc_lnamd_f32 rejects take layer._embed, as every input outside the
    # reference's fast path does (models/modules/_encoder_gpu.py:18-22)
    monkeypatch.setattr(torch.version, 'hip', torch.version.hip or '7.0')
    c, layers, dtype, tokens = 8, 2, torch.float32, 26
    if case == 'c_not_mult_4':
        c = 10
    elif case == 'c_too_large':
        c = _lnamd_hip.MAX_CHANNELS + 4
    elif case == 'too_many_layers':
        layers = _lnamd_hip.MAX_LAYERS + 1
    elif case == 'bf16':
        dtype = torch.bfloat16
    elif case == 'fp64':
        dtype = torch.float64
    elif case == 'no_grid':
        tokens = 1
    layer = _lnamd_hip.LNAMD(feature_dim=c, feature_layer=list(range(layers)), r=3)
    feats = [_dev((2, tokens, c), dtype) for _ in range(layers)]
    assert not _lnamd_hip.supported(layer, feats)
    calls = []
    layer._embed = lambda features, return_cpu=True: calls.append((features, return_cpu)) or 'embedded'
    assert _lnamd_hip.aggregate_features(layer, feats, return_cpu=False) == 'embedded'
    assert calls and calls[0][1] is False
    from musc_hip._aggregation_cache import RadiusAggregationCache
    assert RadiusAggregationCache()(layer, feats, return_cpu=True) == 'embedded'
    ok = _lnamd_hip.LNAMD(feature_dim=8, feature_layer=[0, 1], r=3)
    assert _lnamd_hip.supported(ok, [_dev((2, 26, 8)), _dev((2, 26, 8))])   # the same predicate in range


def test_agreement_gate_known_answers():
    # the reference's own known answers for its gate (tools/test_benchmark.py:8-16)
    import numpy as np
    from musc_hip.agreement import compare_arrays
    a = np.arange(24., dtype=np.float64).reshape(6, 4)
    assert compare_arrays(a, a)['pass']
    assert compare_arrays(a, a + 1e-5)['pass']
    assert not compare_arrays(a, a + 3e-5)['pass']
    assert not compare_arrays(a, a[:2])['pass']
    assert not compare_arrays(a[:0], a[:0])['pass']
    b = a.copy()
    b[0, 0] = np.nan
    assert not compare_arrays(a, b)['pass']
    # and the rest of its contract: +-inf rejected on either side, torch tensors accepted,
    # errors reported, more rows than one chunk
    c = a.copy()
    c[5, 3] = np.inf
    r = compare_arrays(c, a)
    assert not r['pass'] and r['finite'] is False and r['max_absolute_error'] is None
    r = compare_arrays(torch.tensor(a), torch.tensor(a + 1.5e-5))
    assert r['pass'] and abs(r['max_absolute_error'] - 1.5e-5) < 1e-12 and r['shape_match']
    big = np.random.default_rng(0).standard_normal((37, 5, 3))
    worse = big.copy()
    worse[36, 4, 2] += 2.5e-5                      # only in the last chunk
    assert compare_arrays(big, big)['pass'] and not compare_arrays(big, worse)['pass']


def test_nan_aware_match():
    import numpy as np
    from musc_hip.agreement import nan_aware_match
    a = np.array([1.0, np.nan, np.inf, 2.0])
    assert nan_aware_match(a, a + np.array([1e-6, 0, 0, -1e-6]))['pass']
    assert not nan_aware_match(a, np.array([1.0, 3.0, np.inf, 2.0]))['pass']     # NaN lost
    assert not nan_aware_match(a, np.array([np.nan, np.nan, np.inf, 2.0]))['pass']  # NaN added
    assert not nan_aware_match(a, np.array([1.0, np.nan, 5.0, 2.0]))['pass']     # inf lost
    assert not nan_aware_match(a, a + 1e-4)['pass']


def test_patch_embedding_hook_predicate_and_cpu_fallback():
    # conv1 (kernel == stride, no padding / dilation / groups) is what the encoding plugin
    # turns into patches @ W^T when PATCH_EMBED_GEMM is set; anything else, and any input
    # the GEMM path does not take (here: a CPU tensor), keeps the module's own forward
    from musc_hip import _encoder_hip
    conv = torch.nn.Conv2d(3, 16, kernel_size=14, stride=14, bias=False)
    assert _encoder_hip._patch_conv(conv)
    assert _encoder_hip._patch_conv(torch.nn.Conv2d(3, 16, kernel_size=(7, 5), stride=(7, 5)))
    for other in (torch.nn.Conv2d(3, 16, 14, stride=7), torch.nn.Conv2d(3, 16, 14, stride=14, padding=1),
                  torch.nn.Conv2d(3, 16, 14, stride=14, dilation=2), torch.nn.Conv2d(4, 16, 14, stride=14, groups=2),
                  torch.nn.Conv2d(3, 16, 3, stride=3, padding='valid'), torch.nn.Linear(3, 16), None):
        assert not _encoder_hip._patch_conv(other)
    calls = []

    def original(x):
        calls.append(x)
        return conv._conv_forward(x, conv.weight, conv.bias)
    hook = _encoder_hip._patch_embed_forward(conv, original)
    x = torch.rand((1, 3, 28, 28))
    with torch.no_grad():
        out = hook(x)
    assert len(calls) == 1 and out.shape == (1, 16, 2, 2)
