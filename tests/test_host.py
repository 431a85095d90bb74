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


def test_select_backend_on_rocm_build():
    sel, reason = select_backend('gpu', 'cuda')
    if torch.version.hip is None:
        assert sel == 'original' and 'ROCm' in reason
    else:
        assert (sel, reason) == ('gpu', None)


def test_configure_backend_preset_isolated():
    # tools/test_super_fast.py:16-24 analogue
    original = deepcopy(CFG)
    changed = configure_backend(CFG, 'cuda')
    if torch.version.hip is None:
        pytest.skip('needs a ROCm torch build to select super_fast')
    assert changed['models']['feature_layers'] == [5] and changed['models']['r_list'] == [3]
    assert CFG == original
    changed['datasets']['divide_num'] = 2
    assert CFG['datasets']['divide_num'] == 1


def test_configure_backend_fallback_and_rejection():
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


def test_aggregation_predicate():
    layer = _lnamd_hip.LNAMD(feature_dim=8, feature_layer=[1, 2], r=3)
    feats = [torch.zeros((2, 26, 8)), torch.zeros((2, 26, 8))]
    assert _lnamd_hip.supported(layer, feats)
    assert not _lnamd_hip.supported(layer, feats[:1])                       # layer count mismatch
    assert not _lnamd_hip.supported(layer, [torch.zeros((2, 27, 8))] * 2)   # not square
    layer7 = _lnamd_hip.LNAMD(feature_dim=8, feature_layer=[1, 2], r=7)
    assert not _lnamd_hip.supported(layer7, feats)                          # r outside {1,3,5}
    stride2 = SimpleNamespace(r=3, patch_maker=SimpleNamespace(stride=2),
                              LNA=SimpleNamespace(output_dim=8, preprocessing_modules=[0, 0]))
    assert not _lnamd_hip.supported(stride2, feats)


def test_patch_embedding_hook_predicate_and_cpu_fallback():
    # conv1 (kernel == stride, no padding / dilation / groups) is what the encoding plugin
    # turns into patches @ W^T; anything else, and any input the GEMM path does not take
    # (here: a CPU tensor), keeps the module's own forward
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
