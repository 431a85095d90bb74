"""Encoding plugin: the encoder with this build's fused attention and block layers.

Mirrors models/modules/_encoder_gpu.py:45-69 and the accelerated encoder of
models/modules/_attention_gpu.py:87-157.  The reference patches F.softmax and
torch.bmm while `model.encode_image` runs, so that nn.MultiheadAttention's math
path (bmm -> softmax -> bmm over (B*16, 1370, 1370) logits) uses its fused
softmax.  Here, for the duration of the call, the forward of every block in
`model.visual.transformer.resblocks` is replaced:

* block level (ResidualAttentionBlock, transformer.py:236-248, with the cast-back
  LayerNorm of :23-29 and QuickGELU of :32-35 or erf GELU): ln_1 is one fused
  LayerNorm pass; the in-projection is torch's GEMM (hipBLASLt); softmax(q k^T /
  sqrt(d)) v runs in one fused kernel that reads q, k, v straight out of the packed
  (T, B, 3E) projection and writes the (T, B, E) layout the out-projection takes
  (libmusc_hip musc_attention_fwd_strided; no logits, no head transposes); the
  residual add and ln_2 are one pass (musc_layernorm_rows with a residual); c_fc
  (GEMM with bias) is followed by one in-place activation pass (musc_activation);
  c_proj and the last residual add are torch.
* attention level, for blocks of any other structure: only the
  nn.MultiheadAttention forward is replaced by in-projection -> fused attention ->
  out-projection.

The tower's ln_pre and ln_post (the same cast-back LayerNorm) are swapped for the
one-pass kernel too.  The patch embedding conv1 (transformer.py:380, :566: a Conv2d
whose kernel equals its stride) keeps the model's own convolution by default, the
one the math path runs: under fp16 autocast the convolution library's result and an
fp32-accumulated GEMM of the same patches round differently in over half of the
outputs, a difference the following blocks carry to every token (on the ViT-L/14 of
BASELINE config 5 with its weights scaled by 1/4 it alone moves the anomaly maps by
2.3e-5, where the fused blocks without it stay within 5.2e-6 of the math path), for
2 ms per 160 images.  Setting PATCH_EMBED_GEMM = True replaces conv1 by what it
computes, a GEMM of the image's non-overlapping patches (one gather of the patches
into (B * grid^2, 3 * p^2) rows in the compute dtype, then torch's GEMM), for
setups whose convolution library falls back to a slow direct kernel.

Only block 12, whose weights Transformer.forward keeps (transformer.py:331-333),
also returns head-averaged probabilities (musc_attention_weights_strided); other
blocks return None for the weights, which their caller discards.  Calls that are
not plain self-attention (masks, separate key/value, batch_first, d != 64,
gradients) keep the module's own forward.  The original forwards are restored on
exit.

Hook attributes match the reference: encode_image.aggregate_features,
encode_image.new_aggregation, encode_image.begin_inference.
"""
from __future__ import annotations

import time

import torch
from torch import nn
from torch.nn import functional as F

from . import _attention_hip, _layers_hip
from . import _runtime as rt
from ._aggregation_cache import RadiusAggregationCache
from ._lnamd_hip import aggregate_features

_STATS = {}

# conv1 as a patch GEMM (see the module docstring); off: the model's own convolution
PATCH_EMBED_GEMM = False


def begin_inference():
    _STATS.clear()
    _STATS.update(fused_blocks=0, fused_attention_calls=0, weight_blocks=0, fused_layer_norms=0, patch_embeds=0,
                  fallback_calls=0, seconds=0.0)


def _count(key: str) -> None:
    _STATS[key] = _STATS.get(key, 0) + 1


def _mha_ok(attn: nn.MultiheadAttention, x: torch.Tensor) -> bool:
    e, h = attn.embed_dim, attn.num_heads
    return (not attn.batch_first and attn._qkv_same_embed_dim and attn.in_proj_bias is not None
            and e % h == 0 and e // h == 64 and x.is_cuda and x.ndim == 3 and x.shape[-1] == e
            and x.dtype in (torch.float32, torch.float16) and not torch.is_grad_enabled())


def _attention(attn: nn.MultiheadAttention, y: torch.Tensor, keep_weights: bool):
    """Self-attention of nn.MultiheadAttention on (T, B, E) input y: (out, weights | None),
    or None when the projection's dtype has no kernel."""
    qkv = F.linear(y, attn.in_proj_weight, attn.in_proj_bias)   # (T, B, 3E), autocast-aware
    if qkv.dtype not in (torch.float32, torch.float16):
        return None
    qkv = qkv.contiguous()
    h = attn.num_heads
    scale = 64 ** -0.5
    o = _attention_hip.attention_packed(qkv, h, scale)                # (T, B, E)
    weights = _attention_hip.attention_weights_packed(qkv, h, scale) if keep_weights else None
    _count('fused_attention_calls')
    if weights is not None:
        _count('weight_blocks')
    return F.linear(o, attn.out_proj.weight, attn.out_proj.bias), weights


def _fused_mha_forward(attn: nn.MultiheadAttention, original, keep_weights: bool):
    def forward(query, key, value, key_padding_mask=None, need_weights=True, attn_mask=None,
                average_attn_weights=True, is_causal=False):
        res = None
        if (query is key and key is value and key_padding_mask is None and attn_mask is None and not is_causal
                and average_attn_weights and _mha_ok(attn, query)):
            res = _attention(attn, query, need_weights and keep_weights)
        if res is None:
            _count('fallback_calls')
            return original(query, key, value, key_padding_mask=key_padding_mask, need_weights=need_weights,
                            attn_mask=attn_mask, average_attn_weights=average_attn_weights, is_causal=is_causal)
        return res
    return forward


def _cast_back_layer_norm(ln) -> bool:
    # the reference's LayerNorm / LayerNormFp32 subclasses return the input dtype;
    # plain nn.LayerNorm under autocast returns fp32 and is left to torch
    return (isinstance(ln, nn.LayerNorm) and type(ln) is not nn.LayerNorm
            and type(ln).__name__ in ('LayerNorm', 'LayerNormFp32') and len(ln.normalized_shape) == 1)


def _activation_mode(act):
    if type(act).__name__ == 'QuickGELU':
        return rt.ACT_QUICK_GELU
    if isinstance(act, nn.GELU) and act.approximate == 'none':
        return rt.ACT_GELU
    return None


def _block_plan(block):
    """Activation mode when `block` has the ResidualAttentionBlock structure this hook
    fuses (transformer.py:190-248 without LayerScale or cross-attention), else None."""
    attn = getattr(block, 'attn', None)
    mlp = getattr(block, 'mlp', None)
    if not isinstance(attn, nn.MultiheadAttention) or hasattr(block, 'ln_1_kv'):
        return None
    if not (_cast_back_layer_norm(getattr(block, 'ln_1', None)) and _cast_back_layer_norm(getattr(block, 'ln_2', None))):
        return None
    for name in ('ls_1', 'ls_2'):
        if not isinstance(getattr(block, name, nn.Identity()), nn.Identity):
            return None
    c_fc, act, c_proj = (getattr(mlp, n, None) for n in ('c_fc', 'gelu', 'c_proj'))
    if not (isinstance(mlp, nn.Sequential) and len(mlp) == 3 and isinstance(c_fc, nn.Linear)
            and isinstance(c_proj, nn.Linear)):
        return None
    return _activation_mode(act)


def _fused_ln_forward(ln, original):
    """ln_pre / ln_post of the vision tower (transformer.py:555-579; the cast-back LayerNorm
    of :23-29) as one pass; other inputs keep the module's own forward."""
    def forward(x):
        if (isinstance(x, torch.Tensor) and x.is_cuda and not torch.is_grad_enabled()
                and _layers_hip.supports_layer_norm(x.shape[-1], x.dtype)):
            _count('fused_layer_norms')
            return _layers_hip.layer_norm(x, ln.weight, ln.bias, ln.eps)
        return original(x)
    return forward


def _patch_conv(conv) -> bool:
    """A bias-free or biased Conv2d that tiles its input into non-overlapping patches."""
    return (isinstance(conv, nn.Conv2d) and tuple(conv.kernel_size) == tuple(conv.stride)
            and tuple(conv.dilation) == (1, 1) and conv.groups == 1 and conv.padding_mode == 'zeros'
            and not isinstance(conv.padding, str) and tuple(conv.padding) == (0, 0))


def _patch_embed_forward(conv, original):
    """conv1 of the vision tower as patches @ weight^T.  Rows and columns the stride does
    not reach are dropped, as the convolution drops them; under autocast the patches are
    gathered already in the autocast dtype (the GEMM would cast them anyway)."""
    ph, pw = conv.kernel_size

    def forward(x):
        if not (isinstance(x, torch.Tensor) and x.is_cuda and x.ndim == 4 and x.shape[1] == conv.in_channels
                and x.shape[2] >= ph and x.shape[3] >= pw and not torch.is_grad_enabled()):
            return original(x)
        b, c = x.shape[:2]
        gh, gw = x.shape[2] // ph, x.shape[3] // pw
        dtype = torch.get_autocast_dtype('cuda') if torch.is_autocast_enabled('cuda') else x.dtype
        patches = torch.empty((b, gh, gw, c, ph, pw), dtype=dtype, device=x.device)
        patches.copy_(x[:, :, :gh * ph, :gw * pw].reshape(b, c, gh, ph, gw, pw).permute(0, 2, 4, 1, 3, 5))
        out = F.linear(patches.view(b * gh * gw, c * ph * pw), conv.weight.reshape(conv.out_channels, -1), conv.bias)
        _count('patch_embeds')
        return out.view(b, gh, gw, conv.out_channels).permute(0, 3, 1, 2)     # (B, width, grid, grid)
    return forward


def _fused_block_forward(block, original, mode: int, keep_weights: bool):
    ln_1, ln_2, attn = block.ln_1, block.ln_2, block.attn
    c_fc, c_proj = block.mlp.c_fc, block.mlp.c_proj

    def forward(*args, **kwargs):
        x = args[0] if len(args) == 1 else None
        extra = {k: v for k, v in kwargs.items() if v is not None}
        if x is None or extra or not _mha_ok(attn, x) or not _layers_hip.supports_layer_norm(x.shape[-1], x.dtype):
            _count('fallback_calls')
            return original(*args, **kwargs)
        y = _layers_hip.layer_norm(x, ln_1.weight, ln_1.bias, ln_1.eps)
        res = _attention(attn, y, keep_weights)
        if res is None:
            _count('fallback_calls')
            return original(*args, **kwargs)
        a, weights = res
        if a.dtype == x.dtype:
            x, y = _layers_hip.layer_norm(x, ln_2.weight, ln_2.bias, ln_2.eps, residual=a)
        else:
            x = x + a
            y = ln_2(x)
        hdn = F.linear(y, c_fc.weight, c_fc.bias)
        if hdn.dtype in (torch.float32, torch.float16) and hdn.is_contiguous():
            _layers_hip.activation_(hdn, mode)
        else:
            hdn = block.mlp.gelu(hdn)
        x = x + F.linear(hdn, c_proj.weight, c_proj.bias)
        _count('fused_blocks')
        return x, weights
    return forward


def encode_image(model, image, out_layers):
    """(pooled (B, D), [tokens (B, T, width)] for out_layers) with the fused blocks."""
    visual = getattr(model, 'visual', None)
    blocks = getattr(getattr(visual, 'transformer', None), 'resblocks', [])
    restored = []
    start = time.perf_counter()
    try:
        for name in ('ln_pre', 'ln_post'):
            ln = getattr(visual, name, None)
            if _cast_back_layer_norm(ln):
                restored.append((ln, 'forward' in ln.__dict__, ln.__dict__.get('forward')))
                ln.forward = _fused_ln_forward(ln, ln.forward)
        conv1 = getattr(visual, 'conv1', None)
        if PATCH_EMBED_GEMM and _patch_conv(conv1):
            restored.append((conv1, 'forward' in conv1.__dict__, conv1.__dict__.get('forward')))
            conv1.forward = _patch_embed_forward(conv1, conv1.forward)
        for index, block in enumerate(blocks):
            keep = (index == 11) or (len(blocks) < 12 and index == len(blocks) - 1)
            mode = _block_plan(block)
            if mode is not None:
                target, make = block, (lambda o, b=block, m=mode, k=keep: _fused_block_forward(b, o, m, k))
            elif isinstance(getattr(block, 'attn', None), nn.MultiheadAttention):
                target, make = block.attn, (lambda o, a=block.attn, k=keep: _fused_mha_forward(a, o, k))
            else:
                continue
            present = 'forward' in target.__dict__
            previous = target.__dict__.get('forward')
            target.forward = make(target.forward)
            restored.append((target, present, previous))
        return model.encode_image(image, out_layers)
    finally:
        for target, present, previous in reversed(restored):
            if present:
                target.forward = previous
            else:
                target.__dict__.pop('forward', None)
        _STATS['seconds'] = _STATS.get('seconds', 0.0) + time.perf_counter() - start


def new_aggregation():
    return RadiusAggregationCache()


def research_diagnostics():
    return dict(_STATS)


encode_image.aggregate_features = aggregate_features
encode_image.new_aggregation = new_aggregation
encode_image.begin_inference = begin_inference
begin_inference()
