"""Encoding plugin: the encoder with this build's fused attention.

Mirrors models/modules/_encoder_gpu.py:45-69 and the accelerated encoder of
models/modules/_attention_gpu.py:87-157.  The reference patches F.softmax and
torch.bmm while `model.encode_image` runs, so that nn.MultiheadAttention's math
path (bmm -> softmax -> bmm over (B*16, 1370, 1370) logits) uses its fused
softmax.  Here the whole attention of every ViT block is replaced for the
duration of the call: `attn.forward` of each `nn.MultiheadAttention` in
`model.visual.transformer.resblocks` computes the input projection, runs
softmax(q k^T / sqrt(d)) v in one fused kernel (libmusc_hip musc_attention_fwd;
the (B*H, T, T) logits never exist), then the output projection.  Only block 12,
whose weights Transformer.forward keeps (transformer.py:331-333), also returns
head-averaged probabilities (musc_attention_weights); other blocks return None
for the weights, which their caller discards.  Calls that are not plain
self-attention (masks, separate key/value, batch_first, d != 64) keep the
module's own forward.  The original forwards are restored on exit.

Hook attributes match the reference: encode_image.aggregate_features,
encode_image.new_aggregation, encode_image.begin_inference.
"""
from __future__ import annotations

import time

import torch
from torch import nn
from torch.nn import functional as F

from . import _attention_hip
from ._aggregation_cache import RadiusAggregationCache
from ._lnamd_hip import aggregate_features

_STATS = {}


def begin_inference():
    _STATS.clear()
    _STATS.update(fused_attention_calls=0, weight_blocks=0, fallback_calls=0, seconds=0.0)


def _fused_forward(attn: nn.MultiheadAttention, original, keep_weights: bool):
    def forward(query, key, value, key_padding_mask=None, need_weights=True, attn_mask=None,
                average_attn_weights=True, is_causal=False):
        e = attn.embed_dim
        h = attn.num_heads
        ok = (query is key and key is value and key_padding_mask is None and attn_mask is None and not is_causal
              and not attn.batch_first and attn._qkv_same_embed_dim and attn.in_proj_bias is not None
              and query.is_cuda and query.ndim == 3 and e // h == 64 and e % h == 0
              and query.dtype in (torch.float32, torch.float16) and average_attn_weights
              and not torch.is_grad_enabled())
        if not ok:
            _STATS['fallback_calls'] = _STATS.get('fallback_calls', 0) + 1
            return original(query, key, value, key_padding_mask=key_padding_mask, need_weights=need_weights,
                            attn_mask=attn_mask, average_attn_weights=average_attn_weights, is_causal=is_causal)
        t, b, _ = query.shape
        qkv = F.linear(query, attn.in_proj_weight, attn.in_proj_bias)       # (T, B, 3E), autocast-aware
        dt = torch.float16 if qkv.dtype == torch.float16 else torch.float32
        qkv = qkv.to(dt).reshape(t, b, 3, h, 64)                             # [q | k | v], each H x 64
        q = qkv[:, :, 0].reshape(t, b * h, 64).transpose(0, 1).contiguous()  # (B*H, T, 64), b-major
        k = qkv[:, :, 1].reshape(t, b * h, 64).transpose(0, 1).contiguous()
        v = qkv[:, :, 2].reshape(t, b * h, 64).transpose(0, 1).contiguous()
        scale = 64 ** -0.5
        out = _attention_hip.attention(q, k, v, scale)                      # (B*H, T, 64)
        weights = _attention_hip.attention_weights(q, k, h, scale) if (need_weights and keep_weights) else None
        out = out.transpose(0, 1).reshape(t, b, e)
        out = F.linear(out, attn.out_proj.weight, attn.out_proj.bias)
        _STATS['fused_attention_calls'] = _STATS.get('fused_attention_calls', 0) + 1
        if weights is not None:
            _STATS['weight_blocks'] = _STATS.get('weight_blocks', 0) + 1
        return out, weights
    return forward


def encode_image(model, image, out_layers):
    """(pooled (B, D), [tokens (B, T, width)] for out_layers) with the fused attention."""
    blocks = getattr(getattr(getattr(model, 'visual', None), 'transformer', None), 'resblocks', [])
    restored = []
    start = time.perf_counter()
    try:
        for index, block in enumerate(blocks):
            attention = getattr(block, 'attn', None)
            if not isinstance(attention, nn.MultiheadAttention):
                continue
            present = 'forward' in attention.__dict__
            previous = attention.__dict__.get('forward')
            keep = (index == 11) or (len(blocks) < 12 and index == len(blocks) - 1)
            attention.forward = _fused_forward(attention, attention.forward, keep)
            restored.append((attention, present, previous))
        return model.encode_image(image, out_layers)
    finally:
        for attention, present, previous in reversed(restored):
            if present:
                attention.forward = previous
            else:
                attention.__dict__.pop('forward', None)
        _STATS['seconds'] = _STATS.get('seconds', 0.0) + time.perf_counter() - start


def new_aggregation():
    return RadiusAggregationCache()


def research_diagnostics():
    return dict(_STATS)


encode_image.aggregate_features = aggregate_features
encode_image.new_aggregation = new_aggregation
encode_image.begin_inference = begin_inference
begin_inference()
