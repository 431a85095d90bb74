"""Random-init CLIP-style vision encoder with the module layout MuSc's encoder hook expects.

MuSc encodes images with OpenCLIP's ViT-L/14 (models/backbone/open_clip/transformer.py);
the encoding plugin only relies on that module structure:
`model.encode_image(image, out_layers) -> (pooled, [tokens (B, T, width)] per layer)`,
`model.visual.transformer.resblocks[i].attn` an `nn.MultiheadAttention` called with
need_weights=True, tokens after the blocks whose 1-based index is in out_layers
(:319-339), the LND layout inside the transformer, and the LayerNorm that casts
back to the input dtype (:23-29).  This module provides an encoder with that
structure and random weights (no checkpoints are available offline); its GEMMs,
LayerNorms and activations are plain torch — only the attention is this build's
kernel, swapped in by musc_hip._encoder_hip.encode_image.
"""
from __future__ import annotations

import math
from collections import OrderedDict

import torch
from torch import nn
from torch.nn import functional as F


class LayerNorm(nn.LayerNorm):
    """LayerNorm that returns the input dtype."""

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        orig = x.dtype
        return F.layer_norm(x, self.normalized_shape, self.weight, self.bias, self.eps).to(orig)


class QuickGELU(nn.Module):
    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return x * torch.sigmoid(1.702 * x)


class ResidualAttentionBlock(nn.Module):
    def __init__(self, width: int, heads: int, mlp_ratio: float = 4.0):
        super().__init__()
        self.ln_1 = LayerNorm(width)
        self.attn = nn.MultiheadAttention(width, heads)
        self.ln_2 = LayerNorm(width)
        hidden = int(width * mlp_ratio)
        self.mlp = nn.Sequential(OrderedDict([('c_fc', nn.Linear(width, hidden)), ('gelu', QuickGELU()),
                                              ('c_proj', nn.Linear(hidden, width))]))

    def forward(self, x: torch.Tensor, attn_mask=None):
        y = self.ln_1(x)
        out, weights = self.attn(y, y, y, need_weights=True, attn_mask=attn_mask)
        x = x + out
        x = x + self.mlp(self.ln_2(x))
        return x, weights


class Transformer(nn.Module):
    def __init__(self, width: int, layers: int, heads: int):
        super().__init__()
        self.width, self.layers = width, layers
        self.resblocks = nn.ModuleList([ResidualAttentionBlock(width, heads) for _ in range(layers)])

    def forward(self, x: torch.Tensor, out_layers, attn_mask=None):
        out_attn, out_tokens = [], []
        # weights are kept from block 12 (transformer.py:331-333); encoders with
        # fewer blocks keep their last block's
        keep = 12 if len(self.resblocks) >= 12 else len(self.resblocks)
        for idx, block in enumerate(self.resblocks, start=1):
            x, weights = block(x, attn_mask=attn_mask)
            if idx == keep:
                out_attn.append(weights)
            if idx in out_layers:
                out_tokens.append(x)
        return x, out_attn, out_tokens


class VisionTransformer(nn.Module):
    def __init__(self, image_size: int = 518, patch_size: int = 14, width: int = 1024, layers: int = 24,
                 heads: int = 16, output_dim: int = 768):
        super().__init__()
        self.grid = image_size // patch_size
        self.conv1 = nn.Conv2d(3, width, kernel_size=patch_size, stride=patch_size, bias=False)
        scale = width ** -0.5
        self.class_embedding = nn.Parameter(scale * torch.randn(width))
        self.positional_embedding = nn.Parameter(scale * torch.randn(self.grid * self.grid + 1, width))
        self.ln_pre = LayerNorm(width)
        self.transformer = Transformer(width, layers, heads)
        self.ln_post = LayerNorm(width)
        self.proj = nn.Parameter(scale * torch.randn(width, output_dim))

    def forward(self, x: torch.Tensor, out_layers):
        x = self.conv1(x)
        x = x.reshape(x.shape[0], x.shape[1], -1).permute(0, 2, 1)
        cls = self.class_embedding.to(x.dtype) + torch.zeros(x.shape[0], 1, x.shape[-1], dtype=x.dtype,
                                                             device=x.device)
        x = torch.cat([cls, x], dim=1) + self.positional_embedding.to(x.dtype)
        x = self.ln_pre(x).permute(1, 0, 2)           # NLD -> LND
        x, attn, tokens = self.transformer(x, out_layers)
        if attn and attn[0] is not None:
            side = math.isqrt(attn[0].shape[-1] - 1)
            attn[0][0, 0, 1:].view(side, side)         # the consumer's read of the kept weights
        x = x.permute(1, 0, 2)
        tokens = [t.permute(1, 0, 2) for t in tokens]  # LND -> NLD
        pooled = self.ln_post(x[:, 0]) @ self.proj
        return pooled, tokens


class CLIPVision(nn.Module):
    def __init__(self, **kw):
        super().__init__()
        self.visual = VisionTransformer(**kw)

    def encode_image(self, image: torch.Tensor, out_layers):
        return self.visual(image, out_layers)


def vit_l14(image_size: int = 518) -> CLIPVision:
    """ViT-L/14 shape (24 blocks, width 1024, 16 heads, patch 14), random init."""
    return CLIPVision(image_size=image_size, patch_size=14, width=1024, layers=24, heads=16, output_dim=768)
