"""CPU oracle for ViT block softmax attention.  TEST INFRASTRUCTURE ONLY.

The reference runs nn.MultiheadAttention's math path with need_weights=True
(models/backbone/open_clip/transformer.py:232-234): logits = (q * d**-0.5) k^T,
row softmax, probabilities times v; its accelerated path only swaps the softmax
for a fused kernel (models/modules/_attention_gpu.py:41-81,115-146).

`attention_f64` computes softmax(q k^T * scale) v in float64 (numerically stable
max-subtracted softmax).  Tests pin it with closed forms: q = 0 gives the mean
of v's rows, and one dominant logit selects that v row.
"""
from __future__ import annotations

import numpy as np


def attention_f64(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float) -> np.ndarray:
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    logits = np.einsum('btd,bsd->bts', q, k) * scale
    logits -= logits.max(-1, keepdims=True)
    w = np.exp(logits)
    w /= w.sum(-1, keepdims=True)
    return np.einsum('bts,bsd->btd', w, v)


def attention_weights_f64(q: np.ndarray, k: np.ndarray, scale: float) -> np.ndarray:
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    logits = np.einsum('btd,bsd->bts', q, k) * scale
    logits -= logits.max(-1, keepdims=True)
    w = np.exp(logits)
    return w / w.sum(-1, keepdims=True)
