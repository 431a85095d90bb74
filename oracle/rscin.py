"""CPU oracle for RsCIN (models/modules/_RsCIN.py:5-32).  TEST INFRASTRUCTURE ONLY.

`rscin` restates the reference: min-max normalised scores, W = X X^T (float32),
for each k the N-k smallest entries of every row zeroed via torch.topk, the
row-normalised W times the scores, averaged over k_list.  `rscin_bruteforce_f64`
is an independent float64 loop over the same definition (keep the k largest
similarities of each row, weighted mean of the normalised scores).
"""
from __future__ import annotations

import numpy as np
import torch


def rscin(scores_old, cls_tokens=None, k_list=(0,)):
    k_list = list(k_list)
    if cls_tokens is None or 0 in k_list:
        return scores_old
    cls = np.array(cls_tokens, dtype=np.float32)
    scores = (scores_old - scores_old.min()) / (scores_old.max() - scores_old.min())
    W = torch.tensor(cls @ cls.T).float()
    score = torch.tensor(scores).float()
    outs = []
    for k in k_list:
        _, drop = torch.topk(W, W.shape[0] - k, largest=False, sorted=True)
        Wm = W.clone()
        for i in range(W.shape[0]):
            Wm[i, drop[i]] = 0
        D = torch.diag(1.0 / Wm.sum(1))
        outs.append((D @ Wm) @ score.unsqueeze(-1))
    return torch.cat(outs, -1).mean(-1).numpy()


def rscin_bruteforce_f64(scores_old, cls_tokens, k_list):
    cls = np.asarray(cls_tokens, dtype=np.float64)
    s = np.asarray(scores_old, dtype=np.float64)
    s = (s - s.min()) / (s.max() - s.min())
    W = cls @ cls.T
    out = np.zeros(len(s))
    for k in k_list:
        for i in range(len(s)):
            keep = np.argsort(-W[i], kind='stable')[:k]
            out[i] += (W[i, keep] * s[keep]).sum() / W[i, keep].sum()
    return out / len(k_list)
