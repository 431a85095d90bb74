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


def check_rscin(got, scores_old, cls_tokens, k_list, atol=2e-5):
    """Gate an RsCIN result against the definition.

    The result must match the float64 brute force (`rscin_bruteforce_f64`) within
    atol on every row.  The fp32 restatement of the reference (`rscin`) is reported
    beside it: where two class-token similarities lie closer together than fp32
    rounding resolves, its top-k keeps one or the other depending on the summation
    order of its matrix product, so on such rows it departs from the definition;
    `fp32_restatement_flips` counts them and the other rows are compared too.
    Returns (passed, details).
    """
    got = np.asarray(got, dtype=np.float64)
    bf = rscin_bruteforce_f64(scores_old, cls_tokens, k_list)
    ref = np.asarray(rscin(scores_old, list(cls_tokens), k_list), dtype=np.float64)
    flips = np.abs(ref - bf) > atol
    err_bf = np.abs(got - bf)
    err_ref = np.abs(got - ref)[~flips]
    passed = bool(np.all(err_bf <= atol) and np.all(err_ref <= atol))
    details = {'rows': int(len(got)), 'max_err_vs_f64': float(err_bf.max()),
               'fp32_restatement_flips': int(flips.sum()),
               'max_err_vs_fp32_other_rows': float(err_ref.max()) if err_ref.size else 0.0}
    return passed, details
