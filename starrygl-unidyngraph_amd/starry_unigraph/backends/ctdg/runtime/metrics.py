"""Link-prediction metrics of a step on the logits' own device
(CTDGOnlineRuntime._metric_dict, backends/ctdg/runtime/runtime.py:202-214,
computes them on the host with scikit-learn).

Scores are sigmoid(logits) in float32 (as the reference takes them), labels
1 for the positive and 0 for the negative logits; the sums are in float64:

* "ap"  -- average precision, scikit-learn's definition: over the distinct
           scores in descending order, sum of (recall step) x precision, with
           every score tied at a threshold counted at that threshold;
* "auc" -- ROC AUC as the Mann-Whitney statistic with tied scores given
           their average rank (equal to the trapezoidal area scikit-learn
           computes);
* "mrr" -- the reference's pairwise statistic mean(pos_i > neg_j) (not a
           reciprocal rank), from the sorted negative scores.

One host transfer of the three numbers; no per-element host work.
"""
from __future__ import annotations

import torch


def link_metrics(pos_logits: torch.Tensor, neg_logits: torch.Tensor) -> dict[str, float]:
    sp = torch.sigmoid(pos_logits.detach().float()).reshape(-1)
    sn = torch.sigmoid(neg_logits.detach().float()).reshape(-1)
    P, N = sp.numel(), sn.numel()
    if P == 0 or N == 0:
        return {"ap": float("nan"), "auc": float("nan"), "mrr": float("nan")}
    scores = torch.cat([sp, sn]).double()
    labels = torch.cat([torch.ones(P, dtype=torch.float64, device=sp.device),
                        torch.zeros(N, dtype=torch.float64, device=sp.device)])
    # groups of equal scores, ascending
    uniq, inv, counts = torch.unique(scores, sorted=True, return_inverse=True, return_counts=True)
    G = uniq.numel()
    pos_in = torch.zeros(G, dtype=torch.float64, device=sp.device).index_add_(0, inv, labels)
    # AUC: average rank of each group (ranks 1..P+N ascending)
    end = torch.cumsum(counts, 0).double()
    avg_rank = end - (counts.double() - 1.0) / 2.0
    auc = ((pos_in * avg_rank).sum() - P * (P + 1) / 2.0) / (P * N)
    # AP: thresholds at the distinct scores, descending
    tp = torch.cumsum(pos_in.flip(0), 0)
    seen = torch.cumsum(counts.flip(0).double(), 0)
    recall_step = pos_in.flip(0) / P
    ap = (recall_step * (tp / seen)).sum()
    # pairwise: for each positive, the negatives strictly below it
    below = torch.searchsorted(torch.sort(sn).values, sp, right=False)
    mrr = below.double().sum() / (P * N)
    ap_v, auc_v, mrr_v = torch.stack([ap, auc, mrr]).tolist()
    return {"ap": ap_v, "auc": auc_v, "mrr": mrr_v}
