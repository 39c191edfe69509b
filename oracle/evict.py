"""Eviction scoring and top-k retention (numpy restatement).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Reference:
  * ``snapkv_scores``                  STRATA_KV.py:932-954 (window queries, causal fp32 softmax,
                                       window columns dropped, mean over window queries,
                                       avg_pool1d(k, pad k//2, count_include_pad), mean over the
                                       query heads of each KV group, window = max + 1)
  * top-k + position order             STRATA_KV.py:975 (``topk``), 1022-1023 (MTLP sorts the
                                       retained indices into position order)
  * the decode-time form (C4)          scores = probabilities of consecutive decode queries over
                                       the packed context, accumulated per KV head (mean over its
                                       query heads), then top-k plus a forced recent window

Tie order: ``torch.topk`` leaves the order of equal scores unspecified (the reference pins
nothing there).  This oracle, and the GPU kernel, keep the lowest positions among scores equal
to the k-th largest.

Pinning (tests/test_oracle_evict.py): snapkv_scores against a per-query float64 loop with an
explicit pooling sum; topk_retain against a full sort; accumulate_decode_scores against the
softmax of chunked_attention's logits; invariants (scores of one step sum to 1 per query head
minus the exact-row mass; the forced window is always kept).
"""
from __future__ import annotations

import numpy as np

from .attention import rep_heads


def snapkv_scores(q: np.ndarray, k: np.ndarray, H: int, scaling: float, window: int,
                  kernel: int) -> np.ndarray:
    """q (B, Hq, >=H, d) queries, k (B, Hkv, >=H, d) -> (B, Hkv, H) float64 (STRATA_KV.py:932-954)."""
    B, Hkv = k.shape[:2]
    rep = q.shape[1] // Hkv
    w = window
    qo = q[:, :, H - w:H].astype(np.float64)
    kk = rep_heads(k[:, :, :H].astype(np.float64), rep)
    att = np.einsum("bhqd,bhkd->bhqk", qo, kk) * scaling                # (B, Hq, w, H)
    qi = np.arange(H - w, H)[:, None]
    att = np.where(np.arange(H)[None, :] <= qi, att, -np.inf)
    att = att - att.max(-1, keepdims=True)
    att = np.exp(att)
    att = att / att.sum(-1, keepdims=True)
    sc = att[..., :-w].mean(-2)                                         # (B, Hq, H - w)
    pad = kernel // 2
    padded = np.pad(sc, [(0, 0), (0, 0), (pad, pad)])
    pooled = np.stack([padded[..., i:i + sc.shape[-1]] for i in range(kernel)], 0).sum(0) / kernel
    pooled = pooled.reshape(B, Hkv, rep, H - w).mean(2)
    out = np.empty((B, Hkv, H))
    out[..., :H - w] = pooled
    out[..., H - w:] = pooled.max() + 1.0
    return out


def decode_step_probs(q: np.ndarray, scaling: float, k_packed: np.ndarray, k_exact: np.ndarray) -> np.ndarray:
    """One decode step's attention probabilities of the packed (dequantised) keys, float64.

    q (B, Hq, Tq, d); k_packed (B, Hkv, n, d) the dequantised packed keys; k_exact (B, Hkv, e, d)
    the exact rows, all visible.  The softmax runs over packed + exact keys (as chunked_attention
    does, STRATA_KV.py:660-670); the returned probabilities are those of the packed keys,
    (B, Hq, Tq, n)."""
    B, Hq, Tq, d = q.shape
    rep = Hq // k_packed.shape[1]
    kk = rep_heads(np.concatenate([k_packed, k_exact], 2).astype(np.float64), rep)
    s = np.einsum("bhqd,bhkd->bhqk", q.astype(np.float64) * scaling, kk)
    s = s - s.max(-1, keepdims=True)
    p = np.exp(s)
    p = p / p.sum(-1, keepdims=True)
    return p[..., :k_packed.shape[2]]


def accumulate_decode_scores(scores: np.ndarray, probs: np.ndarray, weight: float) -> np.ndarray:
    """scores (B, Hkv, n) += weight * sum over the query heads of each KV group and the step's
    query tokens of probs (B, Hq, Tq, n).  With weight = 1 / (rep * Tq * steps) the result after
    all steps is the mean probability per KV head, as snapkv_scores averages (mean over queries,
    then over the group's heads)."""
    B, Hkv, n = scores.shape
    rep = probs.shape[1] // Hkv
    return scores + weight * probs.reshape(B, Hkv, rep, -1, n).sum((2, 3))


def topk_retain(scores: np.ndarray, k: int) -> np.ndarray:
    """Indices of the k largest scores per row (..., n), in increasing position order; among
    scores equal to the k-th largest the lowest positions are kept.  (..., k) int64."""
    n = scores.shape[-1]
    k = min(k, n)
    flat = scores.reshape(-1, n)
    out = np.empty((flat.shape[0], k), np.int64)
    for i, row in enumerate(flat):
        order = np.lexsort((np.arange(n), -row.astype(np.float64)))     # score desc, position asc
        out[i] = np.sort(order[:k])
    return out.reshape(scores.shape[:-1] + (k,))
