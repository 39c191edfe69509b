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


# ---- chunk-local selection (finalize_chunk, STRATA_KV.py:573-592) -----------------------------

def chunk_share(qref: np.ndarray, k: np.ndarray) -> np.ndarray:
    """qref (B, H, nq, d) scaled observed queries, k (B, H, C, d) -> (B, H, C) float64: each query's
    softmax over the chunk's keys, averaged over the queries (STRATA_KV.py:581-582)."""
    s = np.einsum("bhqd,bhcd->bhqc", qref.astype(np.float64), k.astype(np.float64))
    s = np.exp(s - s.max(-1, keepdims=True))
    return (s / s.sum(-1, keepdims=True)).mean(2)


def absmax_fake_quant(x: np.ndarray, bits: int) -> np.ndarray:
    """fake_quant_tokens (STRATA_KV.py:556-563) in float32 as the reference computes it:
    absmax_quant's s = max(fp16(clamp(max|x| / qmax)), 2^-24) per vector (549-554), codes
    clamp(round_half_even(x / s), -qmax, qmax), returned codes * s; bits >= 16 keeps x."""
    if bits >= 16:
        return x
    x = x.astype(np.float32)
    qmax = np.float32(2 ** (bits - 1) - 1)
    ratio = (np.abs(x).max(-1, keepdims=True) / qmax).astype(np.float32)
    s = np.maximum(np.clip(ratio, -65504, 65504).astype(np.float16).astype(np.float32), np.float32(2.0 ** -24))
    c = np.clip(np.rint(x / s), -qmax, qmax).astype(np.float32)
    return (c * s).astype(np.float32)


def finalize_chunk(k: np.ndarray, v: np.ndarray, qref: np.ndarray, m: int, keep_bits: int) -> dict:
    """The top-k families' finalize_chunk (STRATA_KV.py:573-592): the m tokens of largest chunk
    share per (b, h) in position order (ties at the m-th: lowest positions, as topk_retain), their
    rows gathered and stored at keep_bits.  {k, v, idx, share}."""
    share = chunk_share(qref, k)
    idx = topk_retain(share, m)
    d = k.shape[-1]
    gk = np.take_along_axis(k.astype(np.float32), idx[..., None].repeat(d, -1), 2)
    gv = np.take_along_axis(v.astype(np.float32), idx[..., None].repeat(d, -1), 2)
    return {"k": absmax_fake_quant(gk, keep_bits), "v": absmax_fake_quant(gv, keep_bits), "idx": idx,
            "share": share}


# ---- keep sets of the exact-row eviction families ------------------------------------------

BIG = 1 << 40


def streaming_hide(H: int, keep: int, n_sink: int = 4) -> np.ndarray:
    """hide of a frozen StreamingLLMMethod (STRATA_KV.py:1055-1059) over the context positions
    [0, H): H for dropped positions (n_sink <= p < H - recent), BIG for kept ones,
    recent = max(1, keep - n_sink)."""
    pc = np.arange(H)
    recent = max(1, keep - n_sink)
    drop = (pc >= n_sink) & (pc < H - recent)
    return np.where(drop, H, BIG)


def keep_hide(keep: np.ndarray, H: int) -> np.ndarray:
    """Per-KV-head hide of SnapKVMethod (STRATA_KV.py:976-980): keep (B, Hkv, m) kept positions ->
    (B, Hkv, H) BIG where kept, H elsewhere."""
    B, Hkv, _ = keep.shape
    hide = np.full((B, Hkv, H), H, np.int64)
    np.put_along_axis(hide, keep.astype(np.int64), BIG, -1)
    return hide
