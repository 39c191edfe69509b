"""Decode attention over exact rows plus quantised token entries (numpy restatement).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Reference:
  * ``rep_heads`` / GQA order        STRATA_KV.py:527-529, 567-570
  * ``chunked_attention``            STRATA_KV.py:641-675
  * ``LayerState.attend``            STRATA_KV.py:716-719 (exact rows + visible token entries)
  * KIVI token entries               STRATA_KV.py:801-823 (xhat of the quantised rows, b = 0)

Pinning (tests/test_oracle_attention.py): against ``torch.nn.functional.
scaled_dot_product_attention`` on the same dequantised rows (the reference's own harness check,
STRATA_KV.py:2018-2049, documents harness == SDPA to 1.3e-5), against a per-row float64 loop on
tiny inputs, and by invariants (an entry with b = -inf or not yet visible changes nothing; all
weight on one row returns that row; GQA head order by a head-distinct value tensor).
"""
from __future__ import annotations

import numpy as np

from .kivi import kivi_dequant


def rep_heads(x: np.ndarray, rep: int) -> np.ndarray:
    """KV head h serves query heads h*rep .. h*rep+rep-1 (HF repeat_kv order), STRATA_KV.py:527-529."""
    return np.repeat(x, rep, axis=1)


def chunked_attention(q, scaling, q_pos, K, V, kv_pos, hide_at, tok, chunk=256,
                      dtype=np.float64) -> np.ndarray:
    """One softmax over exact rows (readable by query m iff kv_pos <= m < hide_at) and token entries
    (logit q.k + b, visible iff tau <= m).  q (B, Hq, Tq, d) -> out (B, Tq, Hq, d) in ``dtype``.
    STRATA_KV.py:641-675; hide_at is (Tk,) or per KV head (B, Hkv, Tk)."""
    B, Hq, Tq, d = q.shape
    rep = Hq // K.shape[1]
    Kr, Vr = rep_heads(K.astype(dtype), rep), rep_heads(V.astype(dtype), rep)
    kv_pos, hide_at = np.asarray(kv_pos), np.asarray(hide_at)
    if hide_at.ndim == 3:
        hide_at = rep_heads(hide_at, rep)[:, :, None, :]
    if tok is not None:
        tk, tv = rep_heads(tok["k"].astype(dtype), rep), rep_heads(tok["v"].astype(dtype), rep)
        tb = rep_heads(tok["b"].astype(dtype), rep)
        ttau = np.asarray(tok["tau"])
    out = np.empty((B, Hq, Tq, d), dtype=dtype)
    for s in range(0, Tq, chunk):
        qs = q[:, :, s:s + chunk].astype(dtype) * scaling
        qp = np.asarray(q_pos)[s:s + chunk]
        hid = hide_at if hide_at.ndim == 4 else hide_at[None, :]
        readable = (kv_pos[None, :] <= qp[:, None]) & (qp[:, None] < hid)
        blocks = [np.where(readable, qs @ np.swapaxes(Kr, -1, -2), -np.inf)]
        if tok is not None:
            vis = ttau[None, :] <= qp[:, None]
            blocks.append(np.where(vis, qs @ np.swapaxes(tk, -1, -2) + tb[:, :, None], -np.inf))
        logits = np.concatenate(blocks, -1)
        mx = logits.max(-1, keepdims=True)
        e = np.exp(logits - mx)
        p = e / e.sum(-1, keepdims=True)
        T0 = Kr.shape[2]
        o = p[..., :T0] @ Vr
        if tok is not None:
            o = o + p[..., T0:] @ tv
        out[:, :, s:s + chunk] = o
    return np.swapaxes(out, 1, 2)


def kivi_decode_reference(q, scaling, k_exact, v_exact, k_codes, k_lo, k_scale, v_codes, v_lo,
                          v_scale, group_k: int, group_v: int, n_q: int | None = None,
                          dtype=np.float64) -> np.ndarray:
    """Decode of one query step over a KIVI cache: ``n_q`` quantised rows (token entries: xhat of
    their codes, b = 0, visible) plus exact rows, the state LayerState.attend reads after a KIVI
    prefill (STRATA_KV.py:716-719 with KIVIMethod.entries 801-823).

    q (B, Hq, Tq, d); k_exact/v_exact (B, Hkv, n_e, d); codes (B, Hkv, >= n_q, d) uint8;
    k_lo/k_scale (B, Hkv, n_g, 1, d); v_lo/v_scale (B, Hkv, n, d/width, 1).
    Every row is visible to every query (a decode step reads the whole cache).
    Returns (B, Tq, Hq, d) in ``dtype``.
    """
    B, Hkv, n_all, d = k_codes.shape
    n_q = n_all if n_q is None else n_q
    kh = kivi_dequant(k_codes, k_lo, k_scale, group_k, True)[:, :, :n_q]
    vh = kivi_dequant(v_codes[:, :, :n_q], v_lo[:, :, :n_q], v_scale[:, :, :n_q], group_v, False)
    n_e = k_exact.shape[2]
    Tq = q.shape[2]
    big = 1 << 40
    tok = {"k": kh, "v": vh, "b": np.zeros((B, Hkv, n_q)), "tau": np.full(n_q, -1)}
    q_pos = np.full(Tq, n_q + n_e)
    return chunked_attention(q, scaling, q_pos, k_exact, v_exact, np.arange(n_e),
                             np.full(n_e, big), tok, dtype=dtype)


def lse_merge(ms, ls, accs):
    """Exact merge of flash-decoding partials (m, l, acc) in base 2: the combination
    StrataState.attend performs in base e (STRATA_KV.py:1784-1792).  ms, ls (S, ...);
    accs (S, ..., d) unnormalised value sums.  Returns the normalised output."""
    ms, ls, accs = (np.asarray(a, np.float64) for a in (ms, ls, accs))
    M = ms.max(0)
    w = np.exp2(ms - M)
    L = (w * ls).sum(0)
    return (w[..., None] * accs).sum(0) / L[..., None]
