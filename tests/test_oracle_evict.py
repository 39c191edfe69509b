"""Pins the eviction oracle (oracle/evict.py) independently of itself (CPU).

* snapkv_scores: a per-(head, query, key) float64 loop with scipy's softmax, and the pooling by
  torch.nn.functional.avg_pool1d -- the routine the reference calls (STRATA_KV.py:952);
* decode_step_probs: the probabilities read back through chunked_attention with one-hot values
  (out = p @ V = p), and they sum with the exact rows' mass to one;
* accumulate_decode_scores: a mean over steps and the group's heads;
* topk_retain: a brute-force sort with explicit (score desc, position asc) keys, on data with
  many ties.
"""
import math

import numpy as np
import pytest
import torch
from scipy.special import softmax

from oracle.attention import chunked_attention
from oracle.evict import accumulate_decode_scores, decode_step_probs, snapkv_scores, topk_retain


def test_snapkv_scores_brute_force():
    rng = np.random.default_rng(0)
    B, Hq, Hkv, H, d, w, ker = 1, 4, 2, 24, 8, 5, 3
    q = rng.standard_normal((B, Hq, H, d))
    k = rng.standard_normal((B, Hkv, H, d))
    scaling = d ** -0.5
    got = snapkv_scores(q, k, H, scaling, w, ker)
    rep = Hq // Hkv
    att = np.zeros((B, Hq, w, H - w))
    for hq in range(Hq):
        for i, m in enumerate(range(H - w, H)):
            logits = np.array([q[0, hq, m] @ k[0, hq // rep, j] * scaling if j <= m else -np.inf for j in range(H)])
            att[0, hq, i] = softmax(logits)[:H - w]
    sc = torch.from_numpy(att.mean(2))
    pooled = torch.nn.functional.avg_pool1d(sc, kernel_size=ker, padding=ker // 2, stride=1).numpy()
    want = pooled.reshape(B, Hkv, rep, H - w).mean(2)
    np.testing.assert_allclose(got[..., :H - w], want, rtol=1e-12, atol=1e-15)
    assert np.all(got[..., H - w:] == want.max() + 1.0)


def test_decode_step_probs_via_chunked_attention():
    rng = np.random.default_rng(1)
    B, Hq, Hkv, n, e, d = 1, 4, 2, 20, 6, 32
    q = rng.standard_normal((B, Hq, 2, d))
    kp = rng.standard_normal((B, Hkv, n, d))
    ke = rng.standard_normal((B, Hkv, e, d))
    p = decode_step_probs(q, 0.3, kp, ke)
    # one-hot values: chunked_attention returns the probabilities themselves
    eye = np.eye(d)[None, None, :n + e].repeat(Hkv, 1)
    tok = {"k": kp, "v": eye[:, :, :n], "b": np.zeros((B, Hkv, n)), "tau": np.full(n, -1)}
    out = chunked_attention(q, 0.3, np.array([100, 100]), ke, eye[:, :, n:n + e], np.zeros(e, int),
                            np.full(e, 1 << 40), tok)                       # (B, Tq, Hq, d)
    probs_tok = out.transpose(0, 2, 1, 3)[..., :n]
    np.testing.assert_allclose(p, probs_tok, rtol=1e-12, atol=1e-15)
    exact_mass = out.transpose(0, 2, 1, 3)[..., n:n + e].sum(-1)
    np.testing.assert_allclose(p.sum(-1) + exact_mass, 1.0, rtol=1e-12)


def test_accumulate_is_a_mean():
    rng = np.random.default_rng(2)
    B, Hq, Hkv, Tq, n, steps = 2, 8, 2, 1, 10, 3
    rep = Hq // Hkv
    sc = np.zeros((B, Hkv, n))
    allp = []
    for _ in range(steps):
        p = rng.random((B, Hq, Tq, n))
        allp.append(p)
        sc = accumulate_decode_scores(sc, p, 1.0 / (rep * Tq * steps))
    want = np.stack(allp).reshape(steps, B, Hkv, rep, Tq, n).mean((0, 3, 4))
    np.testing.assert_allclose(sc, want, rtol=1e-12)


@pytest.mark.parametrize("k", [1, 7, 50, 64])
def test_topk_retain_brute_force_with_ties(k):
    rng = np.random.default_rng(3 + k)
    rows = rng.integers(0, 6, (3, 64)).astype(np.float32)     # many ties
    rows[1] = 2.0                                              # all equal
    got = topk_retain(rows, k)
    for r, row in enumerate(rows):
        order = sorted(range(64), key=lambda i: (-float(row[i]), i))
        assert list(got[r]) == sorted(order[:k])


def test_chunk_share_by_per_query_loop():
    """finalize_chunk's share against an explicit loop: each query's softmax over the keys (float64
    exp / sum), summed over queries, divided by nq."""
    from oracle.evict import chunk_share
    rng = np.random.default_rng(5)
    B, H, nq, C, d = 2, 3, 5, 7, 4
    q, k = rng.standard_normal((B, H, nq, d)), rng.standard_normal((B, H, C, d))
    want = np.zeros((B, H, C))
    for b in range(B):
        for h in range(H):
            for i in range(nq):
                logits = [sum(q[b, h, i, e] * k[b, h, c, e] for e in range(d)) for c in range(C)]
                mx = max(logits)
                ex = [math.exp(x - mx) for x in logits]
                for c in range(C):
                    want[b, h, c] += ex[c] / sum(ex) / nq
    np.testing.assert_allclose(chunk_share(q, k), want, rtol=1e-12, atol=0)
    assert np.allclose(chunk_share(q, k).sum(-1), 1.0)


def test_absmax_fake_quant_known_answers():
    """absmax_quant at 8 and 4 bits on hand-checked rows: the scale is the fp16 value of
    max|x| / qmax (float32 quotient), codes round half to even, and the scale floor 2^-24."""
    from oracle.evict import absmax_fake_quant
    x = np.array([[1.0, -0.5, 0.25, 0.0]], np.float32)
    s8 = np.float32(np.float16(np.float32(1.0) / np.float32(127)))       # 0.007873535...
    assert s8 == np.float32(0.007873535)
    got = absmax_fake_quant(x, 8)
    np.testing.assert_array_equal(got, (np.rint(x / s8) * s8).astype(np.float32))
    assert got[0, 0] == np.float32(127) * s8 and got[0, 1] == np.float32(-64) * s8   # -63.5 -> -64 (half even)
    # 4 bits: qmax 7, s = fp16(2/7) = 0.28564453 (below 2/7), so 1.0 / s = 3.5009 -> 4; with the
    # float32 scale 2/7 unrounded the quotient would be 3.4999999 -> 3 (a dropped fp16 rounding fails)
    x4 = np.array([[2.0, 1.0, -2.0, 0.7]], np.float32)
    s4 = np.float32(np.float16(np.float32(2.0) / np.float32(7)))
    np.testing.assert_array_equal(absmax_fake_quant(x4, 4), (np.clip(np.rint(x4 / s4), -7, 7) * s4).astype(np.float32))
    assert s4 == np.float32(0.28564453) and absmax_fake_quant(x4, 4)[0, 1] == 4 * s4
    # an all-zero row keeps the 2^-24 floor and zero codes; bits >= 16 returns the input
    np.testing.assert_array_equal(absmax_fake_quant(np.zeros((1, 4), np.float32), 8), np.zeros((1, 4)))
    assert absmax_fake_quant(x, 16) is x


def test_finalize_chunk_keeps_largest_share_in_position_order():
    from oracle.evict import finalize_chunk
    rng = np.random.default_rng(9)
    B, H, nq, C, d = 1, 2, 6, 32, 8
    q, k, v = (rng.standard_normal((B, H, n, d)).astype(np.float32) for n in (nq, C, C))
    out = finalize_chunk(k, v, q, 5, 16)
    for h in range(H):
        order = np.argsort(-out["share"][0, h], kind="stable")[:5]
        assert out["idx"][0, h].tolist() == sorted(order.tolist())
        np.testing.assert_array_equal(out["k"][0, h], k[0, h, out["idx"][0, h]])


def test_streaming_and_keep_hides():
    from oracle.evict import BIG, keep_hide, streaming_hide
    hide = streaming_hide(100, 20)                 # sinks 0..3 and the last 16 kept
    kept = np.nonzero(hide == BIG)[0]
    assert kept.tolist() == [0, 1, 2, 3] + list(range(84, 100)) and (hide[4:84] == 100).all()
    assert (np.nonzero(streaming_hide(10, 3)[4:] == BIG)[0] + 4).tolist() == [9]   # recent = max(1, keep - 4)
    kh = keep_hide(np.array([[[1, 4], [0, 2]]]), 5)
    assert kh.tolist() == [[[5, BIG, 5, 5, BIG], [BIG, 5, BIG, 5, 5]]]
