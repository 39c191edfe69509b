"""Pins the eviction oracle (oracle/evict.py) independently of itself (CPU).

* snapkv_scores: a per-(head, query, key) float64 loop with scipy's softmax, and the pooling by
  torch.nn.functional.avg_pool1d -- the routine the reference calls (STRATA_KV.py:952);
* decode_step_probs: the probabilities read back through chunked_attention with one-hot values
  (out = p @ V = p), and they sum with the exact rows' mass to one;
* accumulate_decode_scores: a mean over steps and the group's heads;
* topk_retain: a brute-force sort with explicit (score desc, position asc) keys, on data with
  many ties.
"""
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
