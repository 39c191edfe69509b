"""Pins the numpy restatement of chunked_attention / KIVI decode (oracle/attention.py).

Against torch's scaled_dot_product_attention on the same rows (the reference's own harness
check), a per-row brute-force loop, and invariants that catch index or head-order mistakes.
"""
import numpy as np
import torch
import torch.nn.functional as F

from oracle.attention import chunked_attention, kivi_decode_reference, lse_merge, rep_heads
from oracle.kivi import kivi_quant

BIG = 1 << 40


def _rand(shape, seed):
    return np.random.default_rng(seed).standard_normal(shape).astype(np.float32)


def test_chunked_attention_equals_sdpa_gqa():
    B, Hq, Hkv, Tq, T, d = 2, 8, 2, 3, 50, 16
    q, K, V = _rand((B, Hq, Tq, d), 1), _rand((B, Hkv, T, d), 2), _rand((B, Hkv, T, d), 3)
    sc = d ** -0.5
    qpos = np.arange(T - Tq, T)
    out = chunked_attention(q, sc, qpos, K, V, np.arange(T), np.full(T, BIG), None, chunk=2)
    mask = torch.arange(T)[None, :] <= torch.tensor(qpos)[:, None]
    ref = F.scaled_dot_product_attention(torch.tensor(q, dtype=torch.float64),
                                         torch.tensor(K, dtype=torch.float64).repeat_interleave(4, 1),
                                         torch.tensor(V, dtype=torch.float64).repeat_interleave(4, 1),
                                         attn_mask=mask, scale=sc).transpose(1, 2).numpy()
    np.testing.assert_allclose(out, ref, rtol=1e-10, atol=1e-12)


def test_token_entries_bruteforce_and_masking():
    B, Hq, Hkv, d = 1, 2, 1, 4
    q = _rand((B, Hq, 1, d), 4)
    K, V = _rand((B, Hkv, 3, d), 5), _rand((B, Hkv, 3, d), 6)
    tk, tv = _rand((B, Hkv, 4, d), 7), _rand((B, Hkv, 4, d), 8)
    tb = np.array([[[0.0, 0.3, -np.inf, 0.0]]])
    tau = np.array([0, 5, 0, 9])                      # entry 3 not yet visible at position 5
    hide = np.array([BIG, 4, BIG])                    # exact row 1 hidden from position 4
    out = chunked_attention(q, 0.5, np.array([5]), K, V, np.arange(3), hide, {"k": tk, "v": tv, "b": tb, "tau": tau})
    q, K, V, tk, tv = (a.astype(np.float64) for a in (q, K, V, tk, tv))
    for h in range(Hq):
        logits, vals = [], []
        for j in (0, 2):
            logits.append(0.5 * q[0, h, 0] @ K[0, 0, j]); vals.append(V[0, 0, j])
        for j, bj in ((0, 0.0), (1, 0.3)):
            logits.append(0.5 * q[0, h, 0] @ tk[0, 0, j] + bj); vals.append(tv[0, 0, j])
        w = np.exp(np.array(logits) - max(logits))
        want = (w[:, None] * np.array(vals)).sum(0) / w.sum()
        np.testing.assert_allclose(out[0, 0, h], want, rtol=1e-12)


def test_gqa_head_order():
    # KV head h must serve query heads h*rep..h*rep+rep-1 (HF repeat_kv order)
    B, Hkv, rep, T, d = 1, 3, 2, 5, 4
    V = np.zeros((B, Hkv, T, d), np.float32)
    for h in range(Hkv):
        V[0, h] = h + 1.0
    K = _rand((B, Hkv, T, d), 9)
    q = _rand((B, Hkv * rep, 1, d), 10)
    out = chunked_attention(q, 1.0, np.array([T]), K, V, np.arange(T), np.full(T, BIG), None)
    np.testing.assert_allclose(out[0, 0, :, 0], np.repeat(np.arange(1, Hkv + 1), rep), rtol=1e-12)
    assert rep_heads(np.arange(3)[None, :, None], 2).ravel().tolist() == [0, 0, 1, 1, 2, 2]


def test_kivi_decode_reference_is_dequant_then_sdpa():
    B, Hq, Hkv, T, d, W, G = 1, 4, 2, 96, 32, 16, 32
    q, K, V = _rand((B, Hq, 1, d), 11), _rand((B, Hkv, T, d), 12), _rand((B, Hkv, T, d), 13)
    kq, vq = kivi_quant(K, 4, G, True, 0), kivi_quant(V, 4, G, False, 0)
    n_q = T - W
    out = kivi_decode_reference(q, d ** -0.5, K[:, :, n_q:], V[:, :, n_q:], kq["codes"], kq["lo"], kq["scale"],
                                vq["codes"], vq["lo"], vq["scale"], G, G, n_q)
    Kmix = np.concatenate([kq["xhat"][:, :, :n_q], K[:, :, n_q:]], 2)
    Vmix = np.concatenate([vq["xhat"][:, :, :n_q], V[:, :, n_q:]], 2)
    ref = F.scaled_dot_product_attention(torch.tensor(q, dtype=torch.float64),
                                         torch.tensor(Kmix, dtype=torch.float64).repeat_interleave(2, 1),
                                         torch.tensor(Vmix, dtype=torch.float64).repeat_interleave(2, 1),
                                         scale=d ** -0.5).transpose(1, 2).numpy()
    np.testing.assert_allclose(out, ref, rtol=1e-9, atol=1e-12)


def test_lse_merge_exact():
    rng = np.random.default_rng(3)
    s = rng.standard_normal(40) * 3
    v = rng.standard_normal((40, 5))
    p = np.exp2(s - s.max())
    want = (p[:, None] * v).sum(0) / p.sum()
    parts = [(slice(0, 7)), slice(7, 30), slice(30, 40)]
    ms = np.array([s[x].max() for x in parts])
    ls = np.array([np.exp2(s[x] - s[x].max()).sum() for x in parts])
    accs = np.array([(np.exp2(s[x] - s[x].max())[:, None] * v[x]).sum(0) for x in parts])
    np.testing.assert_allclose(lse_merge(ms, ls, accs), want, rtol=1e-12)
