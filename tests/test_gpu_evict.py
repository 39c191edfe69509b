"""Eviction path on the GPU against the CPU oracle (oracle/evict.py).

* top-k retention: bit-exact retained positions (position order, lowest positions among ties at
  the k-th score) on random, tied, constant and signed rows of ragged lengths;
* decode-time score accumulation: probabilities of the packed tokens summed over the query
  heads of each KV group, over several steps, for 1, 4 and 8 rows per KV head (rtol 2e-4 in
  fp32; rtol 1e-3 in bf16, where the exact rows and q are bf16 values the oracle sees unchanged
  and the logits use the same fp32-level operand split, so the bar only absorbs the exp2 and
  normalisation rounding of a 16-bit-output instantiation);
* top-k rows longer than 65536 (the general multi-pass kernel, e.g. a 131k-token C5 context);
* gather + dequantise of retained rows: bit-exact against kivi_quant's xhat (fp32);
* a reduced C4: keys with a 1% +3 shift, scores over 4 decode steps, top-k, decode over the
  retained set plus the recent window.  Retained sets equal the oracle's except for positions
  whose oracle score lies within 1e-4 (relative) of the k-th score; outputs within 2e-3.
"""
import numpy as np
import pytest
import torch

import oracle.kivi as ok
from oracle.attention import chunked_attention
from oracle.evict import accumulate_decode_scores, decode_step_probs, topk_retain

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("split", [True, False], ids=["split", "one_wg"])
@pytest.mark.parametrize("n,k", [(1, 1), (100, 7), (1023, 1023), (1024, 300), (5000, 2048), (65280, 2048)])
def test_topk_retain_bit_exact(n, k, split):
    import kvq
    rng = np.random.default_rng(n + k)
    rows = np.stack([
        rng.random(n, dtype=np.float32) * 1e-3,                             # distinct
        rng.integers(0, 5, n).astype(np.float32) * 0.25,                    # heavy ties
        np.full(n, 3.0, np.float32),                                        # all equal
        (rng.standard_normal(n) * 10).astype(np.float32),                   # signed
        (1.0 + rng.integers(0, 3000, n) * 2.0 ** -23).astype(np.float32),   # keys span < 12 bits
        (1.0 + rng.integers(0, 1 << 13, n) * 2.0 ** -23).astype(np.float32),  # span 13 bits
        rng.choice(np.array([-np.inf, np.inf, -3.4e38, 3.4e38, 0.0, 1e-45, -1e-45, 1.0], np.float32), n),
    ])
    got = kvq.topk_retain(torch.from_numpy(rows).cuda(), k, split=split).cpu().numpy()
    want = topk_retain(rows, k)
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("split", [True, False], ids=["split", "one_wg"])
@pytest.mark.parametrize("n,k", [(65537, 2048), (131072, 2048)])
def test_topk_retain_long_rows(n, k, split):
    """Rows beyond 65536 scores take the general kernel: distinct, tied-at-the-k-th (planted) and
    equal rows, bit-exact against the full-sort oracle."""
    import kvq
    rng = np.random.default_rng(n)
    distinct = rng.random(n, dtype=np.float32)
    tied = (rng.random(n, dtype=np.float32) * 0.5).astype(np.float32)
    hot = rng.choice(n, 3 * k, replace=False)
    tied[hot[:k // 2]] = 0.9                                            # clearly kept
    tied[hot[k // 2:]] = 0.75                                           # 2.5k ties straddle the k-th
    c4_like = (rng.lognormal(-11.0, 1.0, n)).astype(np.float32)          # probability-sized scores
    rows = np.stack([distinct, tied, np.full(n, 0.5, np.float32), c4_like])
    got = kvq.topk_retain(torch.from_numpy(rows).cuda(), k, split=split).cpu().numpy()
    want = topk_retain(rows, k)
    np.testing.assert_array_equal(got, want)


def test_topk_retain_split_workspace_reuse_and_strided_rows():
    """The split selection with one caller workspace over several calls (no clearing between them)
    on rows read through a stride wider than n, k from 1 to n: bit-exact against the oracle; a
    workspace one word short is refused."""
    import kvq
    rng = np.random.default_rng(7)
    n, rows_n = 20000, 6
    wide = np.zeros((rows_n, n + 37), np.float32)
    wide[:, :n] = rng.lognormal(-9.0, 2.0, (rows_n, n)).astype(np.float32)
    wide[1, :n] = np.round(wide[1, :n] * 1e4).astype(np.float32)                 # many ties
    wide[2, rng.choice(n, 50, replace=False)] = np.inf
    dev = torch.from_numpy(wide).cuda()[:, :n]
    assert dev.stride(0) == n + 37
    words = kvq.topk_workspace_words(rows_n, n)
    assert words > 0
    ws = torch.empty(words, dtype=torch.int32, device="cuda")
    for k in (1, 50, 2048, 19999, n):
        got = kvq.topk_retain(dev, k, workspace=ws).cpu().numpy()
        np.testing.assert_array_equal(got, topk_retain(wide[:, :n], k))
    with pytest.raises(ValueError):
        kvq.topk_retain(dev, 10, workspace=ws[:words - 1])
    assert kvq.topk_workspace_words(rows_n, 4096) == 0                     # one-workgroup rows


def _packed(B, Hkv, T, W, gk, gv, seed, dtype=torch.float32, shift_frac=0.0):
    import kvq
    g = torch.Generator().manual_seed(seed)
    d = 128
    K = torch.randn((B, Hkv, T, d), generator=g)
    V = torch.randn((B, Hkv, T, d), generator=g)
    if shift_frac:
        n_shift = max(1, int(shift_frac * T))
        for b in range(B):
            for h in range(Hkv):
                K[b, h, torch.randperm(T - W, generator=g)[:n_shift]] += 3.0
    K, V = K.to(dtype), V.to(dtype)
    cache = kvq.PackedKIVICache.from_context(K.cuda(), V.cuda(), window=W, group_k=gk, group_v=gv)
    Kf, Vf = K.float().numpy(), V.float().numpy()
    kq, vq = ok.kivi_quant(Kf, 4, gk, True, 0), ok.kivi_quant(Vf, 4, gv, False, 0)
    n_q = T - W
    kh = ok.kivi_dequant(kq["codes"], kq["lo"], kq["scale"], gk, True)[:, :, :n_q]
    vh = ok.kivi_dequant(vq["codes"][:, :, :n_q], vq["lo"][:, :, :n_q], vq["scale"][:, :, :n_q], gv, False)
    return cache, K, V, kh, vh, g


@pytest.mark.parametrize("Hq,Hkv,Tq,dtype", [(8, 8, 1, torch.float32), (8, 2, 1, torch.float32),
                                             (8, 2, 2, torch.float32), (16, 4, 1, torch.bfloat16),
                                             (8, 2, 2, torch.bfloat16), (8, 8, 1, torch.bfloat16)])
def test_decode_score_accumulation(Hq, Hkv, Tq, dtype):
    """The score pass kivi_score_split<R, GV, DT> for fp32 and for bf16 (the C4 workload's type;
    Hq 16 over Hkv 4 is its rep 4 at Tq 1)."""
    import kvq
    B, T, W, gk, gv, d, steps = 2, 1200, 64, 64, 64, 128, 3
    cache, K, V, kh, vh, g = _packed(B, Hkv, T, W, gk, gv, seed=Hq + Hkv + Tq, dtype=dtype)
    rep = Hq // Hkv
    n_q = T - W
    scores = torch.zeros((B, Hkv, n_q + 5), dtype=torch.float32, device="cuda")   # row stride > n_q
    want = np.zeros((B, Hkv, n_q))
    w = 1.0 / (rep * Tq * steps)
    for _ in range(steps):
        q = torch.randn((B, Hq, Tq, d), generator=g).to(dtype)
        kvq.kivi_decode(q.cuda(), d ** -0.5, cache, scores=scores, score_weight=w)
        p = decode_step_probs(q.float().numpy(), d ** -0.5, kh, K[:, :, n_q:].float().numpy())
        want = accumulate_decode_scores(want, p, w)
    got = scores[..., :n_q].cpu().numpy()
    assert np.all(scores[..., n_q:].cpu().numpy() == 0.0)
    rtol = 2e-4 if dtype == torch.float32 else 1e-3
    np.testing.assert_allclose(got, want, rtol=rtol, atol=1e-9)


@pytest.mark.parametrize("Hq,Hkv,Tq,T,dtype", [(8, 8, 1, 1200, torch.float32), (8, 4, 1, 1111, torch.float32),
                                               (16, 4, 1, 2077, torch.bfloat16), (8, 2, 2, 1300, torch.bfloat16),
                                               (16, 2, 1, 999, torch.bfloat16)])
def test_scored_step_spill_equals_score_pass(Hq, Hkv, Tq, T, dtype):
    """A scored step with a score workspace (the split spills its logits, score_from_logits sums them)
    and with a plain workspace (the score pass reads the keys again): outputs and scores bit-equal
    over three steps, R = 1, 2, 4, 8, packed lengths not a multiple of 32."""
    import kvq
    B, W, gk, gv, d, steps = 2, 40, 64, 64, 128, 3
    cache, K, V, kh, vh, g = _packed(B, Hkv, T, W, gk, gv, seed=T + Hq, dtype=dtype)
    n_q = T - W
    args = (B, Hq, Hkv, Tq, d, cache.n_q, cache.n_exact, gk, gv)
    ws_spill = torch.zeros((kvq.score_workspace_floats(*args),), dtype=torch.float32, device="cuda")
    ws_plain = torch.zeros((kvq.workspace_floats(*args),), dtype=torch.float32, device="cuda")
    assert ws_spill.numel() > ws_plain.numel()
    sc_a = torch.zeros((B, Hkv, n_q), dtype=torch.float32, device="cuda")
    sc_b = torch.zeros_like(sc_a)
    w = 1.0 / ((Hq // Hkv) * Tq * steps)
    for _ in range(steps):
        q = torch.randn((B, Hq, Tq, d), generator=g).to(dtype).cuda()
        oa = kvq.kivi_decode(q, d ** -0.5, cache, workspace=ws_spill, scores=sc_a, score_weight=w)
        ob = kvq.kivi_decode(q, d ** -0.5, cache, workspace=ws_plain, scores=sc_b, score_weight=w)
        assert torch.equal(oa, ob)
    assert torch.equal(sc_a, sc_b)
    assert float(sc_a.sum()) > 0


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_gather_dequant_bit_exact(dtype):
    """Retained rows equal kivi_quant's xhat (fp32, then rounded once to the output type); an index
    outside [0, n_q) gives a NaN row."""
    import kvq
    B, Hkv, T, W, gk, gv = 2, 2, 1000, 40, 64, 32
    cache, K, V, kh, vh, g = _packed(B, Hkv, T, W, gk, gv, seed=7)
    n_q = T - W
    idx = torch.stack([torch.sort(torch.randperm(n_q, generator=g)[:77]).values for _ in range(B * Hkv)])
    idx[0, -1] = n_q - 1                                                   # last row of the last tile
    idx[1, 3] = -1                                                         # outside the packed rows
    idx[2, 5] = n_q
    idx = idx.reshape(B, Hkv, 77).to(torch.int32)
    ko, vo = kvq.gather_dequant(cache, idx.cuda(), dtype)
    ii = idx.long().numpy()
    bad = (ii < 0) | (ii >= n_q)
    jj = np.where(bad, 0, ii)
    want_k = torch.from_numpy(np.take_along_axis(kh.astype(np.float32), jj[..., None], 2)).to(dtype).float().numpy()
    want_v = torch.from_numpy(np.take_along_axis(vh.astype(np.float32), jj[..., None], 2)).to(dtype).float().numpy()
    want_k[bad] = np.nan
    want_v[bad] = np.nan
    np.testing.assert_array_equal(ko.float().cpu().numpy(), want_k)
    np.testing.assert_array_equal(vo.float().cpu().numpy(), want_v)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_c4_reduced_eviction_end_to_end(dtype):
    """fp32 and bf16 (the C4 workload's type): scores over 4 steps, top-k, retained decode."""
    import kvq
    B, Hq, Hkv, T, W, gk, gv, d, steps, keep = 2, 16, 4, 8448, 256, 64, 64, 128, 4, 512
    cache, K, V, kh, vh, g = _packed(B, Hkv, T, W, gk, gv, seed=21, dtype=dtype, shift_frac=0.01)
    tol_rel, tol_out = (1e-4, 2e-3) if dtype == torch.float32 else (1e-3, 1e-2)
    n_q = T - W
    rep = Hq // Hkv
    scores = torch.zeros((B, Hkv, n_q), dtype=torch.float32, device="cuda")
    want = np.zeros((B, Hkv, n_q))
    for _ in range(steps):
        q = torch.randn((B, Hq, 1, d), generator=g).to(dtype)
        kvq.kivi_decode(q.cuda(), d ** -0.5, cache, scores=scores, score_weight=1.0 / (rep * steps))
        want = accumulate_decode_scores(want, decode_step_probs(q.float().numpy(), d ** -0.5, kh,
                                                                K[:, :, n_q:].float().numpy()),
                                        1.0 / (rep * steps))
    idx = kvq.topk_retain(scores, keep)
    got = idx.cpu().numpy()
    ref = topk_retain(want, keep)
    for b in range(B):
        for h in range(Hkv):
            kth = np.sort(want[b, h])[-keep]
            near = set(np.nonzero(np.abs(want[b, h] - kth) <= tol_rel * kth)[0].tolist())
            diff = set(got[b, h].tolist()) ^ set(ref[b, h].tolist())
            assert diff <= near, (b, h, sorted(diff - near)[:10])
    # decode over the retained set + the recent window
    rc = kvq.retained_cache(cache, idx)
    q = torch.randn((B, Hq, 1, d), generator=g).to(dtype)
    out = kvq.kivi_decode(q.cuda(), d ** -0.5, rc).float().cpu().numpy()
    ii = got.astype(np.int64)
    # the retained rows are kivi_quant's xhat rounded once to the cache dtype (gather_dequant)
    kg = torch.from_numpy(np.take_along_axis(kh, ii[..., None], 2).astype(np.float32)).to(dtype).float().numpy()
    vg = torch.from_numpy(np.take_along_axis(vh, ii[..., None], 2).astype(np.float32)).to(dtype).float().numpy()
    kk = np.concatenate([kg, K[:, :, n_q:].float().numpy()], 2)
    vv = np.concatenate([vg, V[:, :, n_q:].float().numpy()], 2)
    ref_out = chunked_attention(q.float().numpy(), d ** -0.5, np.array([T]), kk, vv, np.zeros(kk.shape[2], int),
                                np.full(kk.shape[2], 1 << 40), None)
    assert float(np.abs(out - ref_out).max()) <= tol_out


@pytest.mark.parametrize("Hq,Hkv,Tq,dtype,k,gk,gv", [(16, 4, 1, torch.bfloat16, 512, 64, 32),
                                                     (8, 2, 2, torch.float32, 300, 64, 32),
                                                     (8, 8, 1, torch.float32, 77, 64, 32),
                                                     (32, 4, 3, torch.bfloat16, 1000, 64, 32),
                                                     (8, 2, 1, torch.float32, 0, 64, 32),
                                                     (8, 1, 1, torch.float32, 2900, 64, 32),
                                                     (16, 2, 1, torch.float16, 700, 32, 128),
                                                     (8, 4, 1, torch.float16, 257, 128, 64)])
def test_retained_decode_against_oracle(Hq, Hkv, Tq, dtype, k, gk, gv):
    """The fused retained decode (kvq.retained_decode): the kept rows read from the packed cache as
    kivi_quant's xhat in fp32, the window exact; positions outside [0, n_q) are masked rows.
    Against chunked_attention over exactly those rows (2e-3 fp32, 1e-2 bf16), and against the
    gathered path retained_cache + kivi_decode (bf16 rows there, so the same bars)."""
    import kvq
    B, T, W, d = 2, 3000, 128, 128
    cache, K, V, kh, vh, g = _packed(B, Hkv, T, W, gk, gv, seed=Hq + Tq + k, dtype=dtype)
    n_q = T - W
    k = min(k, n_q)
    idx = torch.stack([torch.sort(torch.randperm(n_q, generator=g)[:k]).values for _ in range(B * Hkv)])
    idx = idx.reshape(B, Hkv, k).to(torch.int32)
    if k:
        idx[0, 0, -1] = n_q                                             # masked rows
        idx[B - 1, Hkv - 1, 0] = -1
    q = torch.randn((B, Hq, Tq, d), generator=g).to(dtype)
    qpos = torch.arange(T, T + Tq)
    out = kvq.retained_decode(q.cuda(), d ** -0.5, cache, idx.cuda(), q_pos=qpos.cuda())
    assert out.shape == (B, Tq, Hq, d) and out.dtype == dtype
    got = out.float().cpu().numpy()
    ii = idx.long().numpy()
    bad = (ii < 0) | (ii >= n_q)
    jj = np.where(bad, 0, ii)
    kk = np.concatenate([np.take_along_axis(kh, jj[..., None], 2), K[:, :, n_q:].float().numpy()], 2)
    vv = np.concatenate([np.take_along_axis(vh, jj[..., None], 2), V[:, :, n_q:].float().numpy()], 2)
    hide = np.full((B, Hkv, k + W), 1 << 40)
    hide[:, :, :k][bad] = 0                                             # never readable
    ref = chunked_attention(q.float().numpy(), d ** -0.5, qpos.numpy(), kk, vv, np.zeros(k + W, int), hide, None)
    tol = 2e-3 if dtype == torch.float32 else 1e-2
    err = float(np.abs(got - ref).max())
    print(f"retained Hq {Hq} Hkv {Hkv} Tq {Tq} {dtype} k {k} groups {gk}/{gv}: max-abs-err {err:.3e}", flush=True)
    assert err <= tol, err
    if not bad.any():
        via = kvq.kivi_decode(q.cuda(), d ** -0.5, kvq.retained_cache(cache, idx.cuda())).float().cpu().numpy()
        assert float(np.abs(via - got).max()) <= tol
    # a caller-owned output and workspace; a second call with the same workspace gives the same bits
    ws = torch.empty((kvq.retained_workspace_floats(q, cache, idx),), dtype=torch.float32, device="cuda")
    o2 = torch.empty_like(out)
    kvq.retained_decode(q.cuda(), d ** -0.5, cache, idx.cuda(), q_pos=qpos.cuda(), out=o2, workspace=ws)
    assert torch.equal(o2, out)


def test_retained_decode_rejects_bad_inputs():
    import kvq
    cache, K, V, kh, vh, g = _packed(1, 2, 600, 64, 32, 32, seed=3)
    q = torch.randn((1, 8, 1, 128), generator=g).cuda()
    with pytest.raises(ValueError):
        kvq.retained_decode(q, 0.1, cache, torch.zeros((1, 2, 5), dtype=torch.int64, device="cuda"))
    with pytest.raises(ValueError):
        kvq.retained_decode(q, 0.1, cache, torch.zeros((1, 3, 5), dtype=torch.int32, device="cuda"))
    with pytest.raises(TypeError):
        kvq.retained_decode(q.bfloat16(), 0.1, cache, torch.zeros((1, 2, 5), dtype=torch.int32, device="cuda"))
    idx = torch.zeros((1, 2, 5), dtype=torch.int32, device="cuda")
    with pytest.raises(kvq.KVQError):
        kvq.retained_decode(q, 0.1, cache, idx, workspace=torch.empty((4,), dtype=torch.float32, device="cuda"))
