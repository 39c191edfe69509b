"""C3, C4 and C5 at their full BASELINE sizes on the GPU, through the plans their bench workloads
time, against the CPU oracle on sampled (batch, KV head) pairs (the oracle of a whole layer would
take minutes; the pairs are first, last and interior ones, which land on different XCDs and split
slots).

* C3 (B 8, Hq 32, Hkv 8, T 16384, 2/4/8-bit blocks by the C3 width rule): the class-major plan of
  12 splits per (b, h); outputs within the bf16 bar (1e-2) of oracle.mixed.
* C4 (B 4, Hq 32, Hkv 8, T 65536 = 65280 packed + 256 exact, group 64, 1% of keys +3): 32 scored
  decode steps, top-k 2048, the decode over the retained rows plus the window.  Scores within 1e-4
  of the float64 oracle (relative to the row's largest score); retained sets equal to the oracle's
  top-k of its own scores except where both candidates tie with the oracle's k-th score within
  1e-4 (torch.topk leaves tie order unspecified); the retained decode within 1e-2.
* C5 (B 1, Hq 64, Hkv 8, T 131072, DCT blocks of 64, 16 coefficients at 4 bits): outputs within
  1e-2 of oracle.dct.
"""
import numpy as np
import pytest
import torch

import oracle.kivi as ok
import oracle.mixed as om
from oracle.attention import chunked_attention
from oracle.dct import dct_decode, dct_encode
from oracle.evict import accumulate_decode_scores, decode_step_probs, topk_retain

pytestmark = pytest.mark.gpu


def test_c3_full_size_sampled_pairs():
    import kvq
    from kvq.synth import C3, c3_inputs
    s = C3
    q, K, V, imp = c3_inputs("cuda")
    widths = kvq.c3_widths(imp)
    cache = kvq.MixedKIVICache.from_context(K, V, widths, window=0)
    assert cache.nb == s.T // 64
    rep = s.Hq // s.Hkv
    assert kvq.mixed_workspace_floats(s.B, s.Hq, s.Hkv, 1, s.d, cache.nb, 0) == s.B * s.Hkv * 12 * rep * (s.d + 2)
    out = kvq.mixed_decode(q, s.d ** -0.5, cache).float().cpu().numpy()
    w = widths.to(torch.int64).cpu().numpy()
    worst = 0.0
    for b, h in [(0, 0), (7, 7), (3, 5), (5, 2)]:
        m = om.mixed_quant(K[b:b + 1, h:h + 1].float().cpu().numpy(), V[b:b + 1, h:h + 1].float().cpu().numpy(),
                           w[b:b + 1, h:h + 1])
        ref = om.mixed_decode(q[b:b + 1, h * rep:(h + 1) * rep].float().cpu().numpy(), s.d ** -0.5, m["xk"], m["xv"])
        err = float(np.abs(out[b, 0, h * rep:(h + 1) * rep] - ref[0, 0]).max())
        print(f"C3 full size (b={b}, h={h}): max-abs-err {err:.3e}", flush=True)
        worst = max(worst, err)
    assert worst <= 1e-2, worst


def test_c4_full_size_episode():
    import kvq
    from kvq.synth import C4, C4_GROUP, C4_KEEP, C4_STEPS, C4_WINDOW, c4_inputs
    s = C4
    qs, K, V = c4_inputs("cuda")
    cache = kvq.PackedKIVICache.from_context(K, V, window=C4_WINDOW, group_k=C4_GROUP, group_v=C4_GROUP)
    n_q = cache.n_q
    rep = s.Hq // s.Hkv
    scaling = s.d ** -0.5
    wgt = 1.0 / (rep * C4_STEPS)
    scores = torch.zeros((s.B, s.Hkv, n_q), dtype=torch.float32, device="cuda")
    for t in range(C4_STEPS):
        kvq.kivi_decode(qs[t], scaling, cache, scores=scores, score_weight=wgt)
    idx = kvq.topk_retain(scores, C4_KEEP)
    kept = kvq.retained_cache(cache, idx)
    out = kvq.kivi_decode(qs[0], scaling, kept).float().cpu().numpy()
    sc_gpu, idx_gpu = scores.cpu().numpy(), idx.cpu().numpy().astype(np.int64)
    q_all = qs.float().cpu().numpy()                                           # (steps, B, Hq, 1, d)
    for b, h in [(0, 0), (3, 7), (1, 4)]:
        Kb = K[b:b + 1, h:h + 1].float().cpu().numpy()
        Vb = V[b:b + 1, h:h + 1].float().cpu().numpy()
        kq, vq = ok.kivi_quant(Kb, 4, C4_GROUP, True, 0), ok.kivi_quant(Vb, 4, C4_GROUP, False, 0)
        kh = ok.kivi_dequant(kq["codes"], kq["lo"], kq["scale"], C4_GROUP, True)[:, :, :n_q]
        vh = ok.kivi_dequant(vq["codes"][:, :, :n_q], vq["lo"][:, :, :n_q], vq["scale"][:, :, :n_q], C4_GROUP, False)
        qb = q_all[:, b, h * rep:(h + 1) * rep, 0].transpose(1, 0, 2)[None]    # (1, rep, steps, d): every step
        sc = accumulate_decode_scores(np.zeros((1, 1, n_q)), decode_step_probs(qb, scaling, kh, Kb[:, :, n_q:]),
                                      wgt)[0, 0]
        sc_err = float(np.abs(sc_gpu[b, h] - sc).max() / sc.max())
        ref_idx = topk_retain(sc[None], C4_KEEP)[0]
        kth = float(np.sort(sc)[::-1][C4_KEEP - 1])
        diff = np.setxor1d(ref_idx, idx_gpu[b, h])
        gap = float(np.abs(sc[diff] - kth).max() / kth) if diff.size else 0.0
        keep = idx_gpu[b, h]
        tok = {"k": kh[:, :, keep], "v": vh[:, :, keep], "b": np.zeros((1, 1, keep.size)), "tau": np.full(keep.size, -1)}
        W = C4_WINDOW
        ref = chunked_attention(q_all[0, b:b + 1, h * rep:(h + 1) * rep], scaling, np.array([s.T]), Kb[:, :, n_q:],
                                Vb[:, :, n_q:], np.arange(W), np.full(W, 1 << 40), tok)
        out_err = float(np.abs(out[b, 0, h * rep:(h + 1) * rep] - ref[0, 0]).max())
        print(f"C4 full size (b={b}, h={h}): scores rel-err {sc_err:.2e}, retained-set differences {diff.size} "
              f"(largest gap to the k-th score {gap:.1e}), retained decode max-abs-err {out_err:.3e}", flush=True)
        assert sc_err <= 1e-4, sc_err
        assert gap <= 1e-4, gap
        assert out_err <= 1e-2, out_err


def test_c5_full_size_sampled_heads():
    import kvq
    from kvq.synth import C5, c5_inputs
    s = C5
    q, K, V = c5_inputs("cuda")
    cache = kvq.DctCache.from_context(K, V, window=0)
    out = kvq.dct_decode(q, s.d ** -0.5, cache).float().cpu().numpy()
    rep = s.Hq // s.Hkv
    worst = 0.0
    for h in (0, 7, 3):
        Kh = K[:, h].float().cpu().numpy()
        Vh = V[:, h].float().cpu().numpy()
        kc, ks, _ = dct_encode(Kh)
        vc, vs, _ = dct_encode(Vh)
        ref = dct_decode(q[:, h * rep:(h + 1) * rep].float().cpu().numpy(), s.d ** -0.5, kc, ks, vc, vs)
        err = float(np.abs(out[0, 0, h * rep:(h + 1) * rep] - ref[0, 0]).max())
        print(f"C5 full size (h={h}): max-abs-err {err:.3e}", flush=True)
        worst = max(worst, err)
    assert worst <= 1e-2, worst
