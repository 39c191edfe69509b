"""Eviction families that keep exact rows, and chunk-local selection, on the GPU against the oracle.

* kvq.gather_rows: bit-exact row copies (bf16, fp32), zero rows for out-of-range indices, and the
  ``out=`` form writing into a larger buffer;
* kvq.finalize_chunk (STRATA_KV.py:573-592): the within-chunk share within 1e-5 of the float64
  oracle, kept positions equal to the oracle's top-k except where both candidates tie with the
  oracle's m-th share within 1e-6, stored rows bit-equal to the oracle's absmax fake quantisation
  of the same rows at 8 and 4 bits (16: the rows themselves);
* EvictedState from snapkv_keep (SnapKVMethod, 955-981) and from streaming_keep
  (StreamingLLMMethod, 1036-1060), driven through DecodeCtl for two decode steps: outputs against
  chunked_attention over ALL context rows with the reference's per-KV-head hide mask (the gather
  of the kept rows is checked against the mask formulation, not against itself);
* MTLPState from mtlp_select (SnapKVQuantMethod, 984-1033): the kept rows KIVI-coded as one
  sequence, the window exact; outputs against chunked_attention over kivi_quant's entries of the
  same rows plus the window and appended rows.
Bars: 2e-3 (fp32), 1e-2 (bf16).
"""
from types import SimpleNamespace

import numpy as np
import pytest
import torch

import oracle.kivi as ok
from oracle.attention import chunked_attention
from oracle.evict import BIG, absmax_fake_quant, chunk_share, keep_hide, snapkv_scores, streaming_hide, topk_retain

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_gather_rows_bit_exact(dtype):
    import kvq
    g = torch.Generator().manual_seed(4)
    B, H, T, d, m = 2, 3, 300, 128, 77
    K = torch.randn((B, H, T, d), generator=g).to(dtype)
    V = torch.randn((B, H, T, d), generator=g).to(dtype)
    idx = torch.randint(0, T, (B, H, m), generator=g, dtype=torch.int32)
    idx[0, 1, 5] = T                                     # out of range: a zero row
    idx[1, 2, 0] = -3
    ko, vo = kvq.gather_rows(K.cuda(), V.cuda(), idx.cuda())
    ii = idx.clamp(0, T - 1).long()
    want_k = torch.gather(K, 2, ii[..., None].expand(B, H, m, d))
    want_v = torch.gather(V, 2, ii[..., None].expand(B, H, m, d))
    want_k[0, 1, 5] = 0
    want_v[0, 1, 5] = 0
    want_k[1, 2, 0] = 0
    want_v[1, 2, 0] = 0
    assert torch.equal(ko.cpu(), want_k) and torch.equal(vo.cpu(), want_v)
    big_k = torch.full((B, H, m + 9, d), 7.0, dtype=dtype, device="cuda")
    kvq.gather_rows(K.cuda(), None, idx.cuda(), out=(big_k, None))
    assert torch.equal(big_k[:, :, :m].cpu(), want_k) and bool((big_k[:, :, m:] == 7.0).all())


@pytest.mark.parametrize("keep_bits", [8, 4, 16])
def test_finalize_chunk_against_oracle(keep_bits):
    import kvq
    g = torch.Generator().manual_seed(keep_bits)
    B, H, rep, W_OBS, C, d, m = 2, 4, 4, 32, 128, 128, 40
    k = torch.randn((B, H, C, d), generator=g) * 1.3
    v = torch.randn((B, H, C, d), generator=g)
    qref = torch.randn((B, H, rep * W_OBS, d), generator=g) * (d ** -0.5) * 2.0
    out = kvq.finalize_chunk(k.cuda(), v.cuda(), qref.cuda(), SimpleNamespace(family="snapkv"), {"tokens": m},
                             keep_bits)
    share = kvq.chunk_share(qref.cuda(), k.cuda()).cpu().numpy()
    ref_share = chunk_share(qref.numpy(), k.numpy())
    assert float(np.abs(share - ref_share).max() / ref_share.max()) <= 1e-5
    idx = out["idx"].cpu().numpy()
    ref_idx = topk_retain(ref_share, m)
    for b in range(B):
        for h in range(H):
            diff = np.setxor1d(idx[b, h], ref_idx[b, h])
            kth = np.sort(ref_share[b, h])[::-1][m - 1]
            assert diff.size == 0 or float(np.abs(ref_share[b, h, diff] - kth).max() / kth) <= 1e-6
    gk = np.take_along_axis(k.numpy(), idx[..., None].repeat(d, -1), 2)
    gv = np.take_along_axis(v.numpy(), idx[..., None].repeat(d, -1), 2)
    np.testing.assert_array_equal(out["k"].cpu().numpy(), absmax_fake_quant(gk, keep_bits))
    np.testing.assert_array_equal(out["v"].cpu().numpy(), absmax_fake_quant(gv, keep_bits))
    assert out["b"].shape == (B, H, m) and not bool(out["b"].any())
    with pytest.raises(NotImplementedError):
        kvq.finalize_chunk(k.cuda(), v.cuda(), qref.cuda(), "am", {"tokens": m}, keep_bits)


def _drive(st, K, V, Q, H, steps, d):
    """Two decode steps through DecodeCtl; returns the outputs (float32 numpy)."""
    import kvq
    ctl = kvq.DecodeCtl({0: st})
    module = SimpleNamespace(layer_idx=0, scaling=d ** -0.5)
    outs, pos = [], H
    with kvq.routed(ctl):
        for t in steps:
            qpos = torch.arange(pos, pos + t)
            ctl.begin(qpos)
            out, _ = kvq.router_attention(module, Q[:, :, pos - H:pos - H + t].cuda(), K[:, :, pos:pos + t].cuda(),
                                          V[:, :, pos:pos + t].cuda(), None)
            outs.append(out.float().cpu().numpy())
            pos += t
    return outs


def _oracle_hidden(q, K_all, V_all, hide_ctx, H, qpos, scaling, tok=None):
    """chunked_attention over every row: context rows with their hide (per KV head), appended rows
    visible from their positions on."""
    B, Hkv, n_all, d = K_all.shape
    hide = np.concatenate([hide_ctx, np.full((B, Hkv, n_all - H), BIG)], 2)
    return chunked_attention(q, scaling, np.asarray(qpos), K_all, V_all, np.arange(n_all), hide, tok)


@pytest.mark.parametrize("family", ["snapkv", "streaming"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_evicted_state_against_hide_mask(family, dtype):
    import kvq
    g = torch.Generator().manual_seed(31)
    B, Hq, Hkv, H, d, keep = 2, 8, 2, 640, 128, 200
    steps = [1, 2]
    T_all = H + sum(steps)
    K = (torch.randn((B, Hkv, T_all, d), generator=g) * 1.2).to(dtype)
    V = torch.randn((B, Hkv, T_all, d), generator=g).to(dtype)
    Qctx = torch.randn((B, Hq, H, d), generator=g).to(dtype)          # the prefill's queries (SnapKV window)
    Q = torch.randn((B, Hq, sum(steps), d), generator=g).to(dtype)
    scaling = d ** -0.5
    if family == "snapkv":
        kept = kvq.snapkv_keep(Qctx.cuda(), K[:, :, :H].cuda(), H, scaling, keep)
        sc = snapkv_scores(Qctx.float().numpy(), K[:, :, :H].float().numpy(), H, scaling, 64, 5)
        ref_keep = topk_retain(sc, keep)
        got = kept.cpu().numpy()
        for b in range(B):
            for h in range(Hkv):
                diff = np.setxor1d(got[b, h], ref_keep[b, h])
                kth = np.sort(sc[b, h])[::-1][keep - 1]
                assert diff.size == 0 or float(np.abs(sc[b, h, diff] - kth).max() / kth) <= 1e-4
        hide = keep_hide(got, H)
    else:
        kept = kvq.streaming_keep(B, Hkv, H, keep)
        hide = np.broadcast_to(streaming_hide(H, keep), (B, Hkv, H))
        assert (kept.cpu().numpy()[0, 0] == np.nonzero(streaming_hide(H, keep) == BIG)[0]).all()
    st = kvq.EvictedState(K[:, :, :H].cuda(), V[:, :, :H].cuda(), kept, extra=4)
    assert st.context_bytes() == 2 * B * Hkv * kept.shape[2] * d * K.element_size()
    outs = _drive(st, K, V, Q, H, steps, d)
    kn, vn = K.float().numpy(), V.float().numpy()
    tol = 2e-3 if dtype == torch.float32 else 1e-2
    pos = H
    for t, out in zip(steps, outs):
        ref = _oracle_hidden(Q[:, :, pos - H:pos - H + t].float().numpy(), kn[:, :, :pos + t], vn[:, :, :pos + t],
                             hide, H, np.arange(pos, pos + t), scaling)
        err = float(np.abs(out - ref).max())
        print(f"{family} {dtype} step of {t}: max-abs-err {err:.3e}", flush=True)
        assert err <= tol, err
        pos += t
    assert st.check_kernel()["kernel"]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_mtlp_state_against_oracle(dtype):
    import kvq
    g = torch.Generator().manual_seed(47)
    B, Hq, Hkv, H, d, group, window = 2, 8, 2, 1000, 128, 32, 64
    steps = [1, 2]
    T_all = H + sum(steps)
    K = (torch.randn((B, Hkv, T_all, d), generator=g) * 1.2 + 0.2).to(dtype)
    V = torch.randn((B, Hkv, T_all, d), generator=g).to(dtype)
    Qctx = torch.randn((B, Hq, H, d), generator=g).to(dtype)
    Q = torch.randn((B, Hq, sum(steps), d), generator=g).to(dtype)
    scaling = d ** -0.5
    n_q = kvq.mtlp_budget(0.25, H, d, 4, group, window)
    assert n_q == int((0.25 * H * 2 * d * 16 - window * 2 * d * 16) // (2 * d * (4 + 32 / group)))
    idx = kvq.mtlp_select(Qctx.cuda(), K[:, :, :H].cuda(), H, scaling, n_q)
    assert idx.shape == (B, Hkv, n_q) and bool((idx[..., 1:] > idx[..., :-1]).all())
    st = kvq.MTLPState(K[:, :, :H].cuda(), V[:, :, :H].cuda(), idx, window=window, group=group, extra=4)
    outs = _drive(st, K, V, Q, H, steps, d)
    kn, vn = K.float().numpy(), V.float().numpy()
    ii = idx.cpu().numpy()
    gk = np.take_along_axis(kn[:, :, :H], ii[..., None].repeat(d, -1), 2)
    gv = np.take_along_axis(vn[:, :, :H], ii[..., None].repeat(d, -1), 2)
    kq, vq = ok.kivi_quant(gk, 4, group, True, 0), ok.kivi_quant(gv, 4, group, False, 0)
    tok = {"k": kq["xhat"], "v": vq["xhat"], "b": np.zeros((B, Hkv, n_q)), "tau": np.full(n_q, -1)}
    hide = np.full((B, Hkv, H), H)
    hide[:, :, H - window:] = BIG                                   # the window stays exact
    tol = 2e-3 if dtype == torch.float32 else 1e-2
    pos = H
    for t, out in zip(steps, outs):
        ref = _oracle_hidden(Q[:, :, pos - H:pos - H + t].float().numpy(), kn[:, :, :pos + t], vn[:, :, :pos + t],
                             hide, H, np.arange(pos, pos + t), scaling, tok)
        err = float(np.abs(out - ref).max())
        print(f"MTLP {dtype} n_q {n_q} step of {t}: max-abs-err {err:.3e}", flush=True)
        assert err <= tol, err
        pos += t
    assert st.check_kernel()["kernel"]
