"""snapkv_scores on the GPU (kvq.snapkv_scores, libkvq kvq_snapkv_scores) against the float64 oracle
(oracle.evict.snapkv_scores, a restatement of STRATA_KV.py:932-954 pinned by a per-query loop).

Scores of the non-window keys within rtol 1e-4 (the logits are exact products accumulated in fp32;
fp32 inputs go through fp16 hi/lo parts, ~2^-22), the window columns equal to the largest score + 1
(the same fp32 rounding as the reference's float(max) + 1).  Shapes: GQA 1/4/8, windows 16/64,
pooling kernels 1/5/7, fp32/bf16/fp16, more rows than one workgroup holds (several row groups),
batch > 1, and the QRows form of the queries.  The top-k of the scores (SnapKVMethod / MTLP
selection, 969-981, 1010-1023) equals the oracle's except at near-ties of the k-th score.
"""
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from oracle.evict import snapkv_scores as oracle_snapkv, topk_retain

pytestmark = pytest.mark.gpu


def _case(B, Hq, Hkv, H, d, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    k = torch.randn((B, Hkv, H + 3, d), generator=g)
    k[:, :, ::97] += 2.0                                               # a few heavy hitters
    q = torch.randn((B, Hq, H + 3, d), generator=g)
    return q.to(dtype), k.to(dtype)


@pytest.mark.parametrize("B,Hq,Hkv,H,w,kern,dtype", [
    (1, 8, 2, 700, 64, 5, torch.float32),
    (1, 8, 2, 700, 64, 5, torch.bfloat16),
    (2, 32, 8, 2000, 64, 5, torch.bfloat16),        # rep 4: 256 rows, one row group
    (1, 16, 2, 1500, 64, 7, torch.bfloat16),        # rep 8: 512 rows, two row groups
    (1, 8, 2, 1200, 64, 1, torch.float32),          # fp32: 256 rows, two row groups of 128
    (2, 4, 4, 333, 16, 5, torch.float16),
])
def test_snapkv_scores_match_oracle(B, Hq, Hkv, H, w, kern, dtype):
    import kvq
    d = 128
    q, k = _case(B, Hq, Hkv, H, d, dtype, seed=H + Hq)
    cfg = SimpleNamespace(SNAPKV_WINDOW=w, SNAPKV_KERNEL=kern)
    got = kvq.snapkv_scores(q.cuda(), k.cuda(), H, d ** -0.5, cfg).cpu().numpy()
    want = oracle_snapkv(q.float().numpy(), k.float().numpy(), H, d ** -0.5, w, kern)
    assert got.shape == (B, Hkv, H)
    np.testing.assert_allclose(got[..., :H - w], want[..., :H - w], rtol=1e-4, atol=1e-7 * want[..., :H - w].max())
    assert np.all(got[..., H - w:] == np.float32(got[..., :H - w].max() + 1.0))
    np.testing.assert_allclose(got[..., H - w:], want[..., H - w:], rtol=1e-6)


@pytest.mark.parametrize("qs,ks", [(2.0 ** -17, 2.0 ** 17), (2.0 ** 20, 2.0 ** -20), (2.0 ** -122, 1.0)])
def test_snapkv_scores_fp32_extreme_magnitudes(qs, ks):
    """fp32 keys past fp16's range (~5e5) or far below it (~4e-6), queries scaled the other way so
    the logits keep their size: the rows are brought into the fp16 parts' range by a power of two
    per tensor and the logits scaled back, so the scores match the oracle as for ordinary rows.
    Queries near fp32's smallest normal (~2^-120): the power stays finite (at most 2^63) and the
    scores are those of uniform attention, as the oracle's, not NaN."""
    import kvq
    B, Hq, Hkv, H, w, kern, d = 1, 8, 2, 700, 64, 5, 128
    q, k = _case(B, Hq, Hkv, H, d, torch.float32, seed=77)
    q, k = q * qs, k * ks
    print(f"snapkv fp32 magnitudes: |k| max {float(k.abs().max()):.3e}", flush=True)
    cfg = SimpleNamespace(SNAPKV_WINDOW=w, SNAPKV_KERNEL=kern)
    got = kvq.snapkv_scores(q.cuda(), k.cuda(), H, d ** -0.5, cfg).cpu().numpy()
    want = oracle_snapkv(q.double().numpy(), k.double().numpy(), H, d ** -0.5, w, kern)
    assert np.isfinite(got).all()
    np.testing.assert_allclose(got[..., :H - w], want[..., :H - w], rtol=1e-4, atol=1e-7 * want[..., :H - w].max())


def test_snapkv_qrows_and_topk_selection():
    """Queries as the reference's QRows (only the kept positions), then the top-k of the scores as
    SnapKVMethod keeps them; against the oracle's sets modulo ties within 1e-4 of the k-th score."""
    import kvq
    B, Hq, Hkv, H, d, keep = 1, 32, 8, 4096, 128, 512
    q, k = _case(B, Hq, Hkv, H, d, torch.bfloat16, seed=4096)
    pos = torch.arange(H - 64, H)

    class Rows:                                                   # QRows: rows at absolute positions
        def __init__(self, rows, positions):
            self.rows, self.positions = rows, positions

        def at(self, p):
            idx = torch.searchsorted(self.positions, p)
            return self.rows[:, :, idx.to(self.rows.device)]

    qr = Rows(q[:, :, H - 64:H].cuda(), pos)
    sc = kvq.snapkv_scores(qr, k.cuda(), H, d ** -0.5)
    idx = kvq.topk_retain(sc, keep).cpu().numpy()
    want_sc = oracle_snapkv(q.float().numpy(), k.float().numpy(), H, d ** -0.5, 64, 5)
    ref = topk_retain(want_sc, keep)
    for h in range(Hkv):
        kth = np.sort(want_sc[0, h])[-keep]
        near = set(np.nonzero(np.abs(want_sc[0, h] - kth) <= 1e-4 * kth)[0].tolist())
        diff = set(idx[0, h].tolist()) ^ set(ref[0, h].tolist())
        assert diff <= near, (h, sorted(diff - near)[:10])
    assert set(range(H - 64, H)) <= set(idx[0, 0].tolist())          # the window is always kept


def test_snapkv_scores_reference_fixture():
    """kvq.snapkv_scores against the reference's own snapkv_scores (tests/golden/kivi_attention.npz:
    q (1, 8, 300, 128), k (1, 2, 300, 128) rebuilt from tests/golden/layer_inputs.py, its default
    window 64 and kernel 5); fp32 input, bar 1e-5 of the scores' scale."""
    import sys
    from pathlib import Path
    import kvq
    gold = Path(__file__).resolve().parent / "golden"
    if str(gold) not in sys.path:
        sys.path.insert(0, str(gold))
    from layer_inputs import kivi_inputs
    g = np.load(gold / "kivi_attention.npz")
    x = kivi_inputs()
    w, kern = (int(v) for v in g["snap_params"])
    cfg = type("Cfg", (), {"SNAPKV_WINDOW": w, "SNAPKV_KERNEL": kern})()
    got = kvq.snapkv_scores(torch.from_numpy(x["qs"]).cuda(), torch.from_numpy(x["ks"]).cuda(), 300, 128 ** -0.5,
                            cfg).cpu().numpy()
    err = float(np.abs(got - g["snap"]).max() / np.abs(g["snap"]).max())
    print(f"device snapkv_scores vs the reference's: {err:.2e}", flush=True)
    assert err < 1e-5, err
