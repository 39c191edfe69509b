"""The headline configuration at full size on the GPU against the float64 oracle.

C2 (B 16, Hq 32, Hkv 8, d 128, T 32768 = 32640 packed + 128 exact bf16 rows, groups of 64) is
generated on the device exactly as the c2 bench workload generates it, packed by the library, and
decoded with the automatic plan the bench times (6 packed splits per (b, h) = one full round of
packed blocks, so class-major splits sized by dispatch class, and the exact window in exact-row
blocks of the same launch).  Sampled (b, h) pairs -- first, last and interior ones,
which land on different XCDs and split slots -- are compared with the oracle's kivi_quant +
chunked_attention of the same rows at the bf16 bar (1e-2 max-abs-err).  The same plan at a
shorter context (T 4096, also 6 splits per (b, h)) is checked on every (b, h), with a window that
is not a multiple of the exact-row block size.
"""
import numpy as np
import pytest
import torch

import oracle.kivi as ok
from oracle.attention import kivi_decode_reference

pytestmark = pytest.mark.gpu

PAIRS = [(0, 0), (0, 7), (5, 3), (9, 6), (12, 1), (15, 7)]


def _oracle_pair(q, K, V, b, h, rep, n_q, n_e, gk, gv):
    Kb = K[b:b + 1, h:h + 1, :n_q + n_e].float().cpu().numpy()
    Vb = V[b:b + 1, h:h + 1, :n_q + n_e].float().cpu().numpy()
    kq, vq = ok.kivi_quant(Kb, 4, gk, True, 0), ok.kivi_quant(Vb, 4, gv, False, 0)
    qb = q[b:b + 1, h * rep:(h + 1) * rep].float().cpu().numpy()
    return kivi_decode_reference(qb, 128 ** -0.5, Kb[:, :, n_q:], Vb[:, :, n_q:], kq["codes"], kq["lo"],
                                 kq["scale"], vq["codes"], vq["lo"], vq["scale"], gk, gv, n_q)[0, :, :]


def test_c2_full_size_sampled_pairs():
    import kvq
    from kvq.synth import C2, decode_inputs
    s = C2
    q, K, V = decode_inputs(s, device="cuda")
    cache = kvq.PackedKIVICache.from_context(K, V, window=s.window, group_k=s.group_k, group_v=s.group_v)
    rep = s.Hq // s.Hkv
    BH, R = s.B * s.Hkv, rep
    # the production plan (the automatic one kivi_decode uses): 6 packed splits per (b, h) and 2
    # exact-row blocks, their partials merged
    ws = kvq.workspace_floats(s.B, s.Hq, s.Hkv, 1, s.d, cache.n_q, cache.n_exact, s.group_k, s.group_v)
    S1 = (ws // BH - 2 * R) // (R * (s.d + 2))
    assert ws == BH * (S1 * R * (s.d + 2) + 2 * R) and S1 == 8
    print(f"C2 plan: {S1} splits per (b, h)", flush=True)
    out = kvq.kivi_decode(q, s.d ** -0.5, cache).float().cpu().numpy()       # (B, 1, Hq, d)
    assert np.isfinite(out).all()
    worst = 0.0
    for b, h in PAIRS:
        ref = _oracle_pair(q, K, V, b, h, rep, cache.n_q, cache.n_exact, s.group_k, s.group_v)   # (1, rep, d)
        err = float(np.abs(out[b, :, h * rep:(h + 1) * rep] - ref).max())
        print(f"C2 full size (b={b}, h={h}): max-abs-err {err:.3e}", flush=True)
        worst = max(worst, err)
    assert worst <= 1e-2, worst


def test_class_plan_every_pair_shorter_context():
    """B 16, Hkv 8 at T 4096 with a 100-row window: the planner again picks 6 packed splits per
    (b, h) (one full round: class-major, class-weighted splits) and puts the window in 2 exact-row
    blocks per (b, h) of 64 and 36 rows; every (b, h) against the oracle, and two runs bit-equal."""
    import kvq
    from kvq.synth import C2, decode_inputs
    s = C2
    T, W = 4096, 100
    q, K, V = decode_inputs(s, device="cuda", T=T)
    cache = kvq.PackedKIVICache.from_context(K, V, window=W, group_k=s.group_k, group_v=s.group_v)
    rep = s.Hq // s.Hkv
    BH, R = s.B * s.Hkv, rep
    ws = kvq.workspace_floats(s.B, s.Hq, s.Hkv, 1, s.d, cache.n_q, cache.n_exact, s.group_k, s.group_v)
    assert ws == BH * (8 * R * (s.d + 2) + 2 * R)
    got = kvq.kivi_decode(q, s.d ** -0.5, cache)
    again = kvq.kivi_decode(q, s.d ** -0.5, cache)
    assert torch.equal(got, again)
    out = got.float().cpu().numpy()
    worst = 0.0
    for b in range(s.B):
        for h in range(s.Hkv):
            ref = _oracle_pair(q, K, V, b, h, rep, cache.n_q, cache.n_exact, s.group_k, s.group_v)
            worst = max(worst, float(np.abs(out[b, :, h * rep:(h + 1) * rep] - ref).max()))
    print(f"class plan T={T}: max-abs-err over all (b, h) {worst:.3e}", flush=True)
    assert worst <= 1e-2, worst
