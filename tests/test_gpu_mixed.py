"""Mixed-width KIVI cache on the GPU against the CPU oracle (oracle/mixed.py).

* kvq_mixed_encode: every block's planar key rows, key (scale, zero), value tiles and slot-ordered
  value (scale, zero), read back through the documented layout, equal kivi_quant's at the block's
  width bit for bit (fp32 and bf16 inputs);
* kvq_mixed_decode: attention over all blocks plus exact rows within 2e-3 (fp32) / 1e-2 (bf16) of
  the oracle for every GQA row count, single-width caches of each width and the C3 width rule.
"""
import numpy as np
import pytest
import torch

import oracle.mixed as om
from layouts import slot_token, tile_codes
from oracle.strata import unpack_planar

pytestmark = pytest.mark.gpu


def _read_block(seg: np.ndarray, bits: int):
    """Bytes of one block -> (kc (64,128), k_sc (2,128), k_lo (2,128), vc (64,128), v_sc (64,4), v_lo (64,4))."""
    kc = unpack_planar(seg[:1024 * bits].reshape(64, 16 * bits), bits)
    km = seg[2048 * bits:2048 * bits + 1024].view(np.float16).astype(np.float32)
    vc = np.concatenate([tile_codes(seg[1024 * bits + 512 * bits * c:1024 * bits + 512 * bits * (c + 1)], bits)
                         for c in range(2)], 0)
    vm = seg[2048 * bits + 1024:2048 * bits + 2048].view(np.uint32).reshape(2, 4, 4, 8)   # chunk, group, g, slot
    v_sc = np.zeros((64, 4), np.float32)
    v_lo = np.zeros((64, 4), np.float32)
    for c in range(2):
        for gv in range(4):
            for g in range(4):
                for j in range(8):
                    t = 32 * c + slot_token(g, j)
                    word = int(vm[c, gv, g, j])
                    v_sc[t, gv] = np.array([word & 0xFFFF], np.uint16).view(np.float16)[0]
                    v_lo[t, gv] = np.array([word >> 16], np.uint16).view(np.float16)[0]
    return kc, km[:256].reshape(2, 128), km[256:].reshape(2, 128), vc, v_sc, v_lo


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_encode_bit_exact(dtype):
    import kvq
    g = torch.Generator().manual_seed(21)
    B, H, nb = 2, 2, 5
    K = (torch.randn((B, H, nb * 64 + 7, 128), generator=g) * 2 + 0.5).to(dtype)
    V = torch.randn((B, H, nb * 64 + 7, 128), generator=g).to(dtype)
    K[0, 0, 64:96, 3] = 1.25                                                # a constant key group
    widths = torch.tensor([2, 4, 8])[torch.randint(0, 3, (B, H, nb), generator=g)]
    cache = kvq.MixedKIVICache.from_context(K.cuda(), V.cuda(), widths, window=7)
    assert cache.nb == nb and cache.n_exact == 7
    ref = om.mixed_quant(K[:, :, :nb * 64].float().numpy(), V[:, :, :nb * 64].float().numpy(), widths.numpy())
    buf = cache.buf.cpu().numpy()
    bits_t, off, base = cache.blk_bits.cpu().numpy(), cache.blk_off.cpu().numpy(), cache.bh_base.cpu().numpy()
    for b in range(B):
        for h in range(H):
            for i in range(nb):
                bits = int(bits_t[b, h, i])
                assert bits == int(widths[b, h, i])
                s0 = (int(base[b * H + h]) + int(off[b, h, i])) * 2048
                kc, k_sc, k_lo, vc, v_sc, v_lo = _read_block(buf[s0:s0 + (bits + 1) * 2048], bits)
                np.testing.assert_array_equal(kc, ref["kc"][b, h, i])
                np.testing.assert_array_equal(k_sc, ref["k_sc"][b, h, i])
                np.testing.assert_array_equal(k_lo, ref["k_lo"][b, h, i])
                np.testing.assert_array_equal(vc, ref["vc"][b, h, i])
                np.testing.assert_array_equal(v_sc, ref["v_sc"][b, h, i])
                np.testing.assert_array_equal(v_lo, ref["v_lo"][b, h, i])


def _oracle(cache, K, V, widths, q, scaling):
    nc = cache.nb * 64
    m = om.mixed_quant(K[:, :, :nc].float().numpy(), V[:, :, :nc].float().numpy(), widths.numpy())
    ne = cache.n_exact
    return om.mixed_decode(q.float().numpy(), scaling, m["xk"], m["xv"],
                           K[:, :, nc:nc + ne].float().numpy(), V[:, :, nc:nc + ne].float().numpy())


@pytest.mark.parametrize("dtype,Hq,Hkv,Tq,T,W,mode", [
    (torch.float32, 4, 4, 1, 1000, 40, "random"),     # R = 1
    (torch.float32, 8, 4, 1, 640, 64, "random"),      # R = 2
    (torch.bfloat16, 8, 2, 1, 2048, 0, "c3"),         # R = 4, coded only, the C3 width rule
    (torch.float32, 8, 2, 2, 777, 9, "random"),       # R = 8
    (torch.float32, 8, 2, 1, 1024, 0, "2"),
    (torch.float32, 8, 2, 1, 1024, 0, "4"),
    (torch.float32, 8, 2, 1, 1024, 0, "8"),
    (torch.bfloat16, 32, 8, 1, 1536, 128, "c3"),      # C3 head shape
])
def test_decode_matches_oracle(dtype, Hq, Hkv, Tq, T, W, mode):
    import kvq
    g = torch.Generator().manual_seed(T + Hq + Tq)
    B, d = 2, 128
    K = (torch.randn((B, Hkv, T, d), generator=g) * 1.5 + 0.3).to(dtype)
    V = torch.randn((B, Hkv, T, d), generator=g).to(dtype)
    q = torch.randn((B, Hq, Tq, d), generator=g).to(dtype)
    nb = (T - W) // 64
    if mode == "random":
        widths = torch.tensor([2, 4, 8])[torch.randint(0, 3, (B, Hkv, nb), generator=g)]
    elif mode == "c3":
        widths = kvq.c3_widths(torch.exp(torch.randn((B, Hkv, nb), generator=g)))
    else:
        widths = torch.full((B, Hkv, nb), int(mode))
    cache = kvq.MixedKIVICache.from_context(K.cuda(), V.cuda(), widths, window=W)
    out = kvq.mixed_decode(q.cuda(), d ** -0.5, cache).float().cpu().numpy()
    ref = _oracle(cache, K, V, widths.to(torch.int64), q, d ** -0.5)
    err = float(np.abs(out - ref).max())
    tol = 2e-3 if dtype == torch.float32 else 1e-2
    assert err <= tol, err


def test_decode_peaked_logits():
    """One dominant block (large logits): the lazy-maximum rescale across width segments."""
    import kvq
    g = torch.Generator().manual_seed(8)
    B, Hq, Hkv, T, d = 1, 8, 2, 4096, 128
    K = torch.randn((B, Hkv, T, d), generator=g) * 0.3
    K[:, :, 1000:1064] += 3.0
    V = torch.randn((B, Hkv, T, d), generator=g)
    q = torch.ones((B, Hq, 1, d)) * 0.5
    nb = T // 64
    widths = torch.tensor([2, 4, 8])[torch.randint(0, 3, (B, Hkv, nb), generator=g)]
    cache = kvq.MixedKIVICache.from_context(K.cuda(), V.cuda(), widths, window=0)
    out = kvq.mixed_decode(q.cuda(), d ** -0.5, cache).cpu().numpy()
    ref = _oracle(cache, K, V, widths, q, d ** -0.5)
    assert float(np.abs(out - ref).max()) <= 2e-3


def test_phases_split_then_merge_equals_full():
    import kvq
    g = torch.Generator().manual_seed(77)
    B, Hq, Hkv, T, d = 1, 8, 2, 700, 128
    K = torch.randn((B, Hkv, T, d), generator=g).to(torch.bfloat16)
    V = torch.randn((B, Hkv, T, d), generator=g).to(torch.bfloat16)
    q = torch.randn((B, Hq, 1, d), generator=g).to(torch.bfloat16)
    nb = (T - 20) // 64
    widths = torch.tensor([2, 4, 8])[torch.randint(0, 3, (B, Hkv, nb), generator=g)]
    qc = q.cuda()
    for make, dec in ((lambda: kvq.MixedKIVICache.from_context(K.cuda(), V.cuda(), widths, window=20), kvq.mixed_decode),
                      (lambda: kvq.DctCache.from_context(K.cuda(), V.cuda(), window=20), kvq.dct_decode)):
        cache = make()
        full = dec(qc, d ** -0.5, cache)
        ws = torch.empty((1 << 20,), dtype=torch.float32, device="cuda")
        out = torch.empty_like(full)
        dec(qc, d ** -0.5, cache, workspace=ws, out=out, phases=1)
        dec(qc, d ** -0.5, cache, workspace=ws, out=out, phases=2)
        assert torch.equal(out, full)


def test_decode_many_query_tokens():
    """Tq 6 at rep 4: query-token pieces of 2 tokens (one launch each) against the oracle."""
    import kvq
    g = torch.Generator().manual_seed(66)
    B, Hq, Hkv, Tq, T, W, d = 1, 8, 2, 6, 1100, 76, 128
    K = (torch.randn((B, Hkv, T, d), generator=g) * 1.5 + 0.3)
    V = torch.randn((B, Hkv, T, d), generator=g)
    q = torch.randn((B, Hq, Tq, d), generator=g)
    nb = (T - W) // 64
    widths = torch.tensor([2, 4, 8])[torch.randint(0, 3, (B, Hkv, nb), generator=g)]
    cache = kvq.MixedKIVICache.from_context(K.cuda(), V.cuda(), widths, window=W)
    out = kvq.mixed_decode(q.cuda(), d ** -0.5, cache).float().cpu().numpy()
    ref = _oracle(cache, K, V, widths.to(torch.int64), q, d ** -0.5)
    assert float(np.abs(out - ref).max()) <= 2e-3


def test_decode_c3_class_plan_every_pair():
    """The plan the c3 workload times, at a shorter context: B 8 x Hkv 8 = 64 (b, h) with 64 blocks
    each takes the class-major plan (3 dispatch classes x 4 splits = 12 splits per (b, h), one full
    round of 768 blocks, splits sized by the class weights), asserted through the workspace size;
    every (b, h) against the oracle at the bf16 bar, and two runs bit-equal."""
    import kvq
    from kvq.synth import C3, c3_inputs
    s = C3
    T = 4096
    q, K, V, imp = c3_inputs("cpu", T=T)
    widths = kvq.c3_widths(imp)
    cache = kvq.MixedKIVICache.from_context(K.cuda(), V.cuda(), widths.cuda(), window=0)
    assert cache.nb == 64 and cache.n_exact == 0
    BH, R = s.B * s.Hkv, s.Hq // s.Hkv
    ws = kvq.mixed_workspace_floats(s.B, s.Hq, s.Hkv, 1, s.d, cache.nb, 0)
    assert ws == BH * 12 * R * (s.d + 2), ws                    # 12 class-weighted splits per (b, h)
    qc = q.cuda()
    got = kvq.mixed_decode(qc, s.d ** -0.5, cache)
    assert torch.equal(got, kvq.mixed_decode(qc, s.d ** -0.5, cache))
    out = got.float().cpu().numpy()
    ref = _oracle(cache, K, V, widths.to(torch.int64), q, s.d ** -0.5)
    err = float(np.abs(out - ref).max())
    print(f"C3 class plan (12 splits per (b, h)), every pair: max-abs-err {err:.3e}", flush=True)
    assert err <= 1e-2, err
