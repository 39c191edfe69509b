"""Blockwise DCT coder and decode on the GPU against the CPU oracle (oracle/dct.py).

* dct_encode: key and value layouts read back to (coefficient, channel) codes and fp16 scales
  equal the oracle's bit for bit (same fixed float32 arithmetic order), fp32 and bf16 inputs;
* dct_decode: attention over the reconstructed rows plus exact rows, within 2e-3 (fp32) /
  1e-2 (bf16) of the oracle's float64 result, for every GQA row count R = rep * Tq in 1..8,
  with and without exact rows, and over a coded-only context.
"""
import numpy as np
import pytest
import torch

import oracle.dct as od

pytestmark = pytest.mark.gpu

_NIB = [0, 4, 1, 5, 2, 6, 3, 7]


def _keys_to_oracle(codes: np.ndarray) -> np.ndarray:
    """(BH, nb, 1024) key layout -> (BH, nb, 16, 128) codes: row k = 16 words, word D holds channel
    8D + e of coefficient k at nibble _NIB[e]."""
    words = codes.view(np.uint32).reshape(codes.shape[0], codes.shape[1], 16, 16)      # k, D
    out = np.empty(words.shape[:3] + (128,), np.uint8)
    for e in range(8):
        out[..., e::8] = (words >> (4 * _NIB[e])) & 15
    return out


def _values_to_oracle(codes: np.ndarray, scales: np.ndarray):
    """(BH, nb, 1024) value tiles + (BH, nb, 128) [n][blk] scales -> (BH, nb, 16, 128), (BH, nb, 128)."""
    words = codes.view(np.uint32).reshape(codes.shape[0], codes.shape[1], 2, 16, 8)   # gp, n, blk
    out = np.empty((codes.shape[0], codes.shape[1], 16, 128), np.uint8)
    for gp in range(2):
        for e in range(8):
            nib = (words[:, :, gp] >> (4 * _NIB[e])) & 15                               # (BH, nb, n, blk)
            out[:, :, 8 * gp + e] = nib.transpose(0, 1, 3, 2).reshape(codes.shape[0], codes.shape[1], 128)
    sc = scales.reshape(scales.shape[0], scales.shape[1], 16, 8).transpose(0, 1, 3, 2).reshape(scales.shape)
    return out, sc


def test_dct_table_matches_oracle():
    import kvq
    np.testing.assert_array_equal(kvq.dct_table().cpu().numpy(), od.dct_table())


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_encode_bit_exact(dtype):
    import kvq
    g = torch.Generator().manual_seed(11)
    B, H, T = 2, 3, 320
    x = (torch.randn((B, H, T, 128), generator=g).cumsum(2) * 0.3 + 0.5).to(dtype)
    x[0, 0, :64, 5] = 0                                                 # an all-zero (block, channel)
    kc, ks = kvq.dct_encode(x.cuda())
    vc, vs = kvq.dct_encode(x.cuda(), for_values=True)
    c_o, s_o, _ = od.dct_encode(x.float().numpy().reshape(B * H, T, 128))
    nb = T // 64
    got_k = _keys_to_oracle(kc.cpu().numpy().reshape(B * H, nb, 1024))
    np.testing.assert_array_equal(got_k, c_o)
    np.testing.assert_array_equal(ks.float().cpu().numpy().reshape(B * H, nb, 128), s_o)
    got_v, got_vs = _values_to_oracle(vc.cpu().numpy().reshape(B * H, nb, 1024),
                                      vs.float().cpu().numpy().reshape(B * H, nb, 128))
    np.testing.assert_array_equal(got_v, c_o)
    np.testing.assert_array_equal(got_vs, s_o)
    assert s_o[0, 0, 5] == np.float32(2.0 ** -24) and (c_o[0, 0, :, 5] == 7).all()


def _oracle(cache, q, scaling):
    B = q.shape[0]
    nb = cache.T // 64
    BH = cache.kc.shape[0] * cache.kc.shape[1]
    kc = _keys_to_oracle(cache.kc.cpu().numpy().reshape(BH, nb, 1024))
    ks = cache.ks.float().cpu().numpy().reshape(BH, nb, 128)
    vc, vs = _values_to_oracle(cache.vc.cpu().numpy().reshape(BH, nb, 1024),
                               cache.vs.float().cpu().numpy().reshape(BH, nb, 128))
    ne = cache.n_exact
    ke = cache.k_exact[:, :, :ne].float().cpu().numpy()
    ve = cache.v_exact[:, :, :ne].float().cpu().numpy()
    return od.dct_decode(q.float().numpy(), scaling, kc, ks, vc, vs, ke, ve)


@pytest.mark.parametrize("dtype,Hq,Hkv,Tq,T,W", [
    (torch.float32, 4, 4, 1, 1000, 40),     # R = 1, coded tail spills into the exact rows
    (torch.float32, 8, 4, 1, 640, 64),      # R = 2
    (torch.float32, 8, 2, 1, 2048, 0),      # R = 4, coded only
    (torch.float32, 8, 2, 2, 777, 9),       # R = 8
    (torch.bfloat16, 8, 2, 1, 1500, 30),
    (torch.float32, 8, 1, 1, 130, 2),       # R = 8 over two blocks
])
def test_decode_matches_oracle(dtype, Hq, Hkv, Tq, T, W):
    import kvq
    g = torch.Generator().manual_seed(T + Hq)
    B, d = 2, 128
    K = (torch.randn((B, Hkv, T, d), generator=g).cumsum(2) * 0.2 + 0.4).to(dtype)
    V = torch.randn((B, Hkv, T, d), generator=g).to(dtype)
    q = torch.randn((B, Hq, Tq, d), generator=g).to(dtype)
    cache = kvq.DctCache.from_context(K.cuda(), V.cuda(), window=W)
    assert cache.T == (T - W) // 64 * 64 and cache.n_exact == T - cache.T
    out = kvq.dct_decode(q.cuda(), d ** -0.5, cache).float().cpu().numpy()
    ref = _oracle(cache, q, d ** -0.5)
    err = float(np.abs(out - ref).max())
    tol = 2e-3 if dtype == torch.float32 else 1e-2
    assert err <= tol, err


@pytest.mark.parametrize("T,W", [(4096, 0), (4096 + 64, 64), (8192 + 37, 37)])
def test_decode_c5_shape_bf16(T, W):
    """The C5 instantiation itself: bf16, Hq 64 over Hkv 8 (R = 8, the dct_pair_split<bf16> kernel
    the c5 workload times: blocks two at a time) on the C5 generator's AR(1) + noise rows at a
    reduced context, with and without an exact tail.  bf16 bar (1e-2) against the float64 oracle."""
    import kvq
    from kvq.synth import C5, c5_inputs
    q, K, V = c5_inputs("cpu", T=T)
    assert q.dtype == torch.bfloat16 and q.shape[1] == 64 and K.shape[1] == 8
    cache = kvq.DctCache.from_context(K.cuda(), V.cuda(), window=W)
    assert cache.T == (T - W) // 64 * 64
    scaling = C5.d ** -0.5
    out = kvq.dct_decode(q.cuda(), scaling, cache).float().cpu().numpy()
    ref = _oracle(cache, q, scaling)
    err = float(np.abs(out - ref).max())
    print(f"C5-shaped bf16 T={T} W={W}: max-abs-err {err:.3e}")
    assert err <= 1e-2, err


def test_decode_r8_bf16_gqa8():
    """bf16 at R = 8 with GQA 8 over two KV heads and batch 2 (a second bh layout of the same kernel).
    Values are unit-scale: the 1e-2 bar is absolute, and bf16 rounding of outputs near 16 alone is
    ~0.03 (a random-walk V of this length gave exactly that error, equal to bf16(ref) - ref)."""
    import kvq
    g = torch.Generator().manual_seed(808)
    B, Hq, Hkv, T, W, d = 2, 16, 2, 3000, 56, 128
    K = (torch.randn((B, Hkv, T, d), generator=g).cumsum(2) * 0.1).to(torch.bfloat16)
    V = torch.randn((B, Hkv, T, d), generator=g).to(torch.bfloat16)
    q = torch.randn((B, Hq, 1, d), generator=g).to(torch.bfloat16)
    cache = kvq.DctCache.from_context(K.cuda(), V.cuda(), window=W)
    out = kvq.dct_decode(q.cuda(), d ** -0.5, cache).float().cpu().numpy()
    ref = _oracle(cache, q, d ** -0.5)
    assert float(np.abs(out - ref).max()) <= 1e-2


@pytest.mark.parametrize("dtype,B,Hq,Hkv,Tq,T,W,seed", [
    (torch.float16, 2, 16, 2, 1, 64 * 33 + 50, 50, 1),     # fp16, odd block count: a final single block
    (torch.bfloat16, 1, 4, 2, 3, 64 + 10, 10, 2),          # rep 2 x Tq 3 = 6 rows padded to 8, one block
    (torch.bfloat16, 1, 8, 2, 2, 640, 0, 3),               # rep 4 x Tq 2 = 8 rows, coded only
    (torch.bfloat16, 1, 64, 8, 1, 64 * 259, 0, 4),         # C5 heads, odd block count, many splits
])
def test_decode_r8_pairs(dtype, B, Hq, Hkv, Tq, T, W, seed):
    """The 16-bit R = 8 kernel (dct_pair_split: blocks two at a time) against the float64 oracle:
    fp16 and bf16, 6 or 8 rows, a single block, odd block counts (the last pair's slot B masked)."""
    import kvq
    g = torch.Generator().manual_seed(seed)
    d = 128
    K = (torch.randn((B, Hkv, T, d), generator=g).cumsum(2) * 0.15).to(dtype)
    V = torch.randn((B, Hkv, T, d), generator=g).to(dtype)
    q = torch.randn((B, Hq, Tq, d), generator=g).to(dtype)
    cache = kvq.DctCache.from_context(K.cuda(), V.cuda(), window=W)
    out = kvq.dct_decode(q.cuda(), d ** -0.5, cache).float().cpu().numpy()
    ref = _oracle(cache, q, d ** -0.5)
    err = float(np.abs(out - ref).max())
    print(f"pairs {dtype} B={B} Hq={Hq} Hkv={Hkv} Tq={Tq} T={T}: max-abs-err {err:.3e}")
    assert err <= 1e-2, err


def test_decode_r8_pairs_peaked_logits():
    """bf16 R = 8 with one dominant block late in the context: the lazy maximum rescales the value
    accumulators of both slots through the alpha hand-off."""
    import kvq
    g = torch.Generator().manual_seed(5)
    B, Hq, Hkv, T, d = 1, 16, 2, 64 * 40, 128
    K = torch.randn((B, Hkv, T, d), generator=g) * 0.3
    K[:, :, 1920:1984] += 3.0
    K[:, :, 640:704] += 1.5
    V = torch.randn((B, Hkv, T, d), generator=g)
    q = (torch.ones((B, Hq, 1, d)) * 0.5).to(torch.bfloat16)
    K, V = K.to(torch.bfloat16), V.to(torch.bfloat16)
    cache = kvq.DctCache.from_context(K.cuda(), V.cuda(), window=0)
    out = kvq.dct_decode(q.cuda(), d ** -0.5, cache).float().cpu().numpy()
    ref = _oracle(cache, q, d ** -0.5)
    assert float(np.abs(out - ref).max()) <= 1e-2


def test_decode_peaked_logits():
    """Large logits (one block dominates): the online maximum and lazy rescale path."""
    import kvq
    g = torch.Generator().manual_seed(3)
    B, Hq, Hkv, T, d = 1, 8, 2, 4096, 128
    K = torch.randn((B, Hkv, T, d), generator=g) * 0.3
    K[:, :, 2000:2064] += 4.0
    V = torch.randn((B, Hkv, T, d), generator=g)
    q = torch.ones((B, Hq, 1, d)) * 0.5
    cache = kvq.DctCache.from_context(K.cuda(), V.cuda(), window=0)
    out = kvq.dct_decode(q.cuda(), d ** -0.5, cache).cpu().numpy()
    ref = _oracle(cache, q, d ** -0.5)
    assert float(np.abs(out - ref).max()) <= 2e-3


def test_decode_many_query_tokens():
    """Tq 7 at rep 4, in pieces of 2 query tokens and with an explicit chunk of 3 (pieces of 2):
    against the oracle over all seven queries."""
    import kvq
    g = torch.Generator().manual_seed(77)
    B, Hq, Hkv, Tq, T, W, d = 1, 8, 2, 7, 1300, 20, 128
    K = (torch.randn((B, Hkv, T, d), generator=g).cumsum(2) * 0.2)
    V = torch.randn((B, Hkv, T, d), generator=g)
    q = torch.randn((B, Hq, Tq, d), generator=g)
    cache = kvq.DctCache.from_context(K.cuda(), V.cuda(), window=W)
    ref = _oracle(cache, q, d ** -0.5)
    for chunk in (None, 3):
        out = kvq.dct_decode(q.cuda(), d ** -0.5, cache, chunk=chunk).cpu().numpy()
        assert float(np.abs(out - ref).max()) <= 2e-3
