"""STRATA codec, planar packing and value tiles on the GPU against the CPU oracle (bit-exact).

* pack_planar / unpack_planar (STRATA_KV.py:1171-1189) for 2/4/8 bits;
* centring + rotation (1546-1547): fp16 means and float32 rotated rows equal the oracle's bit for
  bit (same fixed arithmetic order), for fp32 and bf16 inputs;
* strata_quantize (1158-1168): planar codes and fp16 scales, all rows and a gathered subset;
* the decode kernel's value tiles: every (token, channel) code read back through the documented
  word layout equals the planar code; slot-ordered scales.
"""
import numpy as np
import pytest
import torch

import oracle.strata as os_
from layouts import slot_token as _slot_token, tile_codes as _tile_codes

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_planar_pack_unpack(bits):
    import kvq
    rng = np.random.default_rng(bits)
    codes = rng.integers(0, 2 ** bits, (3, 37, 128)).astype(np.uint8)
    packed = kvq.pack_planar(torch.from_numpy(codes).cuda(), bits).cpu().numpy()
    np.testing.assert_array_equal(packed, os_.pack_planar(codes, bits))
    back = kvq.unpack_planar(torch.from_numpy(packed).cuda(), bits)
    assert back.dtype == torch.int32                         # the reference's return type
    np.testing.assert_array_equal(back.cpu().numpy(), codes)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_center_rotate_and_quantize_bit_exact(dtype):
    import kvq
    g = torch.Generator().manual_seed(3)
    B, H, n, d = 2, 3, 301, 128
    x = (torch.randn((B, H, n, d), generator=g) * 3 + 0.7).to(dtype)
    mu, y = kvq.strata_center_rotate(x.cuda())
    s = os_.rotation_signs(d)
    mu_o, y_o = os_.strata_center_rotate(x.float().numpy().reshape(B * H, n, d), s)
    np.testing.assert_array_equal(mu.float().cpu().numpy().reshape(B * H, d), mu_o)
    np.testing.assert_array_equal(y.cpu().numpy().reshape(B * H, n, d), y_o)
    for bits in (2, 4, 8):
        assert kvq.uniform_step(bits) == os_.uniform_step(bits)            # (step, mse)
        codes, sc = kvq.strata_quantize_planar(y, bits)
        c_o, s_o, yh_o = os_.strata_quantize(y_o, bits, os_.uniform_step(bits)[0])
        np.testing.assert_array_equal(codes.cpu().numpy().reshape(B * H, n, -1), os_.pack_planar(c_o, bits))
        np.testing.assert_array_equal(sc.float().cpu().numpy().reshape(B * H, n), s_o)
        # the reference's call shape: (codes uint8 (..., d), s (...), y_hat (..., d)) of any leading shape
        c_r, s_r, yh_r = kvq.strata_quantize(y[1], bits)
        assert c_r.dtype == torch.uint8 and tuple(c_r.shape) == (H, n, d) and tuple(s_r.shape) == (H, n)
        np.testing.assert_array_equal(c_r.cpu().numpy(), c_o.reshape(B, H, n, d)[1])
        np.testing.assert_array_equal(s_r.cpu().numpy(), s_o.reshape(B, H, n)[1])
        np.testing.assert_array_equal(yh_r.cpu().numpy(), yh_o.reshape(B, H, n, d)[1])
        idx = torch.stack([torch.randperm(n, generator=g)[:50] for _ in range(B * H)]).reshape(B, H, 50)
        cg, sg = kvq.strata_quantize_planar(y, bits, idx.cuda())
        ii = idx.numpy().reshape(B * H, 50)
        want = os_.pack_planar(np.take_along_axis(c_o, ii[..., None], 1), bits)
        np.testing.assert_array_equal(cg.cpu().numpy().reshape(B * H, 50, -1), want)
        np.testing.assert_array_equal(sg.float().cpu().numpy().reshape(B * H, 50), np.take_along_axis(s_o, ii, 1))


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_quantize_scales_at_fp16_ties(bits):
    # every row's float32(step * rms) is an fp16 rounding midpoint: the stored scale is right only
    # if rms is the correctly rounded square root (one ulp either way picks the other neighbour)
    import kvq
    from midpoint_rows import midpoint_rows
    step = os_.uniform_step(bits)[0]
    Y = midpoint_rows(bits, 4096, seed=100 + bits, step=step).reshape(2, 2, 1024, 128)
    codes, sc = kvq.strata_quantize_planar(torch.from_numpy(Y).cuda(), bits)
    c_o, s_o, _ = os_.strata_quantize(Y.reshape(4, 1024, 128), bits, step)
    got = sc.float().cpu().numpy().reshape(4, 1024)
    assert np.array_equal(got, s_o), f"{int((got != s_o).sum())} of 4096 scales differ"
    np.testing.assert_array_equal(codes.cpu().numpy().reshape(4, 1024, -1), os_.pack_planar(c_o, bits))


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_value_tiles_layout(bits):
    import kvq
    rng = np.random.default_rng(10 + bits)
    B, H, n, cap = 1, 2, 70, 96
    codes = rng.integers(0, 2 ** bits, (B, H, n, 128)).astype(np.uint8)
    vs = rng.random((B, H, n)).astype(np.float16)
    rows = torch.from_numpy(os_.pack_planar(codes, bits)).cuda()
    tiles, vsl = kvq.strata_v_tile(rows, torch.from_numpy(vs).cuda(), bits, cap)
    tiles, vsl = tiles.cpu().numpy(), vsl.cpu().numpy()
    full = np.zeros((B, H, cap, 128), np.int64)
    full[:, :, :n] = codes
    vfull = np.zeros((B, H, cap), np.float16)
    vfull[:, :, :n] = vs
    for h in range(H):
        for c in range(cap // 32):
            got = _tile_codes(tiles[0, h, c], bits)
            np.testing.assert_array_equal(got, full[0, h, 32 * c:32 * c + 32])
            want_s = [vfull[0, h, 32 * c + _slot_token(s // 8, s % 8)] for s in range(32)]
            np.testing.assert_array_equal(vsl[0, h, c], np.array(want_s, np.float16))


def _assign(B, H, nc, fracs, g):
    """Per (b, h): tokens ranked by a random importance; the top fracs[0] -> 8 bits, the next
    fracs[1] -> 4 bits, the next fracs[2] -> 2 bits, the rest dropped (level 0)."""
    imp = torch.rand((B, H, nc), generator=g)
    order = imp.argsort(-1, descending=True).to(torch.int32)
    out, a = [], 0
    for bits, f in zip((8, 4, 2), fracs):
        m = int(round(f * nc))
        if m:
            out.append((bits, order[..., a:a + m].contiguous()))
        a += m
    return out


def _oracle_out(cache, q, K, V, window, scaling):
    B = q.shape[0]
    d = q.shape[-1]
    R = os_.rotation_matrix(d)
    outs = []
    for b in range(B):
        tiers = []
        for t in cache.tiers:
            ck = os_.unpack_planar(t.kc[b].cpu().numpy(), t.bits)
            cv = os_.unpack_planar(t.vc[b].cpu().numpy(), t.bits)
            tiers.append((t.bits, ck, t.ks[b, :, :t.n].float().cpu().numpy(), cv, t.vs[b].float().cpu().numpy()))
        nc = K.shape[2] - window
        outs.append(os_.strata_attend(q[b:b + 1].float().numpy(), scaling, K[b, :, nc:].float().numpy(),
                                      V[b, :, nc:].float().numpy(), tiers, cache.mu_k[b].float().cpu().numpy(),
                                      cache.mu_v[b].float().cpu().numpy(), R))
    return np.concatenate(outs, 0)


@pytest.mark.parametrize("dtype,Hq,Hkv,Tq", [(torch.float32, 8, 2, 1), (torch.bfloat16, 8, 2, 1),
                                             (torch.float32, 8, 2, 2)])
def test_strata_decode_mixed_tiers(dtype, Hq, Hkv, Tq):
    import kvq
    g = torch.Generator().manual_seed(5 + Tq)
    B, T, W, d = 2, 700, 40, 128
    K = (torch.randn((B, Hkv, T, d), generator=g) * 1.5 + 0.3).to(dtype)
    V = torch.randn((B, Hkv, T, d), generator=g).to(dtype)
    q = torch.randn((B, Hq, Tq, d), generator=g).to(dtype)
    assign = _assign(B, Hkv, T - W, (0.1, 0.3, 0.5), g)
    cache = kvq.StrataCache.from_context(K.cuda(), V.cuda(), window=W, assign=assign)
    out = kvq.strata_decode(q.cuda(), d ** -0.5, cache).float().cpu().numpy()
    ref = _oracle_out(cache, q, K, V, W, d ** -0.5)
    err = float(np.abs(out - ref).max())
    tol = 2e-3 if dtype == torch.float32 else 1e-2
    assert err <= tol, err


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_strata_decode_single_width_no_exact_rows(bits):
    import kvq
    g = torch.Generator().manual_seed(40 + bits)
    B, Hq, Hkv, T, d = 1, 4, 4, 1000, 128
    K = torch.randn((B, Hkv, T, d), generator=g)
    V = torch.randn((B, Hkv, T, d), generator=g)
    q = torch.randn((B, Hq, 1, d), generator=g)
    idx = torch.stack([torch.randperm(T, generator=g)[:777] for _ in range(Hkv)])[None].to(torch.int32)
    cache = kvq.StrataCache.from_context(K.cuda(), V.cuda(), window=0, assign=[(bits, idx)])
    cache.n_exact = 0
    out = kvq.strata_decode(q.cuda(), d ** -0.5, cache).cpu().numpy()
    ref = _oracle_out(cache, q, K, V, 0, d ** -0.5)
    assert float(np.abs(out - ref).max()) <= 2e-3


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_strata_decode_long_window(dtype):
    """A window of 1100 exact rows, past what the merge attends itself: exact-row blocks write
    partials, and the one-wavefront-per-row merge (at most 32 partials, none attended in the merge)
    combines them, unrotated, with the strata's rotated partials."""
    import kvq
    g = torch.Generator().manual_seed(61)
    B, Hq, Hkv, T, W, d = 1, 8, 2, 2300, 1100, 128
    K = (torch.randn((B, Hkv, T, d), generator=g) * 1.5 + 0.3).to(dtype)
    V = torch.randn((B, Hkv, T, d), generator=g).to(dtype)
    q = torch.randn((B, Hq, 1, d), generator=g).to(dtype)
    assign = _assign(B, Hkv, T - W, (0.1, 0.3, 0.5), g)
    cache = kvq.StrataCache.from_context(K.cuda(), V.cuda(), window=W, assign=assign)
    assert cache.n_exact == W
    print(f"strata long window: {dtype} T {T} W {W}", flush=True)
    out = kvq.strata_decode(q.cuda(), d ** -0.5, cache).float().cpu().numpy()
    ref = _oracle_out(cache, q, K, V, W, d ** -0.5)
    err = float(np.abs(out - ref).max())
    assert err <= (2e-3 if dtype == torch.float32 else 1e-2), err


def test_strata_decode_many_query_tokens():
    """Tq 5 at rep 4 (20 rows per KV head): query-token pieces of 2, 2 and 1 tokens, each a full
    decode launch, against the oracle over the whole block of queries."""
    import kvq
    g = torch.Generator().manual_seed(55)
    B, Hq, Hkv, Tq, T, W, d = 1, 8, 2, 5, 600, 32, 128
    K = (torch.randn((B, Hkv, T, d), generator=g) * 1.5 + 0.3)
    V = torch.randn((B, Hkv, T, d), generator=g)
    q = torch.randn((B, Hq, Tq, d), generator=g)
    assign = _assign(B, Hkv, T - W, (0.1, 0.3, 0.5), g)
    cache = kvq.StrataCache.from_context(K.cuda(), V.cuda(), window=W, assign=assign)
    out = kvq.strata_decode(q.cuda(), d ** -0.5, cache).float().cpu().numpy()
    ref = _oracle_out(cache, q, K, V, W, d ** -0.5)
    assert out.shape == (B, Tq, Hq, d)
    assert float(np.abs(out - ref).max()) <= 2e-3


@pytest.mark.parametrize("B,T,fracs", [(4, 4096, (0.1, 0.3, 0.5)), (4, 2048, (0.01, 0.3, 0.5))])
def test_strata_decode_class_plan(B, T, fracs):
    """B 4 x Hkv 8 = 32 (b, h): one round of 3 blocks per CU holds 768 / 32 = 24 splits per (b, h).
    At T 4096 every stratum has chunks for at least one split per dispatch class (8-bit 403 tokens,
    4-bit 1210, 2-bit 2016), so the splits are mapped class-major and sized by class weight; at
    T 2048 with 1% 8-bit tokens (20 tokens, one chunk) the plan falls back to byte-sized splits.
    Both against the oracle."""
    import kvq
    g = torch.Generator().manual_seed(81 + T)
    Hq, Hkv, W, d = 32, 8, 64, 128
    K = (torch.randn((B, Hkv, T, d), generator=g) * 1.5 + 0.3).to(torch.bfloat16)
    V = torch.randn((B, Hkv, T, d), generator=g).to(torch.bfloat16)
    q = torch.randn((B, Hq, 1, d), generator=g).to(torch.bfloat16)
    assign = _assign(B, Hkv, T - W, fracs, g)
    cache = kvq.StrataCache.from_context(K.cuda(), V.cuda(), window=W, assign=assign)
    out = kvq.strata_decode(q.cuda(), d ** -0.5, cache).float().cpu().numpy()
    ref = _oracle_out(cache, q, K, V, W, d ** -0.5)
    assert float(np.abs(out - ref).max()) <= 1e-2
