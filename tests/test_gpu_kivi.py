"""GPU kivi_quant / pack_codes / tile layouts against the CPU oracle: bit-exact.

Covers keys and values, 2/4/8 bits, groups that do and do not divide the rows, sinks, every
input dtype, a padded last key group, degenerate (constant) groups and heavy-tailed data.
"""
import numpy as np
import pytest
import torch

import oracle.kivi as ok

pytestmark = pytest.mark.gpu


def _data(shape, seed, dtype, heavy=False):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(shape, generator=g)
    if heavy:
        x *= torch.randn((*shape[:2], 1, shape[3]), generator=g).abs() * 10
    x[..., :2, :3] = 1.25                       # constant sub-blocks: zero ranges
    return x.to(dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("bits", [2, 4, 8])
@pytest.mark.parametrize("along,group,n_sink,T", [(True, 32, 0, 4096), (True, 64, 4, 203),
                                                  (True, 16, 0, 100), (False, 32, 0, 300),
                                                  (False, 64, 3, 129), (False, 48, 0, 17),
                                                  (False, 8, 0, 70), (False, 16, 5, 200)])
def test_kivi_quant_bit_exact(dtype, bits, along, group, n_sink, T):
    import kvq
    x = _data((2, 3, T, 128), 1000 + T + bits, dtype, heavy=along)
    ref = ok.kivi_quant(x.float().numpy(), bits, group, along, n_sink)
    got = kvq.kivi_quant(x.cuda(), bits, group, along, n_sink)
    np.testing.assert_array_equal(got["codes"].cpu().numpy(), ref["codes"])
    np.testing.assert_array_equal(got["lo"].cpu().numpy(), ref["lo"])
    np.testing.assert_array_equal(got["scale"].cpu().numpy(), ref["scale"])
    np.testing.assert_array_equal(got["xhat"].cpu().numpy(), ref["xhat"])
    st = kvq.kivi_quant_stored(x.cuda(), bits, group, along, n_sink)
    _check_stored(st, ref, bits, along)


def _check_stored(st, ref, bits, along):
    """The packed-only output (the decode cache's prefill path) against the oracle."""
    ax = 3 if along else 4
    np.testing.assert_array_equal(st["lo"].float().unsqueeze(ax).cpu().numpy(), ref["lo"])
    np.testing.assert_array_equal(st["scale"].float().unsqueeze(ax).cpu().numpy(), ref["scale"])
    B, H = ref["codes"].shape[:2]
    for b_ in range(B):
        for h in range(H):
            want = ok.pack_codes(ref["codes"][b_, h], bits)
            np.testing.assert_array_equal(st["packed"][b_, h].cpu().numpy().ravel(), want)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("along,group", [(True, 64), (True, 32), (False, 64), (False, 128)])
def test_kivi_quant_stored_strided_input(dtype, along, group):
    """A view of the first n rows of a longer cache (row stride kept, as the prefill quantises
    K[:, :, :n]), with a ragged last group and rows whose quotients sit on half-integers."""
    import kvq
    full = _data((2, 4, 700, 128), 77 + group, dtype, heavy=along)
    full[:, :, 10:20] = (torch.arange(128) % 16).to(dtype) * 0.5          # exact code grid
    ref = ok.kivi_quant(full[:, :, :613].float().numpy(), 4, group, along, 0)
    x = full.cuda()[:, :, :613]
    assert x.stride(2) == 128 and x.stride(1) == 700 * 128
    st = kvq.kivi_quant_stored(x, 4, group, along, 0)
    _check_stored(st, ref, 4, along)


@pytest.mark.parametrize("bits", [1, 2, 4, 8])
@pytest.mark.parametrize("count", [1, 5, 4096, 100003])
def test_pack_unpack_codes(bits, count):
    import kvq
    rng = np.random.default_rng(count + bits)
    c = rng.integers(0, 2 ** bits, count).astype(np.uint8)
    packed = kvq.pack_codes(torch.from_numpy(c).cuda(), bits)
    np.testing.assert_array_equal(packed.cpu().numpy(), ok.pack_codes(c, bits))
    back = kvq.unpack_codes(packed, bits, count)
    np.testing.assert_array_equal(back.cpu().numpy(), c)


@pytest.mark.parametrize("n,cap", [(32, 32), (100, 128), (3968, 4096), (1, 64)])
def test_value_tiles_round_trip(n, cap):
    import kvq
    rng = np.random.default_rng(n)
    rows = rng.integers(0, 256, (2, 3, n, 64)).astype(np.uint8)
    t = kvq.v_tile(torch.from_numpy(rows).cuda(), cap)
    back = kvq.v_untile(t, n)
    np.testing.assert_array_equal(back.cpu().numpy(), rows)
    # spot-check the documented word layout: word (q, lane, b4) of chunk 0, nibble k = slot order
    words = t.cpu().numpy()[0, 0, 0].view(np.uint32).reshape(2, 64, 4)
    slot_of_nib = [0, 2, 4, 6, 1, 3, 5, 7]
    for (q, lane, b4) in [(0, 0, 0), (1, 37, 3), (0, 63, 2)]:
        ch = 16 * (4 * q + b4) + lane % 16
        g = lane // 16
        for k in range(8):
            j = slot_of_nib[k]
            tok = 16 * (j // 4) + 4 * g + (j % 4)
            want = 0
            if tok < n:
                byte = rows[0, 0, tok, ch // 2]
                want = (byte & 15) if ch % 2 else (byte >> 4)
            assert (int(words[q, lane, b4]) >> (4 * k)) & 15 == want


def test_vmeta_tile_layout():
    import kvq
    rng = np.random.default_rng(5)
    n, cap, ngv = 70, 96, 2
    lo = rng.standard_normal((1, 2, n, ngv)).astype(np.float16)
    sc = rng.standard_normal((1, 2, n, ngv)).astype(np.float16)
    vm = kvq.vmeta_tile(torch.from_numpy(lo).cuda(), torch.from_numpy(sc).cuda(), cap).cpu().numpy()
    assert vm.shape == (1, 2, cap // 32, ngv, 32, 2)
    for chunk in range(cap // 32):
        for gc in range(ngv):
            for p in range(32):
                g, j = p // 8, p % 8
                tok = chunk * 32 + 16 * (j // 4) + 4 * g + (j % 4)
                want = (sc[0, 1, tok, gc], lo[0, 1, tok, gc]) if tok < n else (0, 0)
                assert tuple(vm[0, 1, chunk, gc, p]) == tuple(np.float16(w) for w in want)


@pytest.mark.parametrize("bits", [1, 2, 4, 8])
def test_pack_rows_and_lut_decode(bits):
    """kvq.pack_rows bit-exact to the restated pack_rows (QUASAR_KV.py:1185-1190); kvq.unpack_rows
    (one table lookup per byte, QUASAR_KV.py:1194-1202) returns levels[code] exactly."""
    import kvq
    rng = np.random.default_rng(40 + bits)
    c = rng.integers(0, 2 ** bits, (3, 5, 256)).astype(np.uint8)
    packed = kvq.pack_rows(torch.from_numpy(c).cuda(), bits)
    np.testing.assert_array_equal(packed.cpu().numpy(), ok.pack_rows(c, bits))
    levels = rng.standard_normal(2 ** bits).astype(np.float32)
    got = kvq.unpack_rows(packed, bits, torch.from_numpy(levels).cuda())
    np.testing.assert_array_equal(got.cpu().numpy(), levels[c])
    np.testing.assert_array_equal(got.cpu().numpy(), ok.unpack_rows_lut(ok.pack_rows(c, bits), bits, levels))
