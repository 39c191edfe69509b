"""The decode kernel's lane mapping, checked on the hardware (in-bounds, one wavefront).

v_mfma_f32_16x16x32_f16 operand layout assumed by kv-project_amd/csrc/decode.hip:
  A (16x32): lane l holds A[l%16][8*(l/16) + k], k = 0..7
  B (32x16): lane l holds B[8*(l/16) + k][l%16]
  D (16x16): lane l register i holds D[4*(l/16) + i][l%16]
DPP row_shr:4: lane i of a 16-lane row reads lane i-4 (lanes 0..3 keep their old value);
row_ror:4 reads lane (i -+ 4) mod 16 of the same row.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def test_mfma_16x16x32_f16_layout_and_dpp():
    from kvq import _lib
    rng = np.random.default_rng(0)
    A = rng.integers(-4, 5, (16, 32)).astype(np.float16)
    Bm = rng.integers(-4, 5, (32, 16)).astype(np.float16)
    a = np.empty((64, 8), np.float16)
    b = np.empty((64, 8), np.float16)
    for l in range(64):
        a[l] = A[l % 16, 8 * (l // 16): 8 * (l // 16) + 8]
        b[l] = Bm[8 * (l // 16): 8 * (l // 16) + 8, l % 16]
    ta = torch.from_numpy(a.view(np.uint16).astype(np.int16)).cuda()
    tb = torch.from_numpy(b.view(np.uint16).astype(np.int16)).cuda()
    out = torch.zeros(640, dtype=torch.float32, device="cuda")
    _lib.call("kvq_selftest_mfma_layout", ta.data_ptr(), tb.data_ptr(), out.data_ptr(), 0)
    torch.cuda.synchronize()
    o = out.cpu().numpy()
    D = A.astype(np.float64) @ Bm.astype(np.float64)
    got = o[:256].reshape(64, 4)
    for l in range(64):
        for i in range(4):
            assert got[l, i] == D[4 * (l // 16) + i, l % 16], (l, i)
    shr = o[256:320].astype(int)
    ror = o[320:384].astype(int)
    for l in range(64):
        base, i = l - l % 16, l % 16
        assert shr[l] == (l - 4 if i >= 4 else -1), (l, shr[l])
        assert ror[l] in (base + (i - 4) % 16, base + (i + 4) % 16), (l, ror[l])
    # permlane swaps: every lane holds itself and its xor-32 / xor-16 partner across the two results
    s32a, s32b, s16a, s16b = (o[384 + 64 * k: 448 + 64 * k].astype(int) for k in range(4))
    for l in range(64):
        assert {s32a[l], s32b[l]} == {l, l ^ 32}, (l, s32a[l], s32b[l])
        assert {s16a[l], s16b[l]} == {l, l ^ 16}, (l, s16a[l], s16b[l])


def test_mfma_f16_subnormal_operands_are_exact():
    """fp16 subnormals (the bit pattern of a 4-bit code masked in place is c * 2^-24 or 16c * 2^-24)
    enter the matrix core unflushed: D = 2^-24 * sum(c * b) to the unit's own dot-product precision
    (measured ~2e-6 of sum|c * b|; flushing would give 0)."""
    from kvq import _lib
    rng = np.random.default_rng(1)
    codes = rng.integers(0, 16, (16, 32))
    kappa = np.where(rng.integers(0, 2, (16, 32)) == 1, 16, 1)       # low or high nibble position
    A_bits = (codes * kappa).astype(np.uint16)                       # subnormal fp16 bit patterns
    Bm = (rng.standard_normal((32, 16)) * 4).astype(np.float16)
    a = np.empty((64, 8), np.uint16)
    b = np.empty((64, 8), np.float16)
    for l in range(64):
        a[l] = A_bits[l % 16, 8 * (l // 16): 8 * (l // 16) + 8]
        b[l] = Bm[8 * (l // 16): 8 * (l // 16) + 8, l % 16]
    ta = torch.from_numpy(a.astype(np.int16)).cuda()
    tb = torch.from_numpy(b.view(np.uint16).astype(np.int16)).cuda()
    out = torch.zeros(640, dtype=torch.float32, device="cuda")
    _lib.call("kvq_selftest_mfma_layout", ta.data_ptr(), tb.data_ptr(), out.data_ptr(), 0)
    torch.cuda.synchronize()
    got = out.cpu().numpy()[:256].reshape(64, 4).astype(np.float64)
    D = (codes * kappa).astype(np.float64) @ Bm.astype(np.float64) * 2.0 ** -24
    mag = (codes * kappa).astype(np.float64) @ np.abs(Bm.astype(np.float64)) * 2.0 ** -24
    worst = 0.0
    for l in range(64):
        for i in range(4):
            m, n = 4 * (l // 16) + i, l % 16
            rel = abs(got[l, i] - D[m, n]) / mag[m, n]
            worst = max(worst, rel)
    print(f"subnormal-operand dot products: worst error / sum|c*b| = {worst:.3e}")
    assert worst <= 1e-5
