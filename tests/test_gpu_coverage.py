"""Device coverage statistics (kvq.coverage_stats, STRATA_KV.py:1225-1298) against the float64 oracle.

The oracle (oracle/coverage.py) is pinned by the reference's group draws, Prop. 1 by brute force and
the value / key terms by exact perturbation and finite differences.  Here the device path runs on
seeded inputs of the storage dtype and is compared with the oracle on the same (dtype-rounded)
values:
* bf16, GQA rep 4, every group reaching the coded range [N_SINK, H - WINDOW);
* fp32 with rep 1 and key / value rows past H filled with NaN (never read: the causal range ends at
  H - 1 and the tiles past it are masked or zeroed);
* fp16 with rep 8 and rs past the first segment's queries (that group is skipped and not live);
* window_only (the window group alone, local distance 1).
Bar: max-abs-err of A, W, DD, S <= 2e-4 x the largest |value| of the output (fp32 sums of a few
thousand positive terms), Mbar <= 1e-5 x its largest |value|; and two runs are bit-identical
(every sum has a fixed order).
"""
import numpy as np
import pytest
import torch

import oracle.coverage as oc

pytestmark = pytest.mark.gpu

D = 128


def _inputs(seed, Hq, Hkv, T, H, dtype, nan_tail=False):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(1, Hq, T, D, generator=g) * 1.5
    k = torch.randn(1, Hkv, T, D, generator=g)
    v = torch.randn(1, Hkv, T, D, generator=g)
    k[:, :, 0] += 2.0 * q[0, ::Hq // Hkv, :, :].mean(1)[None]       # a sink the queries lean on
    Wo = torch.randn(Hq, 32, D, generator=g)
    M = (Wo.transpose(1, 2) @ Wo) / 32
    q, k, v = q.to(dtype), k.to(dtype), v.to(dtype)
    if nan_tail:
        k[:, :, H:] = float("nan")
        v[:, :, H:] = float("nan")
    return q, k, v, M


def _oracle(q, k, v, M, H, rs, re, window_only=False):
    qn = q[0, :, :H].double().numpy()
    st = oc.coverage_stats(qn, np.arange(H), k[0, :, :H].double().numpy(), v[0, :, :H].double().numpy(), D ** -0.5,
                           H, rs, re, M.double().numpy(), oc.CoverageParams(), window_only=window_only)
    return st


def _check(got, ref, name, rel):
    g = got.float().cpu().numpy()
    r = ref[name]
    scale = float(np.abs(r).max())
    err = float(np.abs(g - r).max())
    print(f"  {name}: max-abs-err {err:.3e} (scale {scale:.3e})", flush=True)
    assert np.isfinite(g).all(), name
    # plus fp32's smallest normal: statistics whose true size is below it are zero in any fp32 sum
    assert err <= rel * scale + np.finfo(np.float32).tiny, (name, err, scale)


def _run(q, k, v, M, H, rs, re, window_only=False):
    import kvq
    st = kvq.coverage_stats(q.cuda(), k.cuda(), v.cuda(), D ** -0.5, H, rs, re, M.cuda(), window_only=window_only)
    torch.cuda.synchronize()
    return st


def _compare(st, ref):
    for name in ("A", "W", "DD", "S"):
        _check(st[name], ref, name, 2e-4)
    _check(st["Mbar"], ref, "Mbar", 1e-5)
    assert [len(g) for g in st["groups"]] == [len(g) for g in ref["groups"]]


@pytest.mark.parametrize("case", ["bf16_rep4", "f32_rep1_nan_tail", "f16_rep8_skip", "bf16_rep16", "bf16_rep1",
                                  "f16_rep2_ragged"])
def test_coverage_stats_matches_oracle(case):
    # 16-bit rows with up to 8 query heads per KV head take the LDS form of the token terms; fp32
    # rows and rep 16 the form that reads its tiles from memory
    if case == "bf16_rep4":
        Hq, Hkv, T, H, dt, rs, re, nan = 8, 2, 1200, 1200, torch.bfloat16, 4, 1168, False
    elif case == "bf16_rep16":
        Hq, Hkv, T, H, dt, rs, re, nan = 16, 1, 700, 700, torch.bfloat16, 4, 668, False
    elif case == "bf16_rep1":
        Hq, Hkv, T, H, dt, rs, re, nan = 3, 3, 900, 900, torch.bfloat16, 4, 868, False
    elif case == "f16_rep2_ragged":      # coded range and context not multiples of 16 or 256
        Hq, Hkv, T, H, dt, rs, re, nan = 4, 2, 1011, 1003, torch.float16, 7, 971, False
    elif case == "f32_rep1_nan_tail":
        Hq, Hkv, T, H, dt, rs, re, nan = 4, 4, 336, 300, torch.float32, 4, 268, True
    else:
        Hq, Hkv, T, H, dt, rs, re, nan = 16, 2, 1500, 1500, torch.float16, 600, 1468, False
    print(f"coverage {case}: Hq {Hq} Hkv {Hkv} H {H} T {T} rs {rs} re {re}", flush=True)
    q, k, v, M = _inputs(7, Hq, Hkv, T, H, dt, nan)
    st = _run(q, k, v, M, H, rs, re)
    _compare(st, _oracle(q, k, v, M, H, rs, re))


@pytest.mark.parametrize("qs,ks,vs", [(2.0 ** -17, 2.0 ** 17, 2.0 ** 17), (2.0 ** 20, 2.0 ** -20, 2.0 ** -20),
                                      (2.0 ** -122, 1.0, 1.0)])
def test_coverage_stats_fp32_extreme_magnitudes(qs, ks, vs):
    """fp32 rows far outside fp16's range (keys and values up to ~6e5, past 65504) and far below it
    (~4e-6): each tensor is brought into the fp16 parts' range by a power of two before the products
    and the results scaled back, so the statistics match the oracle at the usual bar.  Queries near
    fp32's smallest normal (~2^-120, logits ~0): the power stays finite (at most 2^63), so the
    statistics are those of uniform attention, as the oracle's, not NaN."""
    q, k, v, M = _inputs(13, 8, 2, 640, 640, torch.float32)
    q, k, v = q * qs, k * ks, v * vs
    print(f"coverage fp32 magnitudes: |k| max {float(k.abs().max()):.3e}, |v| max {float(v.abs().max()):.3e}", flush=True)
    st = _run(q, k, v, M, 640, 4, 608)
    _compare(st, _oracle(q, k, v, M, 640, 4, 608))


def test_coverage_window_only_and_deterministic():
    q, k, v, M = _inputs(11, 8, 2, 1200, 1200, torch.bfloat16)
    print("coverage window_only: Hq 8 Hkv 2 H 1200", flush=True)
    st = _run(q, k, v, M, 1200, 4, 1168, window_only=True)
    _compare(st, _oracle(q, k, v, M, 1200, 4, 1168, window_only=True))
    print("coverage determinism: two runs", flush=True)
    a = _run(q, k, v, M, 1200, 4, 1168)
    b = _run(q, k, v, M, 1200, 4, 1168)
    for name in ("A", "W", "DD", "S", "Mbar"):
        assert torch.equal(a[name], b[name]), name
