"""Seeded inputs of the reference-compressed golden layers (tests/golden/make_fixtures.py writes
the reference's outputs for them; the tests rebuild the same inputs from the seed, so the
fixtures need not hold the layer's queries, keys and values).  numpy's PCG64 streams are
reproducible across machines and versions."""
import numpy as np


def strata_layer(seed: int = 20260104, Hq: int = 8, Hkv: int = 2, H: int = 700, d: int = 128, hidden: int = 256):
    """q (1, Hq, H, d), k, v (1, Hkv, H, d), the output projection Wo (hidden, Hq d), and one
    decode step after the context: kn, vn (1, Hkv, 1, d), qn (1, Hq, 1, d); all float32."""
    rng = np.random.default_rng(seed)
    rep = Hq // Hkv
    q = (rng.standard_normal((1, Hq, H, d)) * 1.5).astype(np.float32)
    k = (rng.standard_normal((1, Hkv, H, d)) * (np.abs(rng.standard_t(3, (1, Hkv, 1, d))) + 0.3)).astype(np.float32)
    v = rng.standard_normal((1, Hkv, H, d)).astype(np.float32)
    k[:, :, 0] += 2.0 * q[0, ::rep].mean(1)[None]                      # a sink the queries lean on
    hot = rng.permutation(H - 64)[:16] + 16                            # a few heavily read tokens
    k[:, :, hot] += 1.5 * q[0, ::rep, -32:].mean(1)[None, :, None]
    Wo = (rng.standard_normal((hidden, Hq * d)) / np.sqrt(Hq * d)).astype(np.float32)
    kn = rng.standard_normal((1, Hkv, 1, d)).astype(np.float32)
    vn = rng.standard_normal((1, Hkv, 1, d)).astype(np.float32)
    qn = (rng.standard_normal((1, Hq, 1, d)) * 1.5).astype(np.float32)
    return q, k, v, Wo, kn, vn, qn


def out_metric(Wo: np.ndarray, Hq: int, d: int) -> np.ndarray:
    """M_a = W_O,a^T W_O,a per query head (Hq, d, d), float32 (STRATA_KV.py:1519-1526)."""
    Wa = Wo.reshape(Wo.shape[0], Hq, d).transpose(1, 0, 2)
    return np.einsum("ahi,ahj->aij", Wa, Wa).astype(np.float32)


def kivi_inputs(seed: int = 20260105):
    """Seeded inputs of the kivi_attention fixture: keys with heavy-tailed channel scales and values
    (1, 2, 100, 128) (100 tokens: a partial group of 32 and of 64), the query and entries of one
    chunked_attention call, SnapKV's layer (q (1, 8, 300, 128), k (1, 2, 300, 128)), and one
    stratum's query / codes for tier_reference; all float32 / uint8."""
    rng = np.random.default_rng(seed)
    d = 128
    K = (rng.standard_normal((1, 2, 100, d)) * (np.abs(rng.standard_t(3, (1, 2, 1, d))) + 0.2)).astype(np.float32)
    V = rng.standard_normal((1, 2, 100, d)).astype(np.float32)
    qa = rng.standard_normal((1, 8, 3, d)).astype(np.float32)
    tk = rng.standard_normal((1, 2, 50, d)).astype(np.float32)
    tv = rng.standard_normal((1, 2, 50, d)).astype(np.float32)
    qs = (rng.standard_normal((1, 8, 300, d)) * 1.5).astype(np.float32)
    ks = rng.standard_normal((1, 2, 300, d)).astype(np.float32)
    ks[:, :, 7] += 2.0 * qs[0, ::4, -64:].mean(1)[None]
    qr = rng.standard_normal((2, 5, d)).astype(np.float32)
    qb = rng.standard_normal((2, 5)).astype(np.float32)
    codes = {b: (rng.integers(0, 2 ** b, (2, 40, d)).astype(np.uint8), rng.integers(0, 2 ** b, (2, 40, d)).astype(np.uint8))
             for b in (2, 4, 8)}
    scales = {b: ((rng.random((2, 40)) * 0.1 + 0.01).astype(np.float32), (rng.random((2, 40)) * 0.1 + 0.01).astype(np.float32))
              for b in (2, 4, 8)}
    return {"K": K, "V": V, "qa": qa, "tk": tk, "tv": tv, "qs": qs, "ks": ks, "qr": qr, "qb": qb,
            "codes": codes, "scales": scales}
