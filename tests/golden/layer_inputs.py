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
