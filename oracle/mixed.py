"""Mixed-width KIVI coding of 64-token blocks and the decode over it (numpy restatement).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Each 64-token block of one (KV head) gets its own code width b in {2, 4, 8}; inside the block the
codes are exactly kivi_quant's (STRATA_KV.py:826-856) at that width with group 32: keys per
channel over the two 32-token groups, values per token over four 32-channel groups.  Because
64 % 32 == 0 no group straddles two blocks, so the coded context equals, block by block, the
output of kivi_quant over the whole context at that block's width; this module computes it that
way.  The decode is chunked_attention (641-675) over the blocks' xhat entries plus exact rows.

Width assignment of the C3 workload (the build fixes the rounding): per (b, h) the blocks are
ranked by importance (descending, stable); the first floor(0.1 nb) get 8 bits, the next
floor(0.4 nb) - floor(0.1 nb) get 4 bits, the rest 2 bits (25 / 77 / 154 of 256 blocks).

Pinning (tests/test_oracle_mixed.py): with every block at one width the codes, metadata and
xhat equal kivi_quant's at that width (pinned in test_oracle_kivi.py), and the decode equals
kivi_decode_reference; the width counts of the C3 rule; every block's codes reconstruct within
half a step of the input (the KIVI error bound) at its own width.
"""
from __future__ import annotations

import numpy as np

from .attention import chunked_attention
from .kivi import kivi_quant

BLOCK = 64
GROUP = 32
WIDTHS = (2, 4, 8)


def c3_widths(importance: np.ndarray) -> np.ndarray:
    """importance (B, H, nb) -> widths (B, H, nb) int: top floor(0.1 nb) -> 8, next
    floor(0.4 nb) - floor(0.1 nb) -> 4, the rest -> 2 (ranking descending, stable)."""
    nb = importance.shape[-1]
    n8 = int(np.floor(0.1 * nb))
    n4 = int(np.floor(0.4 * nb)) - n8
    order = np.argsort(-importance, axis=-1, kind="stable")
    rank = np.argsort(order, axis=-1, kind="stable")                        # inverse permutation
    w = np.full(importance.shape, 2, np.int64)
    w[rank < n8 + n4] = 4
    w[rank < n8] = 8
    return w


def mixed_quant(K: np.ndarray, V: np.ndarray, widths: np.ndarray) -> dict:
    """K, V (B, H, T, d) with T = 64 nb; widths (B, H, nb).  Returns per block
    kc, vc (B, H, nb, 64, d) uint8; k_lo, k_sc (B, H, nb, 2, d); v_lo, v_sc (B, H, nb, 64, d/32)
    (float32 holding fp16 values); xk, xv (B, H, T, d) float32 dequantised rows."""
    B, H, T, d = K.shape
    nb = T // BLOCK
    out = {"kc": np.zeros((B, H, nb, BLOCK, d), np.uint8), "vc": np.zeros((B, H, nb, BLOCK, d), np.uint8),
           "k_lo": np.zeros((B, H, nb, 2, d), np.float32), "k_sc": np.zeros((B, H, nb, 2, d), np.float32),
           "v_lo": np.zeros((B, H, nb, BLOCK, d // GROUP), np.float32),
           "v_sc": np.zeros((B, H, nb, BLOCK, d // GROUP), np.float32),
           "xk": np.zeros((B, H, T, d), np.float32), "xv": np.zeros((B, H, T, d), np.float32)}
    for b in WIDTHS:
        sel = widths == b                                                      # (B, H, nb)
        if not sel.any():
            continue
        qk = kivi_quant(K, b, GROUP, True, 0)
        qv = kivi_quant(V, b, GROUP, False, 0)
        out["kc"][sel] = qk["codes"].reshape(B, H, nb, BLOCK, d)[sel]
        out["vc"][sel] = qv["codes"].reshape(B, H, nb, BLOCK, d)[sel]
        out["k_lo"][sel] = qk["lo"].reshape(B, H, nb, 2, d)[sel]
        out["k_sc"][sel] = qk["scale"].reshape(B, H, nb, 2, d)[sel]
        out["v_lo"][sel] = qv["lo"].reshape(B, H, nb, BLOCK, d // GROUP)[sel]
        out["v_sc"][sel] = qv["scale"].reshape(B, H, nb, BLOCK, d // GROUP)[sel]
        tsel = np.repeat(sel, BLOCK, axis=-1)                                  # (B, H, T)
        out["xk"][tsel] = qk["xhat"][tsel]
        out["xv"][tsel] = qv["xhat"][tsel]
    return out


def dequant_blocks(kc, k_lo, k_sc, vc, v_lo, v_sc):
    """Per-block codes and metadata (mixed_quant's shapes) -> xk, xv (B, H, T, d) float32,
    code * scale + lo with two roundings (STRATA_KV.py:853)."""
    B, H, nb, _, d = kc.shape
    kk = (kc.astype(np.float32).reshape(B, H, nb, 2, GROUP, d) * k_sc[:, :, :, :, None, :]) + k_lo[:, :, :, :, None, :]
    vv = (vc.astype(np.float32).reshape(B, H, nb, BLOCK, d // GROUP, GROUP) * v_sc[..., None]) + v_lo[..., None]
    return kk.reshape(B, H, nb * BLOCK, d), vv.reshape(B, H, nb * BLOCK, d)


def mixed_decode(q: np.ndarray, scaling: float, xk: np.ndarray, xv: np.ndarray, k_exact=None, v_exact=None):
    """Attention of q (B, Hq, Tq, d) over the coded rows xk, xv (B, Hkv, T, d) and exact rows
    (B, Hkv, e, d), all visible.  Returns (B, Tq, Hq, d) float64."""
    B, Hq, Tq, d = q.shape
    Hkv, n = xk.shape[1], xk.shape[2]
    tok = {"k": xk, "v": xv, "b": np.zeros((B, Hkv, n)), "tau": np.full(n, -1)}
    if k_exact is None:
        k_exact = np.zeros((B, Hkv, 0, d))
        v_exact = np.zeros((B, Hkv, 0, d))
    e = k_exact.shape[2]
    return chunked_attention(q, scaling, np.zeros(Tq, int), k_exact, v_exact, np.zeros(e, int),
                             np.full(e, 1 << 40), tok)
