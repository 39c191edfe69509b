"""QUASAR compressed-domain decode (numpy restatement).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Reference:
  * ``lloyd_max_gaussian``  STRATA_KV.py:1082-1098 (Lloyd iterations on a fine grid of N(0, 1))
  * ``stage_codebooks``     QUASAR_KV.py:1143-1169 (embedded residual Lloyd-Max levels)
  * ``embedded_quantize``   QUASAR_KV.py:1172-1182 (codes of every stage by bucketize)
  * ``QuasarState.attend``  QUASAR_KV.py:1945-1968 with the reference (torch) path of
    ``coded_scores`` / ``coded_values`` (1921-1943): per step of a side, the query's coefficients
    of the step's band dotted with the levels of the packed codes of the tokens owning the step
    (a prefix of the coded tokens), scaled per token by rho and offset by q . mu; one softmax over
    exact rows and coded tokens; the coded tokens' weighted levels lifted back by T_V and mu_V.
  * ``QuasarState.__init__`` step table (1883-1898): per side, in step order, [byte offset in the
    side's flat code buffer, n_s, bytes per row, first coefficient a, width w, bits, level offset].

Pinning (tests/test_oracle_quasar.py, tests/test_golden.py):
  * golden vectors written by the reference's own functions (tests/golden/quasar_codebooks.npz):
    ``lloyd_max_gaussian`` levels at 1-4 bits, the stage codebooks of (2, 2, 4), (4, 4) and (8,)
    and ``embedded_quantize`` codes of seeded coefficients, all bit-equal.
  * ``lloyd_max_gaussian`` against Max's (1960) table of the Gaussian Lloyd-Max MSE at 1-4 bits
    (0.3634 / 0.1175 / 0.03454 / 0.009497, the values STRATA_KV.py:1085-1087 quotes).
  * ``stage_codebooks`` against the MSE the reference states for the (2, 2, 4) embedded code
    after each stage (0.1175 / 0.0196 / 0.00056, QUASAR_KV.py:1151-1152), and the symmetry of the
    levels of a symmetric distribution.
  * ``attend`` against plain softmax attention over the exact rows plus the reconstructed coded
    tokens (mu + (rho u_hat) T^T, QuasarMethod.reconstruct 1715-1733): the identity the
    reference's decode is built on (the coded-domain decode never reconstructs a row, 1857-1862).
    The reconstruction path shares no step-loop code with the coded path.
"""
from __future__ import annotations

from functools import lru_cache
from typing import Dict, List, Sequence

import numpy as np
from scipy import stats

from .kivi import unpack_rows_lut


@lru_cache(maxsize=None)
def lloyd_max_gaussian(bits: int) -> np.ndarray:
    """Lloyd-Max levels of N(0, 1) with 2^bits cells (STRATA_KV.py:1082-1098): 500 Lloyd
    iterations on a weighted grid of 360001 points over [-9, 9], started at the normal quantiles."""
    n = 2 ** bits
    x = np.linspace(-9.0, 9.0, 360001)
    w = np.exp(-0.5 * x * x)
    w /= w.sum()
    c = stats.norm.ppf((np.arange(n) + 0.5) / n)
    for _ in range(500):
        cell = np.searchsorted((c[1:] + c[:-1]) / 2, x)
        mass = np.bincount(cell, w, n)
        c = np.bincount(cell, w * x, n) / np.maximum(mass, 1e-300)
    return c.astype(np.float32)


def lloyd_max_mse(bits: int) -> float:
    """MSE of lloyd_max_gaussian(bits) on N(0, 1), on the same grid."""
    c = lloyd_max_gaussian(bits).astype(np.float64)
    x = np.linspace(-9.0, 9.0, 360001)
    w = np.exp(-0.5 * x * x)
    w /= w.sum()
    cell = np.searchsorted((c[1:] + c[:-1]) / 2, x)
    return float((w * (x - c[cell]) ** 2).sum())


def _quantile_sample() -> np.ndarray:
    return stats.norm.ppf((np.arange(200000) + 0.5) / 200000)


@lru_cache(maxsize=None)
def stage_codebooks(stage_bits: Sequence[int]) -> List[np.ndarray]:
    """Levels of each stage of the embedded code (QUASAR_KV.py:1143-1169): stage 0 Lloyd-Max at
    stage_bits[0]; stage t > 0 the Lloyd code (150 iterations from the quantiles) of the residual
    of a deterministic quantile sample of N(0, 1) after the earlier stages."""
    x = _quantile_sample()
    cur, out = np.zeros_like(x), []
    for t, b in enumerate(stage_bits):
        r = x - cur
        if t == 0:
            c = lloyd_max_gaussian(b).astype(np.float64)
        else:
            n = 2 ** b
            c = np.quantile(r, (np.arange(n) + 0.5) / n)
            for _ in range(150):
                cell = np.searchsorted((c[1:] + c[:-1]) / 2, r)
                c = np.bincount(cell, r, n) / np.maximum(np.bincount(cell, None, n), 1)
        cur = cur + c[np.searchsorted((c[1:] + c[:-1]) / 2, r)]
        out.append(c.astype(np.float32))
    return out


def embedded_mse(stage_bits: Sequence[int]) -> List[float]:
    """MSE of the quantile sample after each stage (the figures of QUASAR_KV.py:1151-1152)."""
    x = _quantile_sample()
    cur, out = np.zeros_like(x), []
    for c in stage_codebooks(tuple(stage_bits)):
        c = c.astype(np.float64)
        cur = cur + c[np.searchsorted((c[1:] + c[:-1]) / 2, x - cur)]
        out.append(float(((x - cur) ** 2).mean()))
    return out


def embedded_quantize(u: np.ndarray, stage_bits: Sequence[int]):
    """Codes (uint8) of every stage (QUASAR_KV.py:1172-1182)."""
    codes, cur = [], np.zeros_like(u, dtype=np.float32)
    for cb in stage_codebooks(tuple(stage_bits)):
        c = np.searchsorted((cb[1:] + cb[:-1]) / 2, u - cur, side="left")
        cur = cur + cb[c]
        codes.append(c.astype(np.uint8))
    return codes


def _deq(step: Dict, stage_bits: Sequence[int]) -> np.ndarray:
    """(Hkv, n_s, w) levels of a step's packed rows (QuasarState._deq, 1915-1918)."""
    b = stage_bits[step["stage"]]
    levels = stage_codebooks(tuple(stage_bits))[step["stage"]]
    return unpack_rows_lut(np.asarray(step["codes"]), b, levels).astype(np.float64)


def coded_scores(qt: np.ndarray, packed: Dict, stage_bits: Sequence[int]) -> np.ndarray:
    """QuasarState.coded_scores' torch path (QUASAR_KV.py:1920-1929) in float64: qt (..., Hkv, rows, R)
    -> (..., Hkv, rows, n_c), per key-side step the band of qt dotted with the levels of the tokens
    owning the step."""
    sc = np.zeros(qt.shape[:-1] + (int(packed["n_c"]),))
    for st in packed["steps"]:
        if st["side"] == 0:
            sc[..., :st["n"]] += np.einsum("...hrw,hjw->...hrj", qt[..., st["a"]:st["b"]], _deq(st, stage_bits))
    return sc


def coded_values(pv: np.ndarray, packed: Dict, stage_bits: Sequence[int], R: int) -> np.ndarray:
    """QuasarState.coded_values' torch path (QUASAR_KV.py:1931-1941) in float64: pv (..., Hkv, rows, n_c)
    -> (..., Hkv, rows, R), per value-side step the tokens' weights times their levels, into the band."""
    acc = np.zeros(pv.shape[:-1] + (R,))
    for st in packed["steps"]:
        if st["side"] == 1:
            acc[..., st["a"]:st["b"]] += np.einsum("...hrj,hjw->...hrw", pv[..., :st["n"]], _deq(st, stage_bits))
    return acc


def attend(q: np.ndarray, scaling: float, qpos: np.ndarray, K: np.ndarray, V: np.ndarray, n0: int, H: int,
           packed: Dict, stage_bits: Sequence[int]) -> np.ndarray:
    """QuasarState.attend (QUASAR_KV.py:1945-1968) in float64 for B = 1.

    q (1, Hq, Tq, d); K, V (1, Hkv, n, d) exact rows (the first n0 from the context, later rows
    appended at positions H, H + 1, ...); packed: steps [{side, a, b, stage, n, codes (Hkv, n_s,
    bytes)}], n_c, rho_k / rho_v (Hkv, n_c), T_k / T_v (Hkv, d, R), mu_k / mu_v (Hkv, d).
    Returns (1, Tq, Hq, d)."""
    B, Hq, Tq, d = q.shape
    Hkv, n = K.shape[1], K.shape[2]
    rep = Hq // Hkv
    qg = q.astype(np.float64).reshape(B, Hkv, rep * Tq, d)
    Kf, Vf = K.astype(np.float64), V.astype(np.float64)
    s_ex = np.einsum("bhrd,bhnd->bhrn", qg, Kf) * scaling
    if n > n0:
        row_pos = H + np.arange(n - n0)
        bad = row_pos[None, :] > np.asarray(qpos)[:, None]                      # (Tq, n - n0)
        s_ex[..., n0:] = np.where(np.tile(bad, (rep, 1))[None, None], -np.inf, s_ex[..., n0:])
    n_c = int(packed.get("n_c", 0))
    if n_c > 0:
        Tk = np.asarray(packed["T_k"], dtype=np.float64)
        qt = np.einsum("bhrd,hdk->bhrk", qg, Tk)
        sc = coded_scores(qt, packed, stage_bits)
        rho_k = np.asarray(packed["rho_k"], dtype=np.float64)
        mu_k = np.asarray(packed["mu_k"], dtype=np.float64)
        sc = (sc * rho_k[None, :, None, :] + np.einsum("bhrd,hd->bhr", qg, mu_k)[..., None]) * scaling
        s_all = np.concatenate([s_ex, sc], -1)
    else:
        s_all = s_ex
    m = s_all.max(-1, keepdims=True)
    e = np.exp(s_all - m)
    att = e / e.sum(-1, keepdims=True)
    o = np.einsum("bhrn,bhnd->bhrd", att[..., :n], Vf)
    if n_c > 0:
        pc = att[..., n:]
        rho_v = np.asarray(packed["rho_v"], dtype=np.float64)
        Tv = np.asarray(packed["T_v"], dtype=np.float64)
        mu_v = np.asarray(packed["mu_v"], dtype=np.float64)
        pv = pc * rho_v[None, :, None, :]
        acc = coded_values(pv, packed, stage_bits, Tv.shape[-1])
        o = o + np.einsum("bhrk,hdk->bhrd", acc, Tv) + pc.sum(-1, keepdims=True) * mu_v[None, :, None, :]
    return o.reshape(B, Hq, Tq, d).transpose(0, 2, 1, 3)


def coefficients(packed: Dict, side: int, stage_bits: Sequence[int], R: int) -> np.ndarray:
    """u_hat (Hkv, n_c, R) of a side: per token, the sum of the levels of every step it owns, decoded
    code by code (shift and mask), not through the byte table."""
    n_c = int(packed["n_c"])
    Hkv = np.asarray(packed["steps"][0]["codes"]).shape[0]
    u = np.zeros((Hkv, n_c, R))
    books = stage_codebooks(tuple(stage_bits))
    for st in packed["steps"]:
        if st["side"] != side:
            continue
        b = stage_bits[st["stage"]]
        per = 8 // b
        raw = np.asarray(st["codes"]).astype(np.int64)                        # (Hkv, n_s, bytes)
        shifts = (per - 1 - np.arange(per)) * b
        codes = ((raw[..., None] >> shifts) & ((1 << b) - 1)).reshape(Hkv, st["n"], -1)
        u[:, :st["n"], st["a"]:st["b"]] += books[st["stage"]].astype(np.float64)[codes]
    return u


def reconstruct(packed: Dict, side: int, stage_bits: Sequence[int]) -> np.ndarray:
    """The coded tokens of a side as a reader of the code sees them (QuasarMethod.reconstruct,
    1715-1733): mu + (rho u_hat) T^T, u_hat (``coefficients``) decoded code by code."""
    nm = "k" if side == 0 else "v"
    T = np.asarray(packed[f"T_{nm}"], dtype=np.float64)
    u = coefficients(packed, side, stage_bits, T.shape[-1])
    rho = np.asarray(packed[f"rho_{nm}"], dtype=np.float64)
    mu = np.asarray(packed[f"mu_{nm}"], dtype=np.float64)
    return mu[:, None, :] + np.einsum("hjk,hdk->hjd", rho[..., None] * u, T)


def attend_reconstructed(q: np.ndarray, scaling: float, qpos: np.ndarray, K: np.ndarray, V: np.ndarray, n0: int,
                         H: int, packed: Dict, stage_bits: Sequence[int]) -> np.ndarray:
    """Softmax attention over the exact rows and the reconstructed coded tokens (float64)."""
    B, Hq, Tq, d = q.shape
    Hkv, n = K.shape[1], K.shape[2]
    rep = Hq // Hkv
    qg = q.astype(np.float64).reshape(B, Hkv, rep * Tq, d)
    Kall, Vall = K[0].astype(np.float64), V[0].astype(np.float64)
    if int(packed.get("n_c", 0)) > 0:
        Kall = np.concatenate([Kall, reconstruct(packed, 0, stage_bits)], 1)
        Vall = np.concatenate([Vall, reconstruct(packed, 1, stage_bits)], 1)
    s = np.einsum("hrd,hnd->hrn", qg[0], Kall) * scaling
    if n > n0:
        row_pos = H + np.arange(n - n0)
        bad = row_pos[None, :] > np.asarray(qpos)[:, None]
        s[:, :, n0:n] = np.where(np.tile(bad, (rep, 1))[None], -np.inf, s[:, :, n0:n])
    s -= s.max(-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(-1, keepdims=True)
    o = np.einsum("hrn,hnd->hrd", p, Vall)
    return o.reshape(1, Hq, Tq, d).transpose(0, 2, 1, 3)


def step_table(packed: Dict, side: int, stage_bits: Sequence[int]) -> np.ndarray:
    """QuasarState.__init__'s step table of one side (1883-1898): int32 rows [offset, n_s, bytes per
    row, a, w, bits, level offset] in step order, offsets into the concatenation of the steps'
    codes."""
    books = stage_codebooks(tuple(stage_bits))
    lvl_off = np.cumsum([0] + [len(b_) for b_ in books])[:-1]
    rows, off = [], 0
    for st in packed["steps"]:
        if st["side"] != side:
            continue
        c = np.asarray(st["codes"])
        rows.append([off, st["n"], c.shape[-1], st["a"], st["b"] - st["a"], stage_bits[st["stage"]],
                     int(lvl_off[st["stage"]])])
        off += c.size
    return np.asarray(rows, dtype=np.int32).reshape(-1, 7)
