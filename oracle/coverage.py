"""STRATA coverage statistics (numpy float64 restatement).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Reference (STRATA_KV.py):
  * ``coverage_groups(H, cfg)``  1206-1222: one group per STRATA_SEGMENT context positions starting at
    N_SINK + STRATA_LOCAL (min(len, STRATA_QUERIES) positions drawn without replacement by
    np.random.default_rng([42, crc32("cover_group"), crc32(str(H)), crc32(str(start))]), sorted),
    then the window group (the last W_OBS positions, always last); empty groups dropped.
  * ``coverage_stats``           1225-1298: per group, the exact softmax of every (query head, query)
    row over the keys [0, max position] (causal), its output o; for the coded tokens j in
    [rs, min(re, max position + 1)) read at distance >= local (1 for the window group, STRATA_LOCAL
    otherwise): pR = p_j, u = ||v_j - o||^2_{M_a}, the drop term (pR / max(1 - pR, 1e-6))^2 u, the
    key term pR^2 u and the read mass pR^2, each averaged over the group's queries; the group's
    drop total N normalises all its terms (N summed over every head and token); averaged over the
    live groups; S = sum of alpha q q^T (alpha = the row's key-term mass) normalised by sum_j A_j;
    Mbar = read-weighted mean of the head metrics (plain mean where nothing is read); every output
    gets STRATA_FLOOR x its mean added.

``group_terms`` returns one group's unnormalised terms so that they can be checked against
brute-force perturbations: Prop. 1 (removing token j from the softmax moves the output by exactly
-p_j / (1 - p_j) (v_j - o), so ||delta o||^2_M equals the drop term; STRATA_KV.py:1200-1204,
1931-1944), the exact single-entry value perturbation (delta o = p_j e) and a finite difference of
the first-order key term.  ``coverage_groups`` is pinned by golden draws of the reference.
"""
from __future__ import annotations

import zlib
from dataclasses import dataclass
from typing import Dict, List

import numpy as np


@dataclass(frozen=True)
class CoverageParams:
    """The Config fields coverage_stats reads (the reference's defaults)."""
    N_SINK: int = 4
    STRATA_LOCAL: int = 64
    W_OBS: int = 32
    STRATA_SEGMENT: int = 512
    STRATA_QUERIES: int = 16
    STRATA_FLOOR: float = 1e-3


def _rng(*keys) -> np.random.Generator:
    return np.random.default_rng([42] + [zlib.crc32(str(k).encode()) for k in keys])


def coverage_groups(H: int, c: CoverageParams) -> List[np.ndarray]:
    """STRATA_KV.py:1206-1222."""
    lo = c.N_SINK + c.STRATA_LOCAL
    win = max(lo, H - c.W_OBS)
    groups = []
    for s in range(lo, win, c.STRATA_SEGMENT):
        seg = np.arange(s, min(s + c.STRATA_SEGMENT, win))
        n = min(len(seg), c.STRATA_QUERIES)
        groups.append(np.sort(_rng("cover_group", H, s).choice(seg, n, replace=False)))
    groups.append(np.arange(win, H))
    return [g for g in groups if len(g)]


def group_terms(qg: np.ndarray, pos: np.ndarray, k: np.ndarray, v: np.ndarray, M: np.ndarray, rs: int, re: int,
                local: int) -> Dict:
    """One group's terms (STRATA_KV.py:1253-1283), float64.  qg (Hkv, rep, nq, d): the SCALED queries
    (scaling * q) of the group's positions pos (nq,); k, v (Hkv, T, d); M (Hkv, rep, d, d).
    Returns dd (Hkv, nt) = sum over rows of the drop term / nq, a (Hkv, rep, nq, nt) the key terms
    pR^2 u, wv (Hkv, rep, nt) = sum over queries of pR^2 / nq, alpha (Hkv, rep, nq) = sum_j a / nq,
    N = dd.sum(), nt, and p, o, u2 (for the checks)."""
    Hkv, rep, nq, d = qg.shape
    mmax = int(pos.max()) + 1
    te = min(re, mmax)
    nt = max(0, te - rs)
    Sc = np.einsum("hrqd,hmd->hrqm", qg, k[:, :mmax])
    Sc = np.where(np.arange(mmax)[None, None, None, :] > pos[None, None, :, None], -np.inf, Sc)
    Sc = Sc - Sc.max(-1, keepdims=True)
    p = np.exp(Sc)
    p = p / p.sum(-1, keepdims=True)
    o = np.einsum("hrqm,hmd->hrqd", p, v[:, :mmax])
    out = {"p": p, "o": o, "nt": nt, "mmax": mmax}
    if nt == 0:
        out.update(dd=np.zeros((Hkv, 0)), a=np.zeros((Hkv, rep, nq, 0)), wv=np.zeros((Hkv, rep, 0)),
                   alpha=np.zeros((Hkv, rep, nq)), N=0.0, u2=np.zeros((Hkv, rep, nq, 0)))
        return out
    far = np.arange(rs, te)[None, :] <= (pos[:, None] - local)                  # (nq, nt)
    pR = p[..., rs:te] * far
    VR = v[:, rs:te]
    vMv = np.einsum("hjd,hrde,hje->hrj", VR, M, VR)
    oM = np.einsum("hrqd,hrde->hrqe", o, M)
    u2 = np.maximum(vMv[:, :, None, :] - 2 * np.einsum("hrqe,hje->hrqj", oM, VR) + (oM * o).sum(-1)[..., None], 0.0)
    dd = ((pR / np.maximum(1 - pR, 1e-6)) ** 2 * u2).sum((1, 2)) / nq
    a = pR ** 2 * u2
    out.update(dd=dd, a=a, wv=(pR ** 2).sum(2) / nq, alpha=a.sum(-1) / nq, N=float(dd.sum()), u2=u2)
    return out


def coverage_stats(q: np.ndarray, qpos: np.ndarray, k: np.ndarray, v: np.ndarray, scaling: float, H: int, rs: int,
                   re: int, M: np.ndarray, c: CoverageParams, window_only: bool = False) -> Dict:
    """STRATA_KV.py:1225-1298 in float64.  q (Hq, nrows, d): the query rows kept at positions qpos
    (nrows,) (the reference's QRows); k, v (Hkv, T, d); M (Hq, d, d) per query head.  Returns A, W,
    DD (Hkv, n), S, Mbar (Hkv, d, d), groups (n = re - rs)."""
    Hkv, _, d = k.shape
    Hq = q.shape[0]
    rep = Hq // Hkv
    n = re - rs
    groups = coverage_groups(H, c)
    if window_only:
        groups = groups[-1:]
    index = {int(p_): i for i, p_ in enumerate(qpos)}
    Mg = M.reshape(Hkv, rep, d, d).astype(np.float64)
    k, v = k.astype(np.float64), v.astype(np.float64)
    A = np.zeros((Hkv, n))
    DD = np.zeros((Hkv, n))
    WVa = np.zeros((Hkv, rep, n))
    S = np.zeros((Hkv, d, d))
    live = 0.0
    for gi, P in enumerate(groups):
        if min(re, int(P.max()) + 1) <= rs:
            continue
        rows = np.array([index[int(p_)] for p_ in P])
        qg = (q[:, rows].astype(np.float64) * scaling).reshape(Hkv, rep, len(P), d)
        local = 1 if gi == len(groups) - 1 else c.STRATA_LOCAL
        t = group_terms(qg, np.asarray(P), k, v, Mg, rs, re, local)
        nt = t["nt"]
        wgt = 1.0 / t["N"] if t["N"] > 0 else 0.0
        A[:, :nt] += t["a"].sum((1, 2)) / len(P) * wgt
        DD[:, :nt] += t["dd"] * wgt
        WVa[:, :, :nt] += t["wv"] * wgt
        S += np.einsum("hrq,hrqd,hrqe->hde", t["alpha"], qg, qg) * wgt
        live += float(t["N"] > 0)
    live = max(live, 1.0)
    A, DD, WVa, S = A / live, DD / live, WVa / live, S / live
    S = S / np.maximum(A.sum(-1), 1e-30)[:, None, None]
    omega = WVa.sum(-1)
    Mbar = np.einsum("hr,hrde->hde", omega, Mg) / np.maximum(omega.sum(-1), 1e-30)[:, None, None]
    Mbar = np.where(omega.sum(-1)[:, None, None] > 0, Mbar, Mg.mean(1))
    eta = c.STRATA_FLOOR
    W = WVa.sum(1)
    return {"A": A + eta * A.mean(), "W": W + eta * W.mean(), "DD": DD + eta * DD.mean(), "S": S, "Mbar": Mbar,
            "groups": groups}
