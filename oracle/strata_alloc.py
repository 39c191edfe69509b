"""STRATA allocation: importance order, head-summed distortion table, Lagrangian search (numpy).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Reference (STRATA_KV.py):
  * ``StrataMethod.compress_layer``  1528-1581: D (Hkv, n, nb + 2) columns [drop | b_1 .. b_nb |
    exact] with NaN / inf replaced (1559, ``nan_to_num(posinf=1e30)``); order = per-head argsort
    of D[..., 0] + D[..., 1], most important first (1560); Dsort = D gathered by that order and
    summed over the heads (1561); per-position costs and the fixed bits (1562-1567); the search
    (1569, or nothing but drops when the budget does not cover the level histogram, 1567-1568);
    lev = choice sorted descending (1570), its histogram (1571), the distortion ratio (1577-1581)
  * ``head_sync_allocate``           1307-1351: for a multiplier mu every position takes the
    argmin of D + mu cost among drop / exact / the best level <= the cap c, c minimising the
    total; ``rounds`` rounds of ``grid`` log-spaced multipliers over [-80, 25] bracket the
    smallest feasible mu; the allocation at the bracket's upper end is returned.

Arithmetic fixed here (the GPU kernels compute the same, so both agree bit for bit):
  * the importance key is the float32 sum D[..., 0] + D[..., 1]; ties are broken by ascending
    token index (the reference's unstable sort leaves them open);
  * Dsort sums the heads in float32 in head order 0, 1, ..., Hkv - 1;
  * the search runs in float64: Q = D + mu * cost with the product rounded before the sum, mu =
    exp(log mu); the multipliers are lo + (hi - lo) * (k * (1 / (grid - 1))), the last one hi;
    drop wins ties against exact, the cumulative minimum over levels takes the later level on
    ties (torch.cummin), the cap the first minimal total.  The reference runs the same steps in
    float32, so its choices agree except where two options' costs differ by less than float32
    rounding.

``distortion_table`` (1543-1559) is pinned by the identity e^T (R S R^T) e = (x_hat - x)^T S
(x_hat - x) for the reconstruction x_hat = mu + y_hat R (1597-1609), checked in the original basis.

Pinning (tests/test_oracle_alloc.py): Everett's theorem by brute force on tiny inputs (no
allocation using at most the returned bits has a smaller distortion), the reference's own
allocator checks (1945-1961: feasible, distortion non-increasing in the budget, all exact when
affordable), bits non-increasing in mu, and a planted sign error failing the brute force.
"""
from __future__ import annotations

import numpy as np

_LO, _HI = -80.0, 25.0


def sanitize(D: np.ndarray) -> np.ndarray:
    """torch.nan_to_num(D, posinf=1e30) in float32 (STRATA_KV.py:1559)."""
    D = np.asarray(D, dtype=np.float32)
    return np.nan_to_num(D, nan=0.0, posinf=np.float32(1e30), neginf=np.finfo(np.float32).min)


def importance_order(D: np.ndarray) -> np.ndarray:
    """(Hkv, n) int32: per head, tokens by D[..., 0] + D[..., 1] descending, ties by index
    (STRATA_KV.py:1560)."""
    key = (D[..., 0] + D[..., 1]).astype(np.float32)
    return np.argsort(-key, axis=1, kind="stable").astype(np.int32)


def head_sum(D: np.ndarray, order: np.ndarray) -> np.ndarray:
    """(n, nlev) float32: Dsort[j] = sum over heads of D[h, order[h, j]], heads in order
    (STRATA_KV.py:1561)."""
    Hkv = D.shape[0]
    acc = D[0][order[0]].astype(np.float32)
    for h in range(1, Hkv):
        acc = (acc + D[h][order[h]]).astype(np.float32)
    return acc


def evaluate(Dsort: np.ndarray, cost: np.ndarray, fixed: np.ndarray, log_mu: np.ndarray):
    """(bits (M,), choice (M, n), cap (M,)) for the multipliers exp(log_mu) (STRATA_KV.py:1326-1341)."""
    D = np.asarray(Dsort, dtype=np.float64)
    cost = np.asarray(cost, dtype=np.float64)
    fixed = np.asarray(fixed, dtype=np.float64)
    n, nlev = D.shape
    L = nlev - 2
    mu = np.exp(np.asarray(log_mu, dtype=np.float64))
    Q = D[None] + mu[:, None, None] * cost[None, None, :]
    q0, qx = Q[..., 0], Q[..., -1]
    base = np.minimum(q0, qx)
    bidx = np.where(q0 <= qx, 0, nlev - 1)
    M = len(mu)
    if L > 0:
        cm = np.empty((M, n, L))
        cidx = np.empty((M, n, L), dtype=np.int64)
        cm[..., 0], cidx[..., 0] = Q[..., 1], 0
        for l in range(1, L):
            take = Q[..., 1 + l] <= cm[..., l - 1]                 # later level on ties
            cm[..., l] = np.where(take, Q[..., 1 + l], cm[..., l - 1])
            cidx[..., l] = np.where(take, l, cidx[..., l - 1])
        tot = np.concatenate([base.sum(1)[:, None], np.minimum(base[..., None], cm).sum(1)], 1)
        tot = tot + mu[:, None] * fixed[None, :]
        c = np.argmin(tot, axis=1)
        cc = np.maximum(c - 1, 0)
        cmc = np.take_along_axis(cm, cc[:, None, None].repeat(n, 1), 2)[..., 0]
        cic = np.take_along_axis(cidx, cc[:, None, None].repeat(n, 1), 2)[..., 0]
        use = (c > 0)[:, None] & (cmc < base)
        choice = np.where(use, cic + 1, bidx)
    else:
        c = np.zeros(M, dtype=np.int64)
        choice = bidx
    bits = cost[choice].sum(1) + fixed[c]
    return bits, choice.astype(np.int32), c.astype(np.int32)


def multipliers(lo: float, hi: float, grid: int) -> np.ndarray:
    step = 1.0 / (grid - 1)
    g = np.array([lo + (hi - lo) * (k * step) for k in range(grid)], dtype=np.float64)
    g[-1] = lo + (hi - lo) * 1.0
    return g


def head_sync_allocate(Dsort, cost, fixed, budget: float, rounds: int = 4, grid: int = 32, _evaluate=evaluate):
    """dict(choice (n,) int32, cap, bits) (STRATA_KV.py:1307-1351).  ``_evaluate`` lets a test
    plant a mistake in the per-multiplier evaluation."""
    evaluate = _evaluate
    lo, hi = _LO, _HI
    for _ in range(rounds):
        g = multipliers(lo, hi, grid)
        ok = evaluate(Dsort, cost, fixed, g)[0] <= budget
        i = int(np.argmax(ok)) if ok.any() else grid - 1
        lo, hi = g[max(i - 1, 0)], g[i]
    bits, choice, c = evaluate(Dsort, cost, fixed, np.array([hi]))
    return {"choice": choice[0], "cap": int(c[0]), "bits": float(bits[0])}


def allocate(D, cost, fixed, budget: float, rounds: int = 4, grid: int = 32, search: bool = True):
    """The device allocation's outputs: order, Dsort, choice, lev, counts, cap, bits and the
    distortion ratio sum Dsort[j, lev_j] / sum Dsort[j, 0], each clamped to 1e29 and summed in
    float64 (STRATA_KV.py:1560-1581; ``search`` False = the all-drop branch, 1567-1568)."""
    D = sanitize(D)
    order = importance_order(D)
    Ds = head_sum(D, order)
    n, nlev = Ds.shape
    if search:
        al = head_sync_allocate(Ds, cost, fixed, budget, rounds, grid)
    else:
        al = {"choice": np.zeros(n, np.int32), "cap": 0, "bits": float(np.asarray(fixed, np.float64)[0])}
    counts = np.bincount(al["choice"], minlength=nlev).astype(np.int32)
    lev = np.sort(al["choice"])[::-1].astype(np.int32)
    dfin = np.minimum(np.take_along_axis(Ds, lev[:, None].astype(np.int64), 1)[:, 0].astype(np.float64), 1e29)
    dref = np.minimum(Ds[:, 0].astype(np.float64), 1e29)
    return {"order": order, "dsort": Ds, "choice": al["choice"], "lev": lev, "counts": counts,
            "cap": al["cap"], "bits": al["bits"], "distortion": float(dfin.sum() / max(dref.sum(), 1e-30))}


def layer_costs(bits, d: int, Hkv: int, H: int, keep: float, rs: int, re: int):
    """cost (nb + 2,), fixed (nb + 1,), budget and the histogram bits of one layer, in float64
    as the host computes them (STRATA_KV.py:1562-1567)."""
    nb = len(bits)
    cost_tok = np.array([0.0] + [2.0 * (b * d + 16) for b in bits] + [2.0 * d * 16])
    hist_bits = (nb + 2) * 32.0
    fixed = np.where(np.arange(nb + 1) > 0, Hkv * 2 * d * 16.0, 0.0) + hist_bits
    budget = keep * H * Hkv * 2 * d * 16.0 - (rs + (H - re)) * Hkv * 2 * d * 16.0
    return cost_tok * Hkv, fixed, float(budget), hist_bits, cost_tok


def distortion_table(Yk, Yv, S, Mbar, A, W, DD, bits, key: str = "strata"):
    """D (Hkv, n, nb + 2) float64 = [DD | A e_K^T Mt_K e_K + W e_V^T Mt_V e_V per width | 0] with
    Mt = R S R^T, R Mbar R^T and e = y_hat - y of strata_quantize (STRATA_KV.py:1543-1559)."""
    from oracle.strata import rotation_matrix, strata_quantize, uniform_step
    d = Yk.shape[-1]
    R = rotation_matrix(d, key).astype(np.float64)
    cols = [np.asarray(DD, np.float64)]
    for b in bits:
        errs = []
        for Y, M in ((Yk, S), (Yv, Mbar)):
            Mt = R @ np.asarray(M, np.float64) @ R.T
            e = strata_quantize(Y, b, uniform_step(b)[0])[2].astype(np.float64) - np.asarray(Y, np.float64)
            errs.append(np.einsum("hnd,hde,hne->hn", e, Mt, e))
        cols.append(np.asarray(A, np.float64) * errs[0] + np.asarray(W, np.float64) * errs[1])
    cols.append(np.zeros_like(cols[0]))
    return np.stack(cols, -1)
