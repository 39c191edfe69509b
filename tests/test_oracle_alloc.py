"""Pins of the STRATA allocation oracle (oracle/strata_alloc.py).

* Everett (1963): the allocation the search returns minimises D + mu bits for its multiplier, so
  no allocation using at most its bits has a smaller distortion.  Checked by enumerating every
  (cap, per-position option) pair on tiny inputs; a planted sign error in the evaluation fails it.
* The reference's own allocator checks (STRATA_KV.py:1945-1961): the bits stay within the budget,
  the distortion does not rise with the budget, and a budget for every token in full precision
  makes every position exact.
* Bits are non-increasing in the multiplier (the bracketing relies on it, STRATA_KV.py:1320-1323).
* Order and head sum: a permutation per head, keys non-increasing, ties by index; Dsort's rows
  sum to the heads' totals.
"""
import itertools

import numpy as np
import pytest

import oracle.strata_alloc as oa


def _brute_best(Ds, cost, fixed, max_bits):
    """Smallest distortion over every (cap c, options with levels <= c) using <= max_bits."""
    n, nlev = Ds.shape
    L = nlev - 2
    best = np.inf
    for c in range(L + 1):
        opts = [0, nlev - 1] + list(range(1, c + 1))
        for ch in itertools.product(opts, repeat=n):
            ch = np.array(ch)
            bits = cost[ch].sum() + fixed[c]
            if bits <= max_bits:
                best = min(best, float(Ds[np.arange(n), ch].astype(np.float64).sum()))
    return best


def _tiny(seed, n, nlev):
    rng = np.random.default_rng(seed)
    scale = np.concatenate([[1.0], 0.3 ** np.arange(1, nlev - 1), [0.0]])
    Ds = (rng.random((n, 1)) * scale * rng.uniform(0.5, 2.0, (n, nlev))).astype(np.float32)
    Ds[:, -1] = 0.0
    tok = np.concatenate([[0.0], 544.0 * 2.0 ** np.arange(nlev - 2), [4096.0]])
    fixed = np.array([160.0] + [4256.0] * (nlev - 2))
    return Ds, tok, fixed


@pytest.mark.parametrize("seed", range(12))
def test_everett_brute_force(seed):
    n, nlev = 4 + seed % 2, 3 + seed % 3
    Ds, cost, fixed = _tiny(seed, n, nlev)
    rng = np.random.default_rng(100 + seed)
    budget = float(fixed[0] + rng.uniform(0.1, 0.9) * n * cost[-1])
    al = oa.head_sync_allocate(Ds, cost, fixed, budget)
    got = float(Ds[np.arange(n), al["choice"]].astype(np.float64).sum())
    assert al["bits"] <= budget
    assert got <= _brute_best(Ds, cost, fixed, al["bits"]) * (1 + 1e-12) + 1e-15


def test_planted_sign_error_fails_brute_force():
    def wrong(Dsort, cost, fixed, log_mu):                       # mu cost enters Q with the wrong sign
        _, choice, c = oa.evaluate(Dsort, -np.asarray(cost), fixed, log_mu)
        return np.asarray(cost)[choice].sum(1) + np.asarray(fixed)[c], choice, c

    failures = 0
    for seed in range(12):
        n, nlev = 4 + seed % 2, 3 + seed % 3
        Ds, cost, fixed = _tiny(seed, n, nlev)
        budget = float(fixed[0] + 0.5 * n * cost[-1])
        al = oa.head_sync_allocate(Ds, cost, fixed, budget, _evaluate=wrong)
        got = float(Ds[np.arange(n), al["choice"]].astype(np.float64).sum())
        failures += al["bits"] > budget or got > _brute_best(Ds, cost, fixed, al["bits"]) * (1 + 1e-9)
    assert failures > 0


def test_reference_allocator_checks():
    rng = np.random.default_rng(7)
    Dl = (rng.random((300, 1)) * np.array([1.0, 0.12, 0.012, 1e-4, 0.0])).astype(np.float32)
    cost = np.array([0.0, 544.0, 1056.0, 2080.0, 4096.0])
    fixed = np.array([160.0, 4256.0, 4256.0, 4256.0])
    prev = -1.0
    for budget in (5e3, 3e4, 1e5, 3e5, 2e6):
        al = oa.head_sync_allocate(Dl, cost, fixed, budget)
        assert al["bits"] <= budget + 1e-3
        dist = float(Dl[np.arange(300), al["choice"]].astype(np.float64).sum())
        assert not (prev >= 0 and dist > prev + 1e-6)
        prev = dist
    assert (al["choice"] == 4).all()


def test_bits_non_increasing_in_mu():
    rng = np.random.default_rng(3)
    Ds = (rng.random((200, 1)) * np.array([1.0, 0.1, 0.01, 0.0]) * rng.uniform(0.5, 2, (200, 4))).astype(np.float32)
    cost = np.array([0.0, 1100.0, 2100.0, 4096.0]) * 8
    fixed = np.array([128.0, 32896.0, 32896.0])
    bits = oa.evaluate(Ds, cost, fixed, np.linspace(-80, 25, 400))[0]
    assert (np.diff(bits) <= 1e-6).all()


def test_order_and_head_sum():
    rng = np.random.default_rng(5)
    D = rng.random((3, 50, 5)).astype(np.float32)
    D[1, 10:20, :2] = 0.25                                       # ties: ascending index
    order = oa.importance_order(D)
    for h in range(3):
        assert sorted(order[h].tolist()) == list(range(50))
        key = D[h, order[h], 0] + D[h, order[h], 1]
        assert (np.diff(key) <= 0).all()
        tied = order[h][key == np.float32(0.5)]
        assert (np.diff(tied) > 0).all()
    Ds = oa.head_sum(D, order)
    np.testing.assert_allclose(Ds.sum(0), D.sum((0, 1)), rtol=1e-5)


def test_sanitize_and_all_drop():
    D = np.ones((2, 4, 4), np.float32)
    D[0, 0, 0], D[1, 1, 1], D[0, 2, 2] = np.inf, np.nan, -np.inf
    S = oa.sanitize(D)
    assert S[0, 0, 0] == np.float32(1e30) and S[1, 1, 1] == 0 and S[0, 2, 2] == np.finfo(np.float32).min
    cost, fixed, budget, hist, _ = oa.layer_costs((2, 4, 8), 128, 2, 100, 0.01, 4, 68)
    assert budget < hist
    out = oa.allocate(np.ones((2, 32, 5), np.float32), cost, fixed, budget, search=False)
    assert (out["choice"] == 0).all() and out["counts"].tolist() == [32, 0, 0, 0, 0]


def test_distortion_table_equals_reconstruction_error():
    """e^T (R S R^T) e in the code basis == (x_hat - x)^T S (x_hat - x) for x_hat = mu + y_hat R
    (the reader's reconstruction, STRATA_KV.py:1597-1609); a transposed rotation breaks it."""
    import oracle.strata as os_
    rng = np.random.default_rng(9)
    Hkv, n, d, bits = 2, 40, 128, (2, 4, 8)
    Xk = rng.normal(size=(Hkv, n, d)).astype(np.float32)
    Xv = rng.normal(size=(Hkv, n, d)).astype(np.float32)
    G = rng.normal(size=(2, Hkv, d, d))
    S, Mbar = G[0] @ G[0].transpose(0, 2, 1) / d, G[1] @ G[1].transpose(0, 2, 1) / d
    A, W, DD = rng.random((3, Hkv, n))
    signs = os_.rotation_signs(d)
    R = os_.rotation_matrix(d).astype(np.float64)
    (mk, Yk), (mv, Yv) = os_.strata_center_rotate(Xk, signs), os_.strata_center_rotate(Xv, signs)
    D = oa.distortion_table(Yk, Yv, S, Mbar, A, W, DD, bits)
    assert D.shape == (Hkv, n, len(bits) + 2) and (D[..., -1] == 0).all() and (D[..., 0] == DD).all()
    for i, b in enumerate(bits):
        step = os_.uniform_step(b)[0]
        want = 0.0
        for Y, mu, X, M, wgt in ((Yk, mk, Xk, S, A), (Yv, mv, Xv, Mbar, W)):
            xh = mu[:, None, :].astype(np.float64) + os_.strata_quantize(Y, b, step)[2].astype(np.float64) @ R
            xr = mu[:, None, :].astype(np.float64) + Y.astype(np.float64) @ R      # == X up to fp32 rounding
            e = xh - xr
            want = want + wgt * np.einsum("hnd,hde,hne->hn", e, M, e)
        np.testing.assert_allclose(D[..., 1 + i], want, rtol=1e-9)
        bad = 0.0
        for Y, M, wgt in ((Yk, S, A), (Yv, Mbar, W)):
            e = os_.strata_quantize(Y, b, step)[2].astype(np.float64) - Y
            bad = bad + wgt * np.einsum("hnd,hde,hne->hn", e, R.T @ M @ R, e)
        assert np.abs(bad - want).max() > 1e-3 * np.abs(want).max()
