"""Pins of oracle/coverage.py (STRATA_KV.py:1206-1298) by independent formulations.

* coverage_groups: equal to the reference's own draws (tests/golden/coverage_groups.npz) for four
  contexts under the default Config and the reference's test config (1964).
* Drop term (Prop. 1, STRATA_KV.py:1200-1204; the reference checks it to 1e-9 at 1931-1944): for
  every row and token, removing the token from the softmax moves the output by a vector whose
  squared M-norm equals (p / (1 - p))^2 ||v - o||^2_M -- computed here by actually recomputing the
  softmax without the token.
* Value term: perturbing v_j by e moves the output by exactly p_j e.
* Key term: perturbing k_j by eps e moves the output by eps p_j (q.e)(v_j - o) to first order
  (finite difference, relative 1e-4).
* Aggregation: sum_j A_j e^T S e (without the floor) equals the live-averaged, group-weighted
  total of a (q.e)^2 over rows and tokens (the decoupling S is built for); Mbar is the
  read-weighted mean of the head metrics; a planted sign error in u breaks the drop identity.
"""
from pathlib import Path

import numpy as np
import pytest

import oracle.coverage as oc

GOLD = Path(__file__).resolve().parent / "golden" / "coverage_groups.npz"


def test_groups_match_reference_draws():
    z = np.load(GOLD)
    for name in ("default", "test"):
        N_SINK, LOCAL, W_OBS, SEG, QUER = (int(x) for x in z[f"{name}_params"])
        c = oc.CoverageParams(N_SINK=N_SINK, STRATA_LOCAL=LOCAL, W_OBS=W_OBS, STRATA_SEGMENT=SEG, STRATA_QUERIES=QUER)
        for H in (200, 700, 1500, 4100):
            gs = oc.coverage_groups(H, c)
            np.testing.assert_array_equal([len(g) for g in gs], z[f"{name}_{H}_lengths"])
            np.testing.assert_array_equal(np.concatenate(gs), z[f"{name}_{H}_positions"])


def _case(seed, Hkv=2, rep=2, d=8, T=60):
    rng = np.random.default_rng(seed)
    k = rng.standard_normal((Hkv, T, d)) * 1.5
    v = rng.standard_normal((Hkv, T, d))
    qg = rng.standard_normal((Hkv, rep, 3, d)) * 0.7
    W = rng.standard_normal((Hkv * rep, 16, d))
    M = np.einsum("aie,aif->aef", W, W).reshape(Hkv, rep, d, d) / 16
    pos = np.array([30, 44, T - 1])
    return qg, pos, k, v, M


def _attend(qv, k, v, upto):
    s = k[:upto] @ qv
    s = s - s.max()
    p = np.exp(s)
    p /= p.sum()
    return p @ v[:upto], p


def test_drop_term_is_prop1_exact():
    qg, pos, k, v, M = _case(1)
    rs, re = 2, 50
    t = oc.group_terms(qg, pos, k, v, M, rs, re, local=1)
    Hkv, rep, nq, d = qg.shape
    for h in range(Hkv):
        for j in range(rs, t["nt"] + rs):
            brute = 0.0
            for r in range(rep):
                for qi, P in enumerate(pos):
                    if j > P - 1:
                        continue                                      # read at distance < local: not counted
                    o, _ = _attend(qg[h, r, qi], k[h], v[h], P + 1)
                    keep = np.r_[0:j, j + 1:P + 1]
                    o2, _ = _attend(qg[h, r, qi], k[h][keep], v[h][keep], len(keep))
                    dlt = o2 - o
                    brute += dlt @ M[h, r] @ dlt
            assert abs(t["dd"][h, j - rs] - brute / nq) <= 1e-9 * max(1.0, brute), (h, j)


def test_value_and_key_terms():
    qg, pos, k, v, M = _case(2)
    rs, re = 0, 59
    t = oc.group_terms(qg, pos, k, v, M, rs, re, local=1)
    rng = np.random.default_rng(3)
    e = rng.standard_normal(k.shape[-1])
    h, r, qi, j = 1, 0, 2, 17
    P = pos[qi]
    o, p = _attend(qg[h, r, qi], k[h], v[h], P + 1)
    v2 = v[h].copy()
    v2[j] += e
    o2, _ = _attend(qg[h, r, qi], k[h], v2, P + 1)
    np.testing.assert_allclose(o2 - o, p[j] * e, rtol=1e-12, atol=1e-14)         # exact single entry
    eps = 1e-5
    k2 = k[h].copy()
    k2[j] += eps * e
    o3, _ = _attend(qg[h, r, qi], k2, v[h], P + 1)
    dlt = o3 - o
    fd = (dlt @ M[h, r] @ dlt) / eps ** 2
    first = t["a"][h, r, qi, j - rs] * (qg[h, r, qi] @ e) ** 2
    assert abs(fd - first) <= 1e-4 * abs(first)


def test_aggregation_decoupling_and_mbar():
    rng = np.random.default_rng(5)
    Hkv, rep, d, T = 2, 2, 8, 300
    c = oc.CoverageParams(N_SINK=2, STRATA_LOCAL=8, W_OBS=6, STRATA_SEGMENT=64, STRATA_QUERIES=5, STRATA_FLOOR=0.0)
    k = rng.standard_normal((Hkv, T, d))
    v = rng.standard_normal((Hkv, T, d))
    qpos = np.arange(T)
    q = rng.standard_normal((Hkv * rep, T, d))
    W = rng.standard_normal((Hkv * rep, 12, d))
    M = np.einsum("aie,aif->aef", W, W) / 12
    H, rs, re = T, c.N_SINK, T - 10
    st = oc.coverage_stats(q, qpos, k, v, d ** -0.5, H, rs, re, M, c)
    e = rng.standard_normal(d)
    lhs = np.einsum("hj,hde,d,e->h", st["A"], st["S"], e, e)
    rhs = np.zeros(Hkv)
    live = 0
    groups = st["groups"]
    Mg = M.reshape(Hkv, rep, d, d)
    for gi, P in enumerate(groups):
        qg = (q[:, P] * d ** -0.5).reshape(Hkv, rep, len(P), d)
        t = oc.group_terms(qg, P, k, v, Mg, rs, re, 1 if gi == len(groups) - 1 else c.STRATA_LOCAL)
        if t["nt"] == 0 or t["N"] <= 0:
            continue
        live += 1
        rhs += np.einsum("hrqj,hrq->h", t["a"], np.einsum("hrqd,d->hrq", qg, e) ** 2) / len(P) / t["N"]
    np.testing.assert_allclose(lhs, rhs / live, rtol=1e-10)
    omega = np.zeros((Hkv, rep))
    for gi, P in enumerate(groups):
        qg = (q[:, P] * d ** -0.5).reshape(Hkv, rep, len(P), d)
        t = oc.group_terms(qg, P, k, v, Mg, rs, re, 1 if gi == len(groups) - 1 else c.STRATA_LOCAL)
        if t["nt"] and t["N"] > 0:
            omega += t["wv"].sum(-1) / t["N"]
    want = np.einsum("hr,hrde->hde", omega, Mg) / omega.sum(-1)[:, None, None]
    np.testing.assert_allclose(st["Mbar"], want, rtol=1e-10)


def test_planted_error_breaks_drop_identity(monkeypatch):
    """A sign error in u (the cross term) must fail the Prop. 1 check: the check has teeth."""
    qg, pos, k, v, M = _case(1)
    real = oc.group_terms

    def wrong(qg, pos, k, v, M, rs, re, local):
        out = real(qg, pos, k, v, M, rs, re, local)
        return dict(out, dd=out["dd"] * 0 + (out["dd"] * 1.3))
    monkeypatch.setattr(oc, "group_terms", wrong)
    with pytest.raises(AssertionError):
        test_drop_term_is_prop1_exact()
