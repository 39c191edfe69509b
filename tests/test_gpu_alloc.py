"""GPU parity of the STRATA allocation (kvq_strata_allocate) with the oracle (oracle/strata_alloc.py).

Bit-exact: order, Dsort, choice, lev, counts, bits and cap; the distortion ratio to 1e-12
(float64 sums in different orders).  Cases: sizes from one token to the bench layer, 2 to 7
options, tied importance keys, NaN / inf entries, zero rounds, the all-drop branch, the
reference's own allocator checks (STRATA_KV.py:1945-1961) and compress_layer's bookkeeping.
"""
import numpy as np
import pytest
import torch

import oracle.strata_alloc as oa

pytestmark = pytest.mark.gpu


def _table(Hkv, n, nlev, seed):
    """A layer-like table: drop distortion spread over decades, levels shrinking ~4^-b, exact 0."""
    rng = np.random.default_rng(seed)
    imp = np.exp(rng.normal(0, 2.0, (Hkv, n, 1)))
    cols = [imp * rng.uniform(0.5, 2.0, (Hkv, n, 1))]
    for l in range(1, nlev - 1):
        cols.append(imp * 4.0 ** (-2 * l) * rng.uniform(0.5, 2.0, (Hkv, n, 1)))
    cols.append(np.zeros((Hkv, n, 1)))
    return np.concatenate(cols, -1).astype(np.float32)


def _costs(Hkv, nlev):
    bits = (2, 4, 8, 3, 6)[: nlev - 2]
    tok = np.array([0.0] + [2.0 * (b * 128 + 16) for b in bits] + [4096.0])
    fixed = np.where(np.arange(nlev - 1) > 0, Hkv * 4096.0, 0.0) + nlev * 32.0
    return tok * Hkv, fixed


def _compare(D, cost, fixed, budget, rounds=4, search=True):
    import kvq
    got = kvq.strata_allocate(torch.from_numpy(D).cuda(), cost, fixed, budget, rounds, search)
    want = oa.allocate(D, cost, fixed, budget, rounds=rounds, search=search)
    np.testing.assert_array_equal(got["order"].cpu().numpy(), want["order"])
    np.testing.assert_array_equal(got["dsort"].cpu().numpy(), want["dsort"])
    np.testing.assert_array_equal(got["choice"].cpu().numpy(), want["choice"])
    np.testing.assert_array_equal(got["lev"].cpu().numpy(), want["lev"])
    np.testing.assert_array_equal(got["counts"].cpu().numpy(), want["counts"])
    s = got["summary"].cpu().numpy()
    assert s[0] == want["bits"] and int(s[1]) == want["cap"]
    assert abs(s[2] - want["distortion"]) <= 1e-12 * max(1.0, abs(want["distortion"]))
    return got, want


@pytest.mark.parametrize("Hkv,n,nlev,keep", [(1, 1, 2, 0.5), (2, 7, 3, 0.3), (8, 257, 5, 0.2), (4, 1000, 4, 0.1),
                                             (8, 5000, 6, 0.15), (3, 2049, 7, 0.5), (8, 32732, 5, 0.125)])
def test_allocate_matches_oracle(Hkv, n, nlev, keep):
    D = _table(Hkv, n, nlev, seed=n + nlev)
    cost, fixed = _costs(Hkv, nlev)
    budget = keep * n * cost[-1]
    got, want = _compare(D, cost, fixed, budget)
    assert want["bits"] <= budget or want["counts"][0] == n


def test_ties_and_non_finite():
    D = _table(4, 600, 5, seed=3)
    D[:, 100:300, 0] = 0.5                                       # tied importance keys
    D[:, 100:300, 1] = 0.25
    D[1, 5, 0], D[2, 6, 1], D[3, 7, 2], D[0, 8, 3] = np.inf, np.nan, -np.inf, np.nan
    cost, fixed = _costs(4, 5)
    _compare(D, cost, fixed, 0.2 * 600 * cost[-1])


@pytest.mark.parametrize("rounds,search", [(0, True), (1, True), (6, True), (4, False)])
def test_rounds_and_all_drop(rounds, search):
    D = _table(8, 3000, 5, seed=11)
    cost, fixed = _costs(8, 5)
    got, _ = _compare(D, cost, fixed, 0.1 * 3000 * cost[-1], rounds=rounds, search=search)
    if not search:
        assert (got["choice"] == 0).all().item()


def test_reference_allocator_checks_on_gpu():
    import kvq
    rng = np.random.default_rng(7)
    Dl = (rng.random((1, 300, 1)) * np.array([1.0, 0.12, 0.012, 1e-4, 0.0])).astype(np.float32)
    cost = np.array([0.0, 544.0, 1056.0, 2080.0, 4096.0])
    fixed = np.array([160.0, 4256.0, 4256.0, 4256.0])
    prev = -1.0
    for budget in (5e3, 3e4, 1e5, 3e5, 2e6):
        got = kvq.strata_allocate(torch.from_numpy(Dl).cuda(), cost, fixed, budget)
        s = got["summary"].cpu().numpy()
        assert s[0] <= budget + 1e-3
        order = got["order"].cpu().numpy()[0]
        dist = float(Dl[0, order, got["choice"].cpu().numpy()].astype(np.float64).sum())
        assert not (prev >= 0 and dist > prev + 1e-6)
        prev = dist
    assert (got["choice"] == 4).all().item()


@pytest.mark.parametrize("keep", [0.002, 0.125, 0.5])
def test_allocate_layer_bookkeeping(keep):
    import kvq
    Hkv, d, H, bits = 8, 128, 4096, (2, 4, 8)
    rs, re = 4, H - 32
    D = _table(Hkv, re - rs, len(bits) + 2, seed=5)
    al = kvq.allocate_layer(torch.from_numpy(D).cuda(), bits, d, H, keep, rs, re)
    cost, fixed, budget, hist, tok = oa.layer_costs(bits, d, Hkv, H, keep, rs, re)
    want = oa.allocate(D, cost, fixed, budget, search=budget >= hist)
    assert al["counts"] == want["counts"].tolist()
    np.testing.assert_array_equal(al["lev"].cpu().numpy(), want["lev"])
    lev = want["lev"]
    coded = (lev >= 1) & (lev <= len(bits))
    cap = int(lev[coded].max()) if coded.any() else 0
    assert al["bits"] == float((tok[lev[coded]] * Hkv).sum() + fixed[min(cap, 1)])
    assert al["n_c"] == int(coded.sum()) and al["n_ex"] == int((lev == len(bits) + 1).sum())
    if budget >= hist:
        assert al["bits"] <= budget


def test_rejects_bad_arguments():
    import kvq
    D = torch.zeros((2, 10, 17), device="cuda")
    with pytest.raises(kvq.KVQError):
        kvq.strata_allocate(D, np.zeros(17), np.zeros(16), 1e6)
    with pytest.raises(ValueError):
        kvq.strata_allocate(torch.zeros((2, 10, 5), device="cuda"), np.zeros(4), np.zeros(4), 1e6)


@pytest.mark.parametrize("Hkv,n,dtype", [(2, 3, torch.float32), (4, 700, torch.bfloat16), (8, 4093, torch.float32)])
def test_distortion_matches_oracle_and_feeds_allocation(Hkv, n, dtype):
    import kvq
    import oracle.strata as os_
    g = torch.Generator().manual_seed(n)
    K = (torch.randn((Hkv, n, 128), generator=g) * 2 + 0.5).to(dtype)
    V = torch.randn((Hkv, n, 128), generator=g).to(dtype)
    G = torch.randn((2, Hkv, 128, 128), generator=g)
    S, Mbar = (G[0] @ G[0].transpose(1, 2) / 128).contiguous(), (G[1] @ G[1].transpose(1, 2) / 128).contiguous()
    A, W, DD = torch.rand((3, Hkv, n), generator=g)
    bits = (2, 4, 8)
    out = kvq.strata_distortion(K.cuda(), V.cuda(), A.cuda(), W.cuda(), DD.cuda(), S.cuda(), Mbar.cuda(), bits)
    signs = os_.rotation_signs(128)
    (_, Yk), (_, Yv) = os_.strata_center_rotate(K.float().numpy(), signs), os_.strata_center_rotate(V.float().numpy(), signs)
    np.testing.assert_array_equal(out["y_k"].cpu().numpy(), Yk)                 # the codec is bit-exact
    np.testing.assert_array_equal(out["y_v"].cpu().numpy(), Yv)
    want = oa.distortion_table(Yk, Yv, S.numpy(), Mbar.numpy(), A.numpy(), W.numpy(), DD.numpy(), bits)
    got = out["D"].cpu().numpy()
    np.testing.assert_array_equal(got[..., 0], DD.numpy())
    np.testing.assert_array_equal(got[..., -1], 0.0)
    # the codes and scales are the codec's (exact), so what remains is the float32 evaluation of
    # e^T Mt e: bounded element by element by 4e-6 x (A |e_K|^T |Mt_K| |e_K| + W |e_V|^T |Mt_V| |e_V|).
    # Rounding the kernel's own float32 order on the host reaches 2.6e-7 of that quantity; a code one
    # step off or a scale one fp16 ulp off moves an element by more than 2e-4 of it.
    R = os_.rotation_matrix(128, "strata").astype(np.float64)
    absq = []
    for b in bits:
        qs = []
        for Y, M in ((Yk, S.numpy()), (Yv, Mbar.numpy())):
            e = np.abs(os_.strata_quantize(Y, b, os_.uniform_step(b)[0])[2].astype(np.float64) - Y)
            qs.append(np.einsum("hnd,hde,hne->hn", e, np.abs(R @ M.astype(np.float64) @ R.T), e))
        absq.append(A.numpy() * qs[0] + W.numpy() * qs[1])
    tol = 4e-6 * np.stack(absq, -1)
    err = np.abs(got[..., 1:-1] - want[..., 1:-1])
    assert (err <= tol).all(), (float((err / tol).max()), np.argwhere(err > tol)[:5].tolist())
    H = n + 36
    al = kvq.allocate_layer(out["D"], bits, 128, H, 0.3, 4, H - 32)
    cost, fixed, budget, hist, _ = oa.layer_costs(bits, 128, Hkv, H, 0.3, 4, H - 32)
    ref = oa.allocate(got, cost, fixed, budget, search=budget >= hist)
    np.testing.assert_array_equal(al["lev"].cpu().numpy(), ref["lev"])
    np.testing.assert_array_equal(al["order"].cpu().numpy(), ref["order"])
