"""GPU QUASAR compressed-domain decode (kvq.QuasarState.attend) against the oracle
(oracle/quasar.py: QuasarState.attend, QUASAR_KV.py:1945-1968, in float64).

Tolerances (relative to the output's max magnitude): float32 2e-3, bfloat16 1e-2.  Cases: GQA 4
with one and two query rows, one and two rows per KV head (GQA 1 and 2), codes at (2, 2, 4),
(4, 4), (8,) and (1, 2, 4) bits, coded-token counts around
the 64-token chunk (1, 63, 64, 65) and long ones, exact rows in the merge (up to 128) and in 128-row blocks of the split launch (129 .. 1500), appended
causal rows, no coded tokens, and the state's own kernel check.
"""
import numpy as np
import pytest
import torch

import oracle.quasar as oq

pytestmark = pytest.mark.gpu


def _state(Hkv, n_c, n0, extra, stages, dtype, seed, bands=None):
    import kvq
    from kvq.quasar import synthetic_packed
    g = torch.Generator().manual_seed(seed)
    kw = {} if bands is None else {"bands": bands}
    p = synthetic_packed(Hkv, 128, n_c, stages=stages, seed=seed, **kw) if n_c > 0 else {"steps": [], "n_c": 0}
    K = torch.randn((1, Hkv, n0, 128), generator=g).to(dtype)
    V = torch.randn((1, Hkv, n0, 128), generator=g).to(dtype)
    H = 5000
    st = kvq.QuasarState(K.cuda(), V.cuda(), p, stages, extra, H)
    return st, p, K, V, H, g


def _check(st, p, K_all, V_all, n0, H, q, qpos, stages, tol):
    got = st.attend(q.cuda(), 128 ** -0.5, qpos).float().cpu().numpy()
    want = oq.attend(q.float().numpy(), 128 ** -0.5, np.asarray(qpos), K_all.float().numpy(), V_all.float().numpy(),
                     n0, H, p, stages)
    err = np.abs(got - want).max() / np.abs(want).max()
    assert err < tol, err


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 2e-3), (torch.bfloat16, 1e-2)])
@pytest.mark.parametrize("n_c,n0", [(1, 40), (63, 40), (64, 300), (65, 129), (1000, 36), (5000, 700), (2000, 1500)])
def test_quasar_decode_matches_oracle(dtype, tol, n_c, n0):
    st, p, K, V, H, g = _state(2, n_c, n0, 0, (2, 2, 4), dtype, 100 + n_c)
    q = torch.randn((1, 8, 1, 128), generator=g).to(dtype)
    _check(st, p, K, V, n0, H, q, [H], (2, 2, 4), tol)


@pytest.mark.parametrize("stages", [(4, 4), (8,), (2, 2, 4)])
def test_quasar_decode_stages_two_rows_and_appends(stages):
    dtype = torch.bfloat16
    st, p, K, V, H, g = _state(4, 777, 200, 4, stages, dtype, 7)
    k = torch.randn((1, 4, 3, 128), generator=g).to(dtype)
    v = torch.randn((1, 4, 3, 128), generator=g).to(dtype)
    st.append(k.cuda(), v.cuda(), torch.tensor([H, H + 1, H + 2]))
    q = torch.randn((1, 16, 2, 128), generator=g).to(dtype)
    qpos = [H + 1, H + 2]                                   # row H+2 visible to the second query only
    _check(st, p, torch.cat([K, k], 2), torch.cat([V, v], 2), 200, H, q, qpos, stages, 1e-2)


@pytest.mark.parametrize("rep,Tq,stages,bands,dtype", [(1, 1, (1, 2, 4), (0.25, 0.25, 0.5), torch.float32),
                                                      (2, 1, (2, 2, 4), None, torch.bfloat16),
                                                      (1, 2, (4, 4), None, torch.float32),
                                                      (2, 2, (1, 2, 4), (0.25, 0.25, 0.5), torch.bfloat16)])
def test_quasar_decode_one_and_two_rows_one_bit(rep, Tq, stages, bands, dtype):
    """One and two query rows per KV head (the split's R = 1, 2 instantiations) and 1-bit stage codes
    (bands of at least 32 coefficients, so every step's rows fill whole 4-byte slots)."""
    Hkv = 4
    st, p, K, V, H, g = _state(Hkv, 1300, 150, 0, stages, dtype, 50 + rep + Tq, bands)
    q = torch.randn((1, Hkv * rep, Tq, 128), generator=g).to(dtype)
    qpos = [H] * Tq
    _check(st, p, K, V, 150, H, q, qpos, stages, 2e-3 if dtype == torch.float32 else 1e-2)


def test_quasar_exact_only_and_kernel_check():
    st, p, K, V, H, g = _state(2, 0, 300, 0, (2, 2, 4), torch.float32, 3)
    q = torch.randn((1, 8, 1, 128), generator=g)
    _check(st, p, K, V, 300, H, q, [H], (2, 2, 4), 2e-3)
    st2, *_ = _state(2, 3000, 100, 2, (2, 2, 4), torch.bfloat16, 4)
    assert st2.check_kernel()["kernel"]


def test_quasar_rejects_bad_input():
    import kvq
    st, p, K, V, H, g = _state(2, 100, 40, 0, (2, 2, 4), torch.float32, 9)
    with pytest.raises(ValueError):
        st.attend(torch.randn((1, 8, 1, 128)).cuda(), 0.1, [H, H + 1])
    with pytest.raises(RuntimeError):
        st.append(torch.zeros((1, 2, 1, 128)).cuda(), torch.zeros((1, 2, 1, 128)).cuda(), [H])


def test_quasar_question_step_of_many_tokens():
    """A 6-token step at rep 4 (24 rows per KV head): query pieces of 2 tokens, the appended rows
    causal among them, against the oracle."""
    dtype = torch.float32
    st, p, K, V, H, g = _state(2, 900, 120, 6, (2, 2, 4), dtype, 21)
    k = torch.randn((1, 2, 6, 128), generator=g).to(dtype)
    v = torch.randn((1, 2, 6, 128), generator=g).to(dtype)
    st.append(k.cuda(), v.cuda(), torch.arange(H, H + 6))
    q = torch.randn((1, 8, 6, 128), generator=g).to(dtype)
    _check(st, p, torch.cat([K, k], 2), torch.cat([V, v], 2), 120, H, q, list(range(H, H + 6)), (2, 2, 4), 2e-3)


def test_quasar_reference_packed_layer():
    """The stored code of a layer compressed and packed by the reference's own QuasarMethod
    (tests/golden/quasar_state.npz: 456 coded tokens over 23 levels, rank 128, 76 exact rows)
    decoded on the GPU after one appended token, against the reference's QuasarState.attend output
    for the same query (fp32, bar 2e-3 of the output's scale, as the synthetic cases)."""
    import kvq
    from test_golden import reference_packed_layer
    packed, stages, H, Ke, Ve, kn, vn, qn, out = reference_packed_layer()
    to = lambda x: torch.from_numpy(np.ascontiguousarray(x)).cuda()
    p = dict(packed)
    p["steps"] = [dict(st, codes=torch.from_numpy(np.ascontiguousarray(st["codes"]))) for st in packed["steps"]]
    st = kvq.QuasarState(to(Ke), to(Ve), p, stages, 1, H)
    st.append(to(kn), to(vn), torch.tensor([H]))
    got = st.attend(to(qn), 128 ** -0.5, torch.tensor([H])).float().cpu().numpy()
    err = float(np.abs(got - out).max() / np.abs(out).max())
    print(f"GPU QUASAR decode vs the reference on its own packed layer: {err:.2e}", flush=True)
    assert err < 2e-3, err


@pytest.mark.parametrize("stages", [(2, 2, 4), (4, 4), (8,)])
def test_quasar_scores_and_values_wrappers(stages):
    """kvq.quasar_scores / quasar_values with the reference's call shapes (QUASAR_KV.py:1556-1577):
    on a QuasarState's own sides and on a side laid out as the reference's QuasarState holds it (step
    table on the device, concatenated levels), against the oracle's per-step products (float64) at
    rtol 1e-5 of the largest entry; n_c crosses a 1024-token chunk of the values partials."""
    import kvq
    from kvq.quasar import synthetic_packed
    Hkv, n_c, rows = 2, 2500, 6
    p = synthetic_packed(Hkv, 128, n_c, stages=stages, seed=9)
    K = torch.zeros((1, Hkv, 4, 128), device="cuda")
    st = kvq.QuasarState(K, K, p, stages, 2, 100)
    R = st.T_k.shape[-1]
    g = torch.Generator().manual_seed(3)
    qt = torch.randn((Hkv, rows, R), generator=g)
    pv = torch.rand((Hkv, rows, n_c), generator=g)
    want_s = oq.coded_scores(qt.double().numpy(), p, stages)
    want_v = oq.coded_values(pv.double().numpy(), p, stages, R)
    ref_side = lambda s_: {"flat": st.sides[s_]["flat"], "table": st.sides[s_]["table"],      # device table
                           "levels": torch.cat([torch.from_numpy(b) for b in kvq.stage_codebooks(stages)]).cuda(),
                           "W": 128}
    for side0, side1 in ((st.sides[0], st.sides[1]), (ref_side(0), ref_side(1))):
        got_s = kvq.quasar_scores(qt.cuda(), side0, n_c).cpu().numpy()
        got_v = kvq.quasar_values(pv.cuda(), side1, R).cpu().numpy()
        assert got_s.shape == (Hkv, rows, n_c) and got_v.shape == (Hkv, rows, R)
        assert np.abs(got_s - want_s).max() <= 1e-5 * np.abs(want_s).max()
        assert np.abs(got_v - want_v).max() <= 1e-5 * np.abs(want_v).max()
    # a step table that points past the code buffer is refused before any launch
    bad = dict(st.sides[0], table_np=st.sides[0]["table_np"].copy())
    bad["table_np"][0, 0] = st.sides[0]["flat"].numel()
    with pytest.raises(kvq.KVQError, match="leave the buffer"):
        kvq.quasar_scores(qt.cuda(), bad, n_c)
