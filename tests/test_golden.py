"""The oracle and the package's host-side restatements against golden vectors written by the
reference's own functions (tests/golden/make_fixtures.py, run in the build container only).

These pin what only the reference fixes exactly:
  * uniform_step(b) floats, b = 1..8 (STRATA_KV.py:1132-1155): bit-equal;
  * rotation_matrix(d, "strata") signs, d = 64, 128 (1110-1128, _rng 306-307): equal;
  * one side's compression (1546-1548 + strata_quantize 1158-1168) on seeded fp32 rows: the fp16
    means bit-equal; Y within float32 rounding of the reference's dense (X - mu) @ R.T (the
    oracle's FWHT order); codes and fp16 scales at 2, 4 and 8 bits bit-equal both on the
    reference's own Y and end to end from X;
  * lloyd_max_gaussian levels, b = 1..4 (STRATA_KV.py:1082-1098), the QUASAR stage codebooks
    (QUASAR_KV.py:1143-1169) and embedded_quantize codes (1172-1183): bit-equal;
  * a layer compressed and packed by the reference's own QuasarMethod (1628-1710, 1786-1808) and
    decoded by its QuasarState.attend (1952-1977): the oracle's attend on that stored code
    within 1e-5 of the output's scale (the reference computes in float32, the oracle in
    float64), and the stored code's structure (embedded prefix order, byte widths);
  * a layer compressed by the reference's own StrataMethod (STRATA_KV.py:1528-1581, inputs rebuilt
    from tests/golden/layer_inputs.py) and decoded by its StrataState.attend (1762-1795): the
    oracle's decode of that stored code within 1e-5 of the output's scale; the oracle's float64
    allocation chain (coverage -> distortion table -> allocate) on the same inputs: every level
    count within 1% of the coded range and the distortion ratio within 2% (tokens near a
    decision boundary may move between float32 and float64 sums);
  * on the seeded inputs of tests/golden/layer_inputs.kivi_inputs, the reference's kivi_quant
    (826-856) codes, fp16 zero points and scales of keys and values: bit-equal; its
    chunked_attention (641-675, exact and token entries, causal positions, per-head hide_at,
    -inf padding bias, chunks of 2), snapkv_scores (932-954) and tier_reference (1751-1760) at 2,
    4 and 8 bits: within 2e-6 of each output's scale (the reference computes in float32).
"""
import sys
from pathlib import Path

import numpy as np
import pytest

import oracle.quasar as oq
import oracle.strata as os_

GOLD = Path(__file__).resolve().parent / "golden"
if str(GOLD) not in sys.path:
    sys.path.insert(0, str(GOLD))


@pytest.fixture(scope="module")
def codec():
    return np.load(GOLD / "strata_codec.npz")


@pytest.fixture(scope="module")
def books():
    return np.load(GOLD / "quasar_codebooks.npz")


def test_uniform_step_floats(codec):
    from kvq.strata import uniform_step
    for b in range(1, 9):
        step, mse = os_.uniform_step(b)
        assert step == codec["uniform_step"][b - 1] and mse == codec["uniform_mse"][b - 1], b
        assert uniform_step(b) == (codec["uniform_step"][b - 1], codec["uniform_mse"][b - 1]), b   # the package's copy


def test_rotation_signs(codec):
    from kvq.strata import _signs_np
    for d in (64, 128):
        np.testing.assert_array_equal(os_.rotation_signs(d).astype(np.int8), codec[f"signs_{d}"])
        np.testing.assert_array_equal(_signs_np(d, "strata").astype(np.int8), codec[f"signs_{d}"])


def test_center_rotate_and_quantize(codec):
    X, mu, Y = codec["X"], codec["mu"], codec["Y"]
    mu_o, Y_o = os_.strata_center_rotate(X, os_.rotation_signs(128))
    np.testing.assert_array_equal(mu_o, mu[:, 0])
    assert np.abs(Y_o - Y).max() <= 1e-6 * np.abs(Y).max()
    for b in (2, 4, 8):
        step = os_.uniform_step(b)[0]
        for y in (Y, Y_o):
            c, s, _ = os_.strata_quantize(y, b, step)
            np.testing.assert_array_equal(c, codec[f"codes_{b}"])
            np.testing.assert_array_equal(s, codec[f"scales_{b}"])


def test_lloyd_max_and_stage_codebooks(books):
    from kvq.quasar import stage_codebooks as pkg_books
    for b in range(1, 5):
        np.testing.assert_array_equal(np.asarray(oq.lloyd_max_gaussian(b), np.float32), books[f"lloyd_{b}"])
    for stages in ((2, 2, 4), (4, 4), (8,)):
        tag = "_".join(map(str, stages))
        for t, (cb_o, cb_p) in enumerate(zip(oq.stage_codebooks(stages), pkg_books(stages))):
            np.testing.assert_array_equal(np.asarray(cb_o, np.float32), books[f"levels_{tag}_{t}"])
            np.testing.assert_array_equal(np.asarray(cb_p, np.float32), books[f"levels_{tag}_{t}"])
        codes = oq.embedded_quantize(books["u"], stages)
        for t, c in enumerate(codes):
            np.testing.assert_array_equal(np.asarray(c, np.uint8), books[f"codes_{tag}_{t}"])


def reference_packed_layer():
    """The reference-packed QUASAR layer of tests/golden/quasar_state.npz as the decoders take it:
    (packed dict, stages, H, Ke, Ve, kn, vn, qn, the reference's attend output)."""
    g = np.load(GOLD / "quasar_state.npz")
    steps = [{"side": int(m[0]), "a": int(m[1]), "b": int(m[2]), "stage": int(m[3]), "n": int(m[4]),
              "codes": g[f"codes_{i}"]} for i, m in enumerate(g["step_meta"])]
    packed = {"steps": steps, "counts": g["counts"], "n_c": int(g["n_c"])}
    for nm in ("rho_k", "rho_v", "T_k", "T_v", "mu_k", "mu_v"):
        packed[nm] = g[nm]
    return (packed, tuple(int(b) for b in g["stages"]), int(g["H"]), g["Ke"], g["Ve"], g["kn"], g["vn"], g["qn"],
            g["out"])


def test_quasar_reference_packed_layer_oracle():
    packed, stages, H, Ke, Ve, kn, vn, qn, out = reference_packed_layer()
    Hkv, n_c = Ke.shape[1], packed["n_c"]
    assert n_c > 0 and Ke.shape[2] > 36
    # the stored code's structure: a non-increasing prefix n per step, each step's rows
    # (Hkv, n, w * bits / 8) bytes for its band width w
    ns = [st["n"] for st in packed["steps"]]
    assert ns[0] == n_c and all(a >= b for a, b in zip(ns, ns[1:]))
    for st in packed["steps"]:
        assert st["codes"].shape == (Hkv, st["n"], (st["b"] - st["a"]) * stages[st["stage"]] // 8)
    K = np.concatenate([Ke, kn], 2)
    V = np.concatenate([Ve, vn], 2)
    got = oq.attend(qn, 128 ** -0.5, np.array([H]), K, V, Ke.shape[2], H, packed, stages)
    err = float(np.abs(got - out).max() / np.abs(out).max())
    print(f"oracle vs the reference's QuasarState.attend on its own packed layer: {err:.2e}")
    assert err < 1e-5, err


def strata_reference_layer():
    """The reference-compressed STRATA layer: (fixture, q, k, v, M, kn, vn, qn, reference
    allocation dict {rs, re, n_ex, order}, packed dict of the reference's stored code)."""
    from layer_inputs import out_metric, strata_layer
    g = np.load(GOLD / "strata_state.npz")
    q, k, v, Wo, kn, vn, qn = strata_layer()
    M = out_metric(Wo, q.shape[1], q.shape[-1])
    al = {"rs": int(g["rs"]), "re": int(g["re"]), "n_ex": int(g["n_ex"]), "order": g["order"].astype(np.int64)}
    tiers = [{"bits": int(b), "n": int(n), "kc": g[f"kc_{i}"], "vc": g[f"vc_{i}"], "ks": g[f"ks_{i}"],
              "vs": g[f"vs_{i}"]} for i, (b, n) in enumerate(g["tier_meta"])]
    packed = {"tiers": tiers, "counts": g["counts"].astype(np.int32), "n_c": int(g["n_c"])}
    if int(g["n_c"]):
        packed["mu_k"], packed["mu_v"] = g["mu_k"], g["mu_v"]
    return g, q, k, v, M, kn, vn, qn, al, packed


def _exact_rows(x, al, H):
    """The exact rows native_state keeps (STRATA_KV.py:1679-1686): sinks, exact-level tokens, window."""
    rs, re, n_ex = al["rs"], al["re"], al["n_ex"]
    Hkv = x.shape[1]
    ids = np.concatenate([np.broadcast_to(np.arange(rs), (Hkv, rs)), al["order"][:, :n_ex] + rs,
                          np.broadcast_to(np.arange(re, H), (Hkv, H - re))], 1)
    return np.take_along_axis(x[0], ids[..., None], 1)


def test_strata_reference_layer_oracle():
    import oracle.coverage as oc
    import oracle.strata_alloc as oa
    g, q, k, v, M, kn, vn, qn, al, packed = strata_reference_layer()
    H, d = k.shape[2], k.shape[3]
    assert int(g["payload"]) * 8 == float(g["bits"])            # the reference's own invariant
    K = np.concatenate([_exact_rows(k, al, H), kn[0]], 1)
    V = np.concatenate([_exact_rows(v, al, H), vn[0]], 1)
    tiers = [(t["bits"], os_.unpack_planar(t["kc"], t["bits"]), t["ks"].astype(np.float32),
              os_.unpack_planar(t["vc"], t["bits"]), t["vs"].astype(np.float32)) for t in packed["tiers"]]
    got = os_.strata_attend(qn, d ** -0.5, K, V, tiers, packed["mu_k"].astype(np.float32),
                            packed["mu_v"].astype(np.float32), os_.rotation_matrix(d))
    out = g["out"]
    err = float(np.abs(got - out).max() / np.abs(out).max())
    print(f"oracle decode vs the reference's StrataState.attend on its own stored code: {err:.2e}")
    assert err < 1e-5, err
    # the allocation: the oracle's float64 chain on the same inputs
    rs, re = al["rs"], al["re"]
    bits = (2, 4, 8)
    st = oc.coverage_stats(q[0].astype(np.float64), np.arange(H), k[0].astype(np.float64), v[0].astype(np.float64),
                           d ** -0.5, H, rs, re, M.astype(np.float64), oc.CoverageParams())
    signs = os_.rotation_signs(d)
    _, Yk = os_.strata_center_rotate(k[0, :, rs:re], signs)
    _, Yv = os_.strata_center_rotate(v[0, :, rs:re], signs)
    Dt = oa.distortion_table(Yk, Yv, st["S"], st["Mbar"], st["A"], st["W"], st["DD"], bits)
    cost, fixed, budget, hist_bits, _ = oa.layer_costs(bits, d, k.shape[1], H, float(g["keep"]), rs, re)
    ref = oa.allocate(Dt, cost, fixed, budget, 4, search=budget >= hist_bits)
    rel = abs(ref["distortion"] - float(g["distortion"])) / float(g["distortion"])
    print(f"oracle counts {np.asarray(ref['counts']).tolist()} vs the reference's {g['counts'].tolist()}; "
          f"distortion {ref['distortion']:.7f} vs {float(g['distortion']):.7f} (relative {rel:.1e})")
    # the float64 chain reproduces the reference's allocation exactly: every level count, the
    # distortion ratio to float32-level accuracy and the payload the counts imply
    assert np.asarray(ref["counts"]).tolist() == g["counts"].tolist()
    assert rel <= 1e-6, rel
    assert float(ref["bits"]) == float(g["bits"])


@pytest.fixture(scope="module")
def kiv():
    from layer_inputs import kivi_inputs
    return np.load(GOLD / "kivi_attention.npz"), kivi_inputs()


def test_kivi_quant_reference(kiv):
    import oracle.kivi as ok
    g, x = kiv
    for bits in (2, 4):
        cases = [(f"k_{bits}_{gr}_{sk}", x["K"], gr, True, sk) for gr in (32, 64) for sk in (0, 4)]
        cases += [(f"v_{bits}_{gr}", x["V"], gr, False, 0) for gr in (32, 64, 128)]
        for tag, X, gr, along, sk in cases:
            r = ok.kivi_quant(X, bits, gr, along, sk)
            np.testing.assert_array_equal(r["codes"], g[f"{tag}_codes"], err_msg=tag)
            np.testing.assert_array_equal(np.asarray(r["lo"], np.float32), g[f"{tag}_lo"], err_msg=tag)
            np.testing.assert_array_equal(np.asarray(r["scale"], np.float32), g[f"{tag}_scale"], err_msg=tag)


def _rel(got, want):
    return float(np.abs(np.asarray(got, np.float64) - want).max() / np.abs(want).max())


def test_chunked_attention_reference(kiv):
    from oracle.attention import chunked_attention
    g, x = kiv
    hide = np.full((1, 2, 100), 10 ** 9, np.int64)
    hide[0, 0, 10:20] = 98
    b = np.zeros((1, 2, 50), np.float32)
    b[:, :, 45:] = -np.inf
    tok = {"k": x["tk"], "v": x["tv"], "b": b, "tau": np.arange(50) + 60}
    got = chunked_attention(x["qa"], 128 ** -0.5, np.array([97, 98, 99]), x["K"], x["V"], np.arange(100), hide, tok, 2)
    assert _rel(got, g["attn"]) < 2e-6


def test_snapkv_scores_reference(kiv):
    import oracle.evict as oe
    g, x = kiv
    w, kern = (int(v) for v in g["snap_params"])
    got = oe.snapkv_scores(x["qs"], x["ks"], 300, 128 ** -0.5, w, kern)
    assert _rel(got, g["snap"]) < 2e-6


def test_tier_reference_partials(kiv):
    g, x = kiv
    for bits in (2, 4, 8):
        ck, cv = x["codes"][bits]
        sk, sv = (s_.astype(np.float16).astype(np.float32) for s_ in x["scales"][bits])
        m, l_, acc = os_.tier_partials(x["qr"], x["qb"], ck, sk, cv, sv, bits)
        assert _rel(m, g[f"tier_{bits}_m"][:, 0]) < 2e-6, bits
        assert _rel(l_, g[f"tier_{bits}_l"][:, 0]) < 2e-6, bits
        assert _rel(acc, g[f"tier_{bits}_acc"][:, 0]) < 2e-6, bits
