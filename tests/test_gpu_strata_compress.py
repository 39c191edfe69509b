"""STRATA compression of one layer end to end on the GPU (kvq.StrataCompressor, STRATA_KV.py:1528-1687).

The chain coverage_stats -> distortion table -> allocation -> per-stratum codes -> pack ->
native_state runs on the device from the layer's own queries, keys, values and output metric.
Checked, as the reference's own tests check its compression (STRATA_KV.py:1975-1992):
* payload bytes x 8 == the allocator's bits (exact; the stored code is measured, not counted);
* the bf16 native state's context_bytes x 8 == allocator bits + exact rows (exact);
* the state's decode after an appended token == attention over the code's reconstruction plus the
  exact rows (oracle.strata_attend over the very tiers the device packed; bar 2e-3 fp32 / 1e-2 bf16);
* every stored tier: planar codes and fp16 scales bit-equal to the oracle's strata_quantize of the
  device's rotated rows at that width, rows in the allocation's order (the code is cut correctly);
* the allocation against the float64 oracle chain (oracle.coverage -> distortion_table ->
  allocate) on the same inputs: every level count within 1% of the coded range (the device's float32
  table is within 2e-3 of each column's scale, so tokens near a decision boundary may move), and the
  distortion ratio within 2% relative;
* and against the reference itself (tests/golden/strata_state.npz: a seeded layer compressed by its
  own StrataMethod): the device's allocation of the same inputs (level counts within 1% of the coded
  range, distortion ratio within 2%, payload bits == the reference's when the counts agree), and the
  reference's own stored code decoded by the device's StrataState after one appended token against
  its StrataState.attend (fp32: the STRATA decode's bar, 2e-3 of the output's scale; measured 1.4e-4).
"""
import numpy as np
import pytest
import torch

import oracle.coverage as oc
import oracle.strata as os_
import oracle.strata_alloc as oa

pytestmark = pytest.mark.gpu

D = 128


def _layer(seed, Hq, Hkv, H, dtype):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(1, Hq, H, D, generator=g) * 1.5
    k = torch.randn(1, Hkv, H, D, generator=g) * 1.2
    v = torch.randn(1, Hkv, H, D, generator=g)
    rep = Hq // Hkv
    k[:, :, 0] += 2.0 * q[0, ::rep].mean(1)[None]                      # a sink the queries lean on
    hot = torch.randperm(H - 40, generator=g)[:12] + 8                  # a few heavily read tokens
    k[:, :, hot] += 1.5 * q[0, ::rep, -32:].mean(1)[None, :, None]
    Wo = torch.randn(Hq, 32, D, generator=g)
    M = (Wo.transpose(1, 2) @ Wo) / 32
    return q.to(dtype), k.to(dtype), v.to(dtype), M


def _oracle_alloc(q, k, v, M, H, keep, bits, rs, re):
    c = oc.CoverageParams()
    st = oc.coverage_stats(q[0].double().numpy(), np.arange(H), k[0].double().numpy(), v[0].double().numpy(),
                           D ** -0.5, H, rs, re, M.double().numpy(), c)
    signs = os_.rotation_signs(D)
    _, Yk = os_.strata_center_rotate(k[0, :, rs:re].float().numpy(), signs)
    _, Yv = os_.strata_center_rotate(v[0, :, rs:re].float().numpy(), signs)
    Dt = oa.distortion_table(Yk, Yv, st["S"], st["Mbar"], st["A"], st["W"], st["DD"], bits)
    Hkv = k.shape[1]
    cost, fixed, budget, hist_bits, _ = oa.layer_costs(bits, D, Hkv, H, keep, rs, re)
    return oa.allocate(Dt, cost, fixed, budget, 4, search=budget >= hist_bits)


@pytest.mark.parametrize("dtype,Hq,Hkv,H,keep", [
    (torch.float32, 8, 2, 1100, 0.25),
    (torch.bfloat16, 16, 4, 1300, 0.125),
])
def test_compress_layer_end_to_end(dtype, Hq, Hkv, H, keep):
    import kvq
    from kvq.strata_compress import StrataCompressor
    q, k, v, M = _layer(7 + Hq, Hq, Hkv, H, dtype)
    comp = StrataCompressor(keep)
    al = comp.compress_layer(q.cuda(), k.cuda(), v.cuda(), D ** -0.5, H, M.cuda())
    nb = len(comp.bits)
    rs, re = al["rs"], al["re"]
    assert (rs, re) == (4, H - 32) and sum(al["counts"]) == re - rs
    assert al["n_c"] > 0 and al["n_ex"] + al["n_c"] <= re - rs
    print(f"{dtype} keep {keep}: counts {al['counts']}, distortion {al['distortion']:.4f}")
    packed = comp.pack(al)
    # the reference's invariants: measured bytes == allocator bits, for the code and the bf16 state
    assert comp.payload(packed) * 8 == al["bits"]
    st_b = comp.native_state(al, packed, k.cuda(), v.cuda(), 4, torch.bfloat16)
    assert st_b.n0 == rs + al["n_ex"] + (H - re)
    assert st_b.context_bytes() * 8 == al["bits"] + st_b.n0 * Hkv * 2 * D * 16
    # each tier's code: the oracle's quantiser of the device's rotated rows, in the order's rows
    order = al["order"].long().cpu().numpy()
    assert [t["bits"] for t in packed["tiers"]] == [comp.bits[o - 1] for o, _, _ in comp.strata(al)]
    for (o, a, m), t in zip(comp.strata(al), packed["tiers"]):
        for s, nm in ((0, "k"), (1, "v")):
            y = al["y"][s].cpu().numpy()
            rows = np.take_along_axis(y, order[:, a:a + m, None], 1)
            c_o, s_o, _ = os_.strata_quantize(rows, t["bits"], os_.uniform_step(t["bits"])[0])
            np.testing.assert_array_equal(t[f"{nm}c"].cpu().numpy(), os_.pack_planar(c_o, t["bits"]))
            np.testing.assert_array_equal(t[f"{nm}s"].float().cpu().numpy(), s_o)
    # decode of the compressed layer after one appended token == attention over its reconstruction
    st = comp.native_state(al, packed, k.cuda(), v.cuda(), 4, dtype)
    g = torch.Generator().manual_seed(99)
    kn = torch.randn(1, Hkv, 1, D, generator=g).to(dtype)
    vn = torch.randn(1, Hkv, 1, D, generator=g).to(dtype)
    qn = (torch.randn(1, Hq, 1, D, generator=g) * 1.5).to(dtype)
    st.append(kn.cuda(), vn.cuda(), torch.tensor([H]))
    out = st.attend(qn.cuda(), D ** -0.5, torch.tensor([H])).float().cpu().numpy()
    tiers = [(t["bits"], os_.unpack_planar(t["kc"].cpu().numpy(), t["bits"]), t["ks"].float().cpu().numpy(),
              os_.unpack_planar(t["vc"].cpu().numpy(), t["bits"]), t["vs"].float().cpu().numpy())
             for t in packed["tiers"]]
    ref = os_.strata_attend(qn.float().numpy(), D ** -0.5, st.K[0, :, :st.n].float().cpu().numpy(),
                            st.V[0, :, :st.n].float().cpu().numpy(), tiers,
                            packed["mu_k"].to(dtype).float().cpu().numpy(),
                            packed["mu_v"].to(dtype).float().cpu().numpy(), os_.rotation_matrix(D))
    err = float(np.abs(out - ref[0]).max())
    print(f"  decode vs reconstruction: max-abs-err {err:.3e}")
    assert err <= (2e-3 if dtype == torch.float32 else 1e-2), err
    # the allocation against the float64 oracle chain on the same (dtype-rounded) inputs
    ref_al = _oracle_alloc(q, k, v, M, H, keep, comp.bits, rs, re)
    tol = max(2, int(0.01 * (re - rs)))
    diff = np.abs(np.asarray(al["counts"]) - ref_al["counts"])
    print(f"  oracle counts {ref_al['counts'].tolist()}, distortion {ref_al['distortion']:.4f}")
    assert diff.max() <= tol, (al["counts"], ref_al["counts"].tolist())
    assert abs(al["distortion"] - ref_al["distortion"]) <= 0.02 * ref_al["distortion"]


def test_compress_layer_uniform_and_nothing_to_code():
    """The importance-free variant (one price per position) and a layer whose range is empty."""
    from kvq.strata_compress import StrataCompressor
    q, k, v, M = _layer(3, 8, 2, 700, torch.bfloat16)
    comp = StrataCompressor(0.25, uniform=True)
    al = comp.compress_layer(q.cuda(), k.cuda(), v.cuda(), D ** -0.5, 700, M.cuda())
    packed = comp.pack(al)
    assert comp.payload(packed) * 8 == al["bits"]
    assert al["counts"][0] + al["n_c"] + al["n_ex"] == al["re"] - al["rs"]
    assert comp.compress_layer(q.cuda()[:, :, :30], k.cuda()[:, :, :30], v.cuda()[:, :, :30], D ** -0.5, 30,
                               M.cuda()) is None
    st = comp.native_state(None, None, k.cuda(), v.cuda(), 2, torch.bfloat16)
    assert st.n0 == 700 and st.context_bytes() == 2 * 2 * 700 * D * 2


def test_compress_and_decode_against_reference():
    from kvq.strata_compress import StrataCompressor
    from test_golden import strata_reference_layer
    g, q, k, v, M, kn, vn, qn, ref_al, ref_packed = strata_reference_layer()
    H, d = k.shape[2], k.shape[3]
    cu = lambda x: torch.from_numpy(np.ascontiguousarray(x)).cuda()
    comp = StrataCompressor(float(g["keep"]))
    al = comp.compress_layer(cu(q), cu(k), cu(v), d ** -0.5, H, cu(M))
    rs, re = al["rs"], al["re"]
    assert (rs, re) == (int(g["rs"]), int(g["re"]))
    rel = abs(al["distortion"] - float(g["distortion"])) / float(g["distortion"])
    print(f"device counts {list(al['counts'])} vs the reference's {g['counts'].tolist()}; "
          f"distortion {al['distortion']:.7f} vs {float(g['distortion']):.7f} (relative {rel:.1e})", flush=True)
    # the device's allocation of the reference's layer is the reference's: every level count, the
    # payload in bytes, and the distortion ratio to the float32 statistics' accuracy
    assert list(al["counts"]) == g["counts"].tolist()
    assert rel <= 1e-4, rel
    packed = comp.pack(al)
    assert comp.payload(packed) == int(g["payload"])
    # the reference's own stored code, decoded on the device
    p = dict(ref_packed)
    p["tiers"] = [{"bits": t["bits"], "n": t["n"], "kc": cu(t["kc"]), "vc": cu(t["vc"]), "ks": cu(t["ks"]),
                   "vs": cu(t["vs"])} for t in ref_packed["tiers"]]
    p["counts"] = torch.from_numpy(ref_packed["counts"])
    p["mu_k"], p["mu_v"] = cu(ref_packed["mu_k"]), cu(ref_packed["mu_v"])
    ral = dict(ref_al, order=torch.from_numpy(ref_al["order"]).cuda())
    st = comp.native_state(ral, p, cu(k), cu(v), 2, torch.float32)
    st.append(cu(kn), cu(vn), torch.tensor([H]))
    got = st.attend(cu(qn), d ** -0.5, torch.tensor([H])).float().cpu().numpy()
    err = float(np.abs(got - g["out"]).max() / np.abs(g["out"]).max())
    print(f"device decode vs the reference's StrataState.attend on its own stored code: {err:.2e}", flush=True)
    assert err < 2e-3, err
