"""The reference-shaped STRATA decode boundary on the GPU against the float64 oracle.

* StrataState(Ke, Ve, packed, extra, H, R) (STRATA_KV.py:1710-1818) built from a packed code in
  StrataMethod.pack's format (1611-1627), driven through DecodeCtl / router_attention as the
  reference's generation loop drives it: one-token steps and a multi-token step whose appended rows
  are causal among themselves; batch 1 (the reference's) and batch 2; fp32 and bf16.  Each step
  against oracle.strata_attend over the visible exact rows (bar 2e-3 fp32 / 1e-2 bf16).
* check_kernel against the state's own torch path, and context_bytes against tensor_bytes of the
  exact rows and the packed code (1729-1735).
* strata_tier_kernel(qr, qb, t) (1450-1469): the reference's shapes (S by its split rule, 12 rows:
  two launches of the 8-row kernel), and its partials merged (log-sum-exp over the splits) equal
  the oracle's single-partial tier_reference (1751-1760) for 2, 4 and 8 bits.
"""
from types import SimpleNamespace

import numpy as np
import pytest
import torch

import oracle.strata as os_

pytestmark = pytest.mark.gpu


def _assign(B, H, nc, fracs, g):
    imp = torch.rand((B, H, nc), generator=g)
    order = imp.argsort(-1, descending=True).to(torch.int32)
    out, a = [], 0
    for bits, f in zip((8, 4, 2), fracs):
        m = int(round(f * nc))
        if m:
            out.append((bits, order[..., a:a + m].contiguous()))
        a += m
    return out


def _rotation(d, dtype):
    return torch.from_numpy(os_.rotation_matrix(d)).to(dtype)


def _oracle(st, packed, q, qpos, scaling, b):
    """oracle.strata_attend for sequence b, query token by token over its visible exact rows."""
    d = q.shape[-1]
    B = st.K.shape[0]
    pick = (lambda x: x) if B == 1 else (lambda x: x[b])
    tiers = []
    for t in packed["tiers"]:
        ck = os_.unpack_planar(pick(t["kc"]).cpu().numpy(), t["bits"])
        cv = os_.unpack_planar(pick(t["vc"]).cpu().numpy(), t["bits"])
        tiers.append((t["bits"], ck, pick(t["ks"]).float().cpu().numpy(), cv, pick(t["vs"]).float().cpu().numpy()))
    # the state reads the stored fp16 means in the model dtype, as the reference's does
    mu_k = pick(packed["mu_k"]).to(st.dtype).float().cpu().numpy()
    mu_v = pick(packed["mu_v"]).to(st.dtype).float().cpu().numpy()
    outs = []
    for t, p in enumerate(qpos):
        n_vis = st.n0 + max(0, min(st.n - st.n0, int(p) - st.H + 1))
        ke = st.K[b, :, :n_vis].float().cpu().numpy()
        ve = st.V[b, :, :n_vis].float().cpu().numpy()
        outs.append(os_.strata_attend(q[b:b + 1, :, t:t + 1].float().cpu().numpy(), scaling, ke, ve, tiers, mu_k,
                                      mu_v, os_.rotation_matrix(d)))
    return np.concatenate(outs, 1)[0]                                   # (Tq, Hq, d)


@pytest.mark.parametrize("B,dtype", [(1, torch.float32), (1, torch.bfloat16), (2, torch.bfloat16)])
def test_strata_state_through_decode_controller(B, dtype):
    import kvq
    g = torch.Generator().manual_seed(90 + B)
    Hq, Hkv, T, W, d = 16, 4, 900, 48, 128
    steps = [1, 1, 3]
    T_all = T + sum(steps)
    K = (torch.randn((B, Hkv, T_all, d), generator=g) * 1.3 + 0.2).to(dtype)
    V = torch.randn((B, Hkv, T_all, d), generator=g).to(dtype)
    Q = torch.randn((B, Hq, sum(steps), d), generator=g).to(dtype)
    assign = _assign(B, Hkv, T - W, (0.1, 0.3, 0.4), g)
    cache = kvq.StrataCache.from_context(K[:, :, :T].cuda(), V[:, :, :T].cuda(), window=W, assign=assign)
    packed = kvq.strata_pack(cache)
    assert [t["bits"] for t in packed["tiers"]] == [8, 4, 2]
    st = kvq.StrataState(K[:, :, T - W:T].cuda(), V[:, :, T - W:T].cuda(), packed, 8, T, _rotation(d, dtype).cuda())
    assert st.n == st.n0 == W
    ctl = kvq.DecodeCtl({0: st})
    module = SimpleNamespace(layer_idx=0, scaling=d ** -0.5)
    tol = 2e-3 if dtype == torch.float32 else 1e-2
    pos = T
    with kvq.routed(ctl):
        for t in steps:
            qpos = torch.arange(pos, pos + t)
            ctl.begin(qpos)
            q = Q[:, :, pos - T:pos - T + t].cuda()
            out, none = kvq.router_attention(module, q, K[:, :, pos:pos + t].cuda(), V[:, :, pos:pos + t].cuda(), None)
            assert none is None and out.shape == (B, t, Hq, d) and out.dtype == dtype
            for b in range(B):
                ref = _oracle(st, packed, q, qpos.tolist(), d ** -0.5, b)
                err = float(np.abs(out[b].float().cpu().numpy() - ref).max())
                assert err <= tol, (b, t, err)
            pos += t
    assert st.n == W + sum(steps)
    info = st.check_kernel()
    assert info["kernel"] and info["kernel_rel_err"] <= 2e-2
    es = K.element_size()
    coded = sum(2 * t["kc"].numel() + 2 * t["ks"].numel() * 2 for t in packed["tiers"]) + 4 * packed["counts"].numel()
    coded += 2 * packed["mu_k"].numel() * es
    assert st.context_bytes() == 2 * B * Hkv * W * d * es + coded


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_strata_tier_kernel_partials(bits):
    import kvq
    g = torch.Generator().manual_seed(7 + bits)
    Hkv, n, d, rows = 4, 1000, 128, 12
    codes_k = torch.randint(0, 2 ** bits, (Hkv, n, d), generator=g).to(torch.uint8)
    codes_v = torch.randint(0, 2 ** bits, (Hkv, n, d), generator=g).to(torch.uint8)
    ks = (torch.rand((Hkv, n), generator=g) * 0.05 + 0.01).to(torch.float16)
    vs = (torch.rand((Hkv, n), generator=g) * 0.05 + 0.01).to(torch.float16)
    t = {"bits": bits, "n": n, "kc": kvq.pack_planar(codes_k.cuda(), bits), "ks": ks.cuda(),
         "vc": kvq.pack_planar(codes_v.cuda(), bits), "vs": vs.cuda()}
    qr = torch.randn((Hkv, rows, d), generator=g) * 0.3
    qb = torch.randn((Hkv, rows), generator=g)
    m, l, acc, z = kvq.strata_tier_kernel(qr.cuda(), qb.cuda(), t)
    cdiv = lambda a, b: -(-a // b)
    S = max(1, min(cdiv(n, 64), cdiv(512, Hkv * cdiv(rows, 16))))
    S = cdiv(n, cdiv(cdiv(n, S), 64) * 64)
    assert m.shape == (Hkv, S, rows) and acc.shape == (Hkv, S, rows, d) and z.shape == (Hkv, S, rows)
    m, l, acc, z = (x.double().cpu().numpy() for x in (m, l, acc, z))
    M = m.max(1)
    w = np.exp(m - M[:, None])
    L = (w * l).sum(1)
    A = (w[..., None] * (acc + z[..., None])).sum(1)
    mo, lo, ao = os_.tier_partials(qr.numpy(), qb.numpy(), codes_k.numpy(), ks.float().numpy(), codes_v.numpy(),
                                   vs.float().numpy(), bits)
    np.testing.assert_allclose(M, mo, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(L * np.exp(M - mo), lo, rtol=1e-4)
    # fp32 accumulation over 1000 tokens: the error follows the magnitude of the accumulated terms
    # p vs c (codes up to 2^bits - 1, vs <= 0.06), not of the centred result, which cancels
    ref = ao / lo[..., None]
    np.testing.assert_allclose(A / L[..., None], ref, rtol=1e-4, atol=1e-5 * 0.06 * (2 ** bits - 1))
