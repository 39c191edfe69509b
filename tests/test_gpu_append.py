"""Streaming append (fused quantise + pack of the token leaving the window) against the one-shot
compression of the whole sequence: codes and metadata bit-exact, decode outputs equal to the
oracle within the bar."""
import numpy as np
import pytest
import torch

import oracle.kivi as ok
from oracle.attention import kivi_decode_reference

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype,gk,gv,W,T0,N", [(torch.bfloat16, 64, 64, 128, 640, 200),
                                                 (torch.float32, 32, 32, 64, 100, 150),
                                                 (torch.float16, 64, 128, 64, 64, 130)])
def test_streaming_append_matches_one_shot(dtype, gk, gv, W, T0, N):
    import kvq
    g = torch.Generator().manual_seed(T0 + N)
    B, Hq, Hkv, d = 2, 16, 4, 128
    K = torch.randn((B, Hkv, T0 + N, d), generator=g).to(dtype)
    V = torch.randn((B, Hkv, T0 + N, d), generator=g).to(dtype)
    q = torch.randn((B, Hq, 1, d), generator=g).to(dtype)
    Kc, Vc = K.cuda(), V.cuda()
    st = kvq.PackedKIVICache.from_context(Kc[:, :, :T0], Vc[:, :, :T0], window=W, group_k=gk, group_v=gv,
                                          extra_tokens=N + gk, ring=True)
    for i in range(N):
        st.append(Kc[:, :, T0 + i:T0 + i + 1], Vc[:, :, T0 + i:T0 + i + 1])
    T = T0 + N
    n_q = T - W
    assert st.n_q == n_q and st.n_exact == W
    full = kvq.PackedKIVICache.from_context(Kc, Vc, window=W, group_k=gk, group_v=gv)
    np.testing.assert_array_equal(st.kc[:, :, :n_q].cpu().numpy(), full.kc[:, :, :n_q].cpu().numpy())
    ng = -(-n_q // gk)
    np.testing.assert_array_equal(st.k_lo[:, :, :ng].cpu().numpy(), full.k_lo[:, :, :ng].cpu().numpy())
    np.testing.assert_array_equal(st.k_sc[:, :, :ng].cpu().numpy(), full.k_sc[:, :, :ng].cpu().numpy())
    np.testing.assert_array_equal(kvq.v_untile(st.vc, n_q).cpu().numpy(), kvq.v_untile(full.vc, n_q).cpu().numpy())
    # value metadata of the valid tokens (slots of later tokens may differ: not yet written)
    sm, fm = st.vmeta.cpu().numpy(), full.vmeta.cpu().numpy()
    for tok in list(range(0, n_q, 37)) + [n_q - 1]:
        c, u = divmod(tok, 32)
        p = 8 * ((u % 16) // 4) + 4 * (u // 16) + u % 4
        np.testing.assert_array_equal(sm[:, :, c, :, p], fm[:, :, c, :, p])
    # ring holds positions T-W .. T-1 at slot p % W
    slots = torch.arange(T - W, T) % W
    np.testing.assert_array_equal(st.k_exact[:, :, slots].cpu().float().numpy(), K[:, :, T - W:].float().numpy())
    # decode over the streamed cache == oracle over the one-shot quantisation
    out = kvq.kivi_decode(q.cuda(), d ** -0.5, st).float().cpu().numpy()
    Kf, Vf = K.float().numpy(), V.float().numpy()
    kq, vq = ok.kivi_quant(Kf, 4, gk, True, 0), ok.kivi_quant(Vf, 4, gv, False, 0)
    ref = kivi_decode_reference(q.float().numpy(), d ** -0.5, Kf[:, :, n_q:], Vf[:, :, n_q:], kq["codes"], kq["lo"],
                                kq["scale"], vq["codes"], vq["lo"], vq["scale"], gk, gv, n_q)
    tol = 2e-3 if dtype == torch.float32 else 1e-2
    assert np.abs(out - ref).max() <= tol


def test_append_capacity_exhausted():
    import kvq
    K = torch.randn((1, 2, 128, 128), device="cuda", dtype=torch.bfloat16)
    st = kvq.PackedKIVICache.from_context(K, K, window=64, group_k=64, group_v=64, extra_tokens=0, ring=True)
    with pytest.raises(RuntimeError):
        for _ in range(200):
            st.append(K[:, :, :1], K[:, :, :1])


def test_append_fills_capacity_to_last_row():
    """The packed capacity fills to its last row: with cap_t = 128 rows, appends continue until token
    127 leaves the window (its key group was written when token 64 left), the next append raises,
    and the full cache decodes as the one-shot compression of the same 192 tokens."""
    import kvq
    g = torch.Generator().manual_seed(5)
    B, Hq, Hkv, d, W, gk, gv, T0 = 1, 8, 2, 128, 64, 64, 64, 128
    K = torch.randn((B, Hkv, 192, d), generator=g).to(torch.bfloat16)
    V = torch.randn((B, Hkv, 192, d), generator=g).to(torch.bfloat16)
    q = torch.randn((B, Hq, 1, d), generator=g).to(torch.bfloat16)
    Kc, Vc = K.cuda(), V.cuda()
    st = kvq.PackedKIVICache.from_context(Kc[:, :, :T0], Vc[:, :, :T0], window=W, group_k=gk, group_v=gv,
                                          extra_tokens=64, ring=True)
    assert st.cap_t == 128
    for i in range(T0, 192):
        st.append(Kc[:, :, i:i + 1], Vc[:, :, i:i + 1])
    assert st.n_q == st.cap_t == 128
    with pytest.raises(RuntimeError, match="exhausted"):
        st.append(Kc[:, :, :1], Vc[:, :, :1])
    out = kvq.kivi_decode(q.cuda(), d ** -0.5, st).float().cpu().numpy()
    Kf, Vf = K.float().numpy(), V.float().numpy()
    kq, vq = ok.kivi_quant(Kf, 4, gk, True, 0), ok.kivi_quant(Vf, 4, gv, False, 0)
    ref = kivi_decode_reference(q.float().numpy(), d ** -0.5, Kf[:, :, 128:], Vf[:, :, 128:], kq["codes"], kq["lo"],
                                kq["scale"], vq["codes"], vq["lo"], vq["scale"], gk, gv, 128)
    assert np.abs(out - ref).max() <= 1e-2
