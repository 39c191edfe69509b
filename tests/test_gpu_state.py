"""The drop-in decode boundary on the GPU: KIVIState through DecodeCtl and router_attention, as
the reference's generation loop drives LayerState (STRATA_KV.py:2817-2834, 682-719), against the
float64 oracle (chunked_attention over the KIVI entries, STRATA_KV.py:641-675, 801-823).

A prefilled context of H tokens, then two decode steps of one token each (append + attend), then
one two-token step (causal among the appended rows).  Bar: 2e-3 (fp32), 1e-2 (bf16).
"""
from types import SimpleNamespace

import numpy as np
import pytest
import torch

import oracle.kivi as ok
from oracle.attention import chunked_attention

pytestmark = pytest.mark.gpu


def _oracle_step(q, K_all, V_all, H, W, gk, gv, qpos, scaling):
    """Reference attention after the context H (quantised below H - W) and appended rows."""
    Kc, Vc = K_all[:, :, :H].astype(np.float64), V_all[:, :, :H].astype(np.float64)
    n_q = H - W
    kq = ok.kivi_quant(Kc, 4, gk, True, 0)
    vq = ok.kivi_quant(Vc, 4, gv, False, 0)
    kh = ok.kivi_dequant(kq["codes"], kq["lo"], kq["scale"], gk, True)[:, :, :n_q]
    vh = ok.kivi_dequant(vq["codes"][:, :, :n_q], vq["lo"][:, :, :n_q], vq["scale"][:, :, :n_q], gv, False)
    tok = {"k": kh, "v": vh, "b": np.zeros(kh.shape[:3]), "tau": np.full(n_q, -1)}
    n_all = K_all.shape[2]
    return chunked_attention(q, scaling, np.asarray(qpos), K_all[:, :, n_q:n_all], V_all[:, :, n_q:n_all],
                             np.arange(n_q, n_all), np.full(n_all - n_q, 1 << 40), tok)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_kivi_state_through_decode_controller(dtype):
    import kvq
    g = torch.Generator().manual_seed(11)
    B, Hq, Hkv, H, W, d, gk, gv = 2, 16, 4, 900, 64, 128, 32, 64
    steps = [1, 1, 2]
    T_all = H + sum(steps)
    K = torch.randn((B, Hkv, T_all, d), generator=g).to(dtype)
    V = torch.randn((B, Hkv, T_all, d), generator=g).to(dtype)
    Q = torch.randn((B, Hq, sum(steps), d), generator=g).to(dtype)
    st = kvq.KIVIState(K[:, :, :H].cuda(), V[:, :, :H].cuda(), window=W, group_k=gk, group_v=gv, extra=8)
    assert st.n == st.n0 == H
    ctl = kvq.DecodeCtl({0: st})
    module = SimpleNamespace(layer_idx=0, scaling=d ** -0.5)
    tol = 2e-3 if dtype == torch.float32 else 1e-2
    kn, vn = K.float().numpy(), V.float().numpy()
    pos = H
    with kvq.routed(ctl):
        for t in steps:
            qpos = torch.arange(pos, pos + t)
            ctl.begin(qpos)
            q = Q[:, :, pos - H:pos - H + t]
            out, none = kvq.router_attention(module, q.cuda(), K[:, :, pos:pos + t].cuda(),
                                             V[:, :, pos:pos + t].cuda(), None)
            assert none is None and out.shape == (B, t, Hq, d) and out.dtype == dtype
            ref = _oracle_step(q.float().numpy(), kn[:, :, :pos + t], vn[:, :, :pos + t], H, W, gk, gv,
                               qpos.numpy(), d ** -0.5)
            err = float(np.abs(out.float().cpu().numpy() - ref).max())
            assert err <= tol, (t, err)
            pos += t
    assert st.n == T_all
    info = st.check_kernel()
    assert info["kernel"] and info["kernel_rel_err"] <= 2e-2
    # context bytes: 4-bit codes + fp16 metadata of the quantised rows, exact window rows
    n_q = H - W
    expect = (2 * B * Hkv * n_q * d // 2 + B * Hkv * (-(-n_q // gk)) * d * 4 + B * Hkv * n_q * (d // gv) * 4
              + 2 * B * Hkv * W * d * K.element_size())
    assert st.context_bytes() == expect


def test_kivi_state_buffer_exhausted():
    import kvq
    K = torch.randn((1, 2, 256, 128), device="cuda")
    st = kvq.KIVIState(K, K, window=32, group_k=32, group_v=32, extra=1)
    st.append(K[:, :, :1], K[:, :, :1], [256])
    with pytest.raises(RuntimeError, match="decode buffer exhausted"):
        st.append(K[:, :, :1], K[:, :, :1], [257])


@pytest.mark.parametrize("dtype,chunk", [(torch.bfloat16, None), (torch.float32, 3)])
def test_question_step_of_many_tokens(dtype, chunk):
    """The reference's run_tokens feeds a whole question in one step (STRATA_KV.py:3238-3248): 40
    tokens at rep 4 through DecodeCtl (query pieces of 2 tokens, or of the controller's chunk),
    causal among the appended rows, then a one-token step; against the oracle."""
    import kvq
    g = torch.Generator().manual_seed(40)
    B, Hq, Hkv, H, W, d, gk, gv = 1, 32, 8, 700, 64, 128, 64, 64
    steps = [40, 1]
    T_all = H + sum(steps)
    K = torch.randn((B, Hkv, T_all, d), generator=g).to(dtype)
    V = torch.randn((B, Hkv, T_all, d), generator=g).to(dtype)
    Q = torch.randn((B, Hq, sum(steps), d), generator=g).to(dtype)
    st = kvq.KIVIState(K[:, :, :H].cuda(), V[:, :, :H].cuda(), window=W, group_k=gk, group_v=gv, extra=48)
    ctl = kvq.DecodeCtl({0: st}, chunk=chunk)
    module = SimpleNamespace(layer_idx=0, scaling=d ** -0.5)
    tol = 2e-3 if dtype == torch.float32 else 1e-2
    kn, vn = K.float().numpy(), V.float().numpy()
    pos = H
    with kvq.routed(ctl):
        for t in steps:
            qpos = torch.arange(pos, pos + t)
            ctl.begin(qpos)
            q = Q[:, :, pos - H:pos - H + t]
            out, _ = kvq.router_attention(module, q.cuda(), K[:, :, pos:pos + t].cuda(), V[:, :, pos:pos + t].cuda(),
                                          None)
            assert out.shape == (B, t, Hq, d)
            ref = _oracle_step(q.float().numpy(), kn[:, :, :pos + t], vn[:, :, :pos + t], H, W, gk, gv,
                               qpos.numpy(), d ** -0.5)
            err = float(np.abs(out.float().cpu().numpy() - ref).max())
            assert err <= tol, (t, err)
            pos += t

