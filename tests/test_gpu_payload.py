"""Wire format of a packed KIVI layer (PackedKIVICache.export / KIVIState.payload, libkvq
kvq_kivi_export) against the oracle's payload sections (payload_bytes, STRATA_KV.py:2736-2769):
byte for byte, for a prefilled cache, a streaming (ring) cache after a key group of appends, and
the state's measured bytes against the analytic bits."""
import numpy as np
import pytest
import torch

from oracle.kivi import kivi_payload_sections, kivi_state_bits

pytestmark = pytest.mark.gpu


def _raw(x: torch.Tensor) -> bytes:
    return x.contiguous().view(torch.uint8).cpu().numpy().tobytes()


def _want(K, V, n_q, gk, gv, exact_k, exact_v):
    """Oracle sections, then the exact rows as fp16 (the reference's .half())."""
    sec = kivi_payload_sections(K.float().numpy(), V.float().numpy(), 4, gk, gv, n_q)
    return b"".join(sec) + _raw(exact_k.to(torch.float16)) + _raw(exact_v.to(torch.float16))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("T,W,gk,gv", [(300, 44, 64, 64), (200, 8, 32, 128), (64, 64, 64, 32)])
def test_export_prefilled_cache(dtype, T, W, gk, gv):
    import kvq
    g = torch.Generator().manual_seed(T + W)
    K = torch.randn((2, 3, T, 128), generator=g).to(dtype)
    V = torch.randn((2, 3, T, 128), generator=g).to(dtype)
    cache = kvq.PackedKIVICache.from_context(K.cuda(), V.cuda(), window=W, group_k=gk, group_v=gv)
    got = cache.export().cpu().numpy().tobytes()
    n_q = T - W
    want = _want(K, V, n_q, gk, gv, K[:, :, n_q:], V[:, :, n_q:])
    assert len(got) == len(want) == cache.wire_bytes()
    assert got == want


def test_export_ring_cache_after_appends():
    import kvq
    g = torch.Generator().manual_seed(5)
    T, W, gk = 320, 64, 64
    K = torch.randn((2, 2, T + gk, 128), generator=g).to(torch.bfloat16)
    V = torch.randn((2, 2, T + gk, 128), generator=g).to(torch.bfloat16)
    cache = kvq.PackedKIVICache.from_context(K[:, :, :T].cuda(), V[:, :, :T].cuda(), window=W, group_k=gk, group_v=gk,
                                             ring=True, extra_tokens=2 * gk)
    for t in range(T, T + gk):
        cache.append(K[:, :, t:t + 1].cuda(), V[:, :, t:t + 1].cuda())
    n_q = T + gk - W
    assert cache.n_q == n_q
    got = cache.export().cpu().numpy().tobytes()
    want = _want(K, V, n_q, gk, gk, K[:, :, n_q:], V[:, :, n_q:])
    assert got == want


def test_state_payload_is_the_analytic_bits():
    import kvq
    g = torch.Generator().manual_seed(11)
    K = torch.randn((2, 4, 576, 128), generator=g).to(torch.bfloat16)
    V = torch.randn((2, 4, 576, 128), generator=g).to(torch.bfloat16)
    st = kvq.KIVIState(K.cuda(), V.cuda(), window=64, group_k=64, group_v=64, extra=8)
    st.append(torch.zeros((2, 4, 2, 128), dtype=torch.bfloat16).cuda(), torch.zeros((2, 4, 2, 128), dtype=torch.bfloat16).cuda(),
              [576, 577])                                              # appended rows are not context
    assert st.payload().numel() == st.payload_bytes()
    assert st.payload_bytes() * 8 == 2 * 4 * kivi_state_bits(512, 64, 128, 4, 64)
    assert kvq.payload_bytes({0: st, 1: st}) == 2 * st.payload_bytes()
