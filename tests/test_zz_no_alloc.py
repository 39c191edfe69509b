"""The allocation-free decode entry point (kvq_kivi_decode_noalloc, static per-GPU scratch) against
kvq_kivi_decode with a caller's workspace, through the C ABI: two calls in a row, the second on a
smaller step (fewer (b, h), a shorter context, a different split plan), each bit-identical to the
workspace entry point (same kernels, same plan, no atomics).  Then a scored step (phases 7) whose
accumulated scores are bit-identical too, and a query that does not match the cache, rejected on
the host."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _cache(B, Hkv, T, W, seed, dtype=torch.bfloat16):
    import kvq
    g = torch.Generator().manual_seed(seed)
    K = torch.randn((B, Hkv, T, 128), generator=g).to(dtype)
    V = torch.randn((B, Hkv, T, 128), generator=g).to(dtype)
    return kvq.PackedKIVICache.from_context(K.cuda(), V.cuda(), window=W, group_k=64, group_v=64), g


def test_noalloc_matches_workspace_entry_point():
    import kvq
    for B, Hq, Hkv, T, W, seed in ((4, 32, 8, 8192, 128, 1), (2, 16, 4, 3000, 100, 2)):
        cache, g = _cache(B, Hkv, T, W, seed)
        q = torch.randn((B, Hq, 1, 128), generator=g).to(torch.bfloat16).cuda()
        ref = kvq.kivi_decode(q, 128 ** -0.5, cache)
        out = torch.full_like(ref, float("nan"))
        got = kvq.kivi_decode(q, 128 ** -0.5, cache, out=out, static_scratch=True)
        torch.cuda.synchronize()
        assert got.data_ptr() == out.data_ptr()
        print(f"noalloc B={B} Hq={Hq} Hkv={Hkv} T={T}: max |diff| "
              f"{float((got.float() - ref.float()).abs().max()):.3e}", flush=True)
        assert torch.equal(got, ref)


def test_noalloc_scored_step_and_limit():
    import kvq
    B, Hq, Hkv, T, W = 2, 8, 2, 2000, 64
    cache, g = _cache(B, Hkv, T, W, 3, torch.float32)
    n_q = T - W
    s_ref = torch.zeros((B, Hkv, n_q), dtype=torch.float32, device="cuda")
    s_got = torch.zeros_like(s_ref)
    for _ in range(2):
        q = torch.randn((B, Hq, 1, 128), generator=g).cuda()
        ref = kvq.kivi_decode(q, 128 ** -0.5, cache, scores=s_ref, score_weight=0.25)
        got = kvq.kivi_decode(q, 128 ** -0.5, cache, scores=s_got, score_weight=0.25, static_scratch=True)
        assert torch.equal(got, ref)
    assert torch.equal(s_got, s_ref)
    # a query whose batch does not match the cache is refused on the host before any launch (the
    # kernels would index the cache by q's batch); the scratch limit itself is checked on the CPU
    # with null pointers (test_abi.py::test_noalloc_rejects_steps_beyond_the_static_scratch)
    q = torch.zeros((4096, Hq, 1, 128), device="cuda")
    with pytest.raises(ValueError, match="does not match the cache"):
        kvq.kivi_decode(q, 128 ** -0.5, cache, static_scratch=True)
