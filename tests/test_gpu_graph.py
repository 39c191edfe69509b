"""The decode step is HIP-graph capturable: every replay (with eager work and synchronisations in
between, and changed inputs) equals the eager result."""
import pytest
import torch

pytestmark = pytest.mark.gpu


def test_graph_replays_match_eager():
    import kvq
    g = torch.Generator(device="cuda").manual_seed(3)
    B, Hq, Hkv, T, d = 2, 32, 8, 1500, 128
    K = torch.randn((B, Hkv, T, d), generator=g, device="cuda").bfloat16()
    V = torch.randn((B, Hkv, T, d), generator=g, device="cuda").bfloat16()
    cache = kvq.PackedKIVICache.from_context(K, V, window=128, group_k=64, group_v=64)
    q = torch.randn((B, Hq, 1, d), generator=g, device="cuda").bfloat16()
    out = torch.empty((B, 1, Hq, d), dtype=torch.bfloat16, device="cuda")
    ws = torch.zeros((kvq.workspace_floats(B, Hq, Hkv, 1, d, cache.n_q, cache.n_exact, 64, 64),), device="cuda")
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        kvq.kivi_decode(q, d ** -0.5, cache, out=out, workspace=ws)
    torch.cuda.current_stream().wait_stream(side)
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr):
        kvq.kivi_decode(q, d ** -0.5, cache, out=out, workspace=ws)
    for it in range(4):
        q.copy_(torch.randn((B, Hq, 1, d), generator=g, device="cuda").bfloat16())
        _ = (K.float() * 2).sum()                      # unrelated eager work between replays
        torch.cuda.synchronize()
        gr.replay()
        torch.cuda.synchronize()
        ref = kvq.kivi_decode(q, d ** -0.5, cache)
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"replay {it} differs from eager"
