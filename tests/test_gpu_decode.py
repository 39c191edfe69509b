"""Split-K packed-KIVI decode on the GPU against the float64 CPU oracle.

Bar: max-abs-err <= 2e-3 for the fp32 configuration, <= 1e-2 for bf16.
Cases: the full C1 configuration, a reduced C2 (B=2, T=2176, heavy-tailed keys), GQA widths
1/2/4/8, value groups 32/64/128, packed counts that end mid-chunk, forced tiny splits (empty
wavefronts), exact-row-only and packed-only caches, and Tq > 1 with causal exact rows.
"""
import numpy as np
import pytest
import torch

import oracle.kivi as ok
from oracle.attention import chunked_attention, kivi_decode_reference

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 2e-3, torch.bfloat16: 1e-2, torch.float16: 1e-2}


def _oracle(q, K, V, scaling, window, gk, gv):
    Kf, Vf, qf = K.float().cpu().numpy(), V.float().cpu().numpy(), q.float().cpu().numpy()
    T = K.shape[2]
    n_q = T - window
    kq = ok.kivi_quant(Kf, 4, gk, True, 0)
    vq = ok.kivi_quant(Vf, 4, gv, False, 0)
    return kivi_decode_reference(qf, scaling, Kf[:, :, n_q:], Vf[:, :, n_q:], kq["codes"], kq["lo"],
                                 kq["scale"], vq["codes"], vq["lo"], vq["scale"], gk, gv, n_q)


def _run(B, Hq, Hkv, T, window, gk, gv, dtype, seed, split_tokens=0, heavy=False, outlier=False):
    import kvq
    g = torch.Generator().manual_seed(seed)
    d = 128
    K = torch.randn((B, Hkv, T, d), generator=g)
    V = torch.randn((B, Hkv, T, d), generator=g)
    q = torch.randn((B, Hq, 1, d), generator=g)
    if heavy:
        from kvq.synth import student_t3
        K *= student_t3((B, Hkv, 1, d), g, "cpu").abs()
    if outlier:
        K[..., torch.randperm(d, generator=g)[:4]] *= 10.0
    q, K, V = q.to(dtype), K.to(dtype), V.to(dtype)
    scaling = d ** -0.5
    cache = kvq.PackedKIVICache.from_context(K.cuda(), V.cuda(), window=window, group_k=gk, group_v=gv)
    out = kvq.kivi_decode(q.cuda(), scaling, cache, split_tokens=split_tokens)
    torch.cuda.synchronize()
    ref = _oracle(q, K, V, scaling, window, gk, gv)
    err = float(np.abs(out.float().cpu().numpy() - ref).max())
    return err, out, ref


def test_c1_full_config_fp32():
    from kvq.synth import C1, decode_inputs
    import kvq
    q, K, V = decode_inputs(C1, "cpu")
    cache = kvq.PackedKIVICache.from_context(K.cuda(), V.cuda(), window=C1.window, group_k=C1.group_k,
                                             group_v=C1.group_v)
    out = kvq.kivi_decode(q.cuda(), C1.d ** -0.5, cache)
    ref = _oracle(q, K, V, C1.d ** -0.5, C1.window, C1.group_k, C1.group_v)
    err = float(np.abs(out.cpu().numpy() - ref).max())
    print(f"C1 max-abs-err {err:.3e}")
    assert err <= 2e-3


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_c2_reduced_bf16_heavy_tails(dtype):
    err, _, _ = _run(2, 32, 8, 2048 + 128, 128, 64, 64, dtype, seed=11, heavy=True)
    print(f"C2-reduced {dtype} max-abs-err {err:.3e}")
    assert err <= TOL[dtype]


@pytest.mark.parametrize("Hq,gv", [(8, 32), (16, 64), (32, 128), (64, 64), (64, 32), (24, 64)])
def test_gqa_widths_and_value_groups(Hq, gv):
    err, _, _ = _run(1, Hq, 8, 1000, 37, 32, gv, torch.float32, seed=Hq + gv, outlier=True)
    assert err <= 2e-3, err


@pytest.mark.parametrize("split", [128, 256, 512])
def test_forced_small_splits(split):
    # 997 packed tokens: last chunk partial, several wavefronts of the last split empty
    err, _, _ = _run(2, 32, 8, 997 + 64, 64, 32, 64, torch.float32, seed=split, split_tokens=split)
    assert err <= 2e-3, err


def test_exact_rows_only_and_packed_only():
    err, _, _ = _run(1, 32, 8, 300, 300, 64, 64, torch.float32, seed=1)     # n_q = 0
    assert err <= 2e-3, err
    err, _, _ = _run(2, 32, 8, 2500, 2500, 64, 64, torch.bfloat16, seed=6)  # n_q = 0, exact-row blocks
    assert err <= TOL[torch.bfloat16], err
    err, _, _ = _run(1, 32, 8, 1024, 0, 64, 64, torch.float32, seed=2)      # n_exact = 0
    assert err <= 2e-3, err
    err, _, _ = _run(1, 32, 8, 3000, 700, 64, 64, torch.float32, seed=3)    # window in the merge
    assert err <= 2e-3, err
    err, _, _ = _run(1, 32, 8, 3000, 2000, 64, 64, torch.float32, seed=4)   # exact-row blocks
    assert err <= 2e-3, err


@pytest.mark.parametrize("W", [40, 400, 1500])
def test_multi_token_queries_causal_exact_rows(W):
    """560 packed tokens over 4 KV heads give at most 5 packed splits per head: a window of
    40 (+2 appended) rows is attended inside the packed splits (9 rows each), 400 inside the
    merge, 1500 by exact-row blocks; every placement applies the causal visibility."""
    import kvq
    g = torch.Generator().manual_seed(5 + W)
    B, Hq, Hkv, Tq, d = 1, 8, 4, 2, 128
    T = 560 + W
    K = torch.randn((B, Hkv, T + Tq, d), generator=g)
    V = torch.randn((B, Hkv, T + Tq, d), generator=g)
    q = torch.randn((B, Hq, Tq, d), generator=g)
    cache = kvq.PackedKIVICache.from_context(K[:, :, :T].cuda(), V[:, :, :T].cuda(), window=W, group_k=32,
                                             group_v=64, extra_exact=Tq)
    cache.k_exact[:, :, W:W + Tq] = K[:, :, T:].cuda()
    cache.v_exact[:, :, W:W + Tq] = V[:, :, T:].cuda()
    cache.n_exact = W + Tq
    cache.exact_pos = torch.arange(T - W, T + Tq, dtype=torch.int64, device="cuda")
    q_pos = torch.arange(T, T + Tq, dtype=torch.int64, device="cuda")
    out = kvq.kivi_decode(q.cuda(), d ** -0.5, cache, q_pos=q_pos)
    n_q = T - W
    kq = ok.kivi_quant(K[:, :, :T].numpy(), 4, 32, True, 0)
    vq = ok.kivi_quant(V[:, :, :T].numpy(), 4, 64, False, 0)
    kh = ok.kivi_dequant(kq["codes"], kq["lo"], kq["scale"], 32, True)[:, :, :n_q]
    vh = ok.kivi_dequant(vq["codes"][:, :, :n_q], vq["lo"][:, :, :n_q], vq["scale"][:, :, :n_q], 64, False)
    tok = {"k": kh, "v": vh, "b": np.zeros((B, Hkv, n_q)), "tau": np.full(n_q, -1)}
    ref = chunked_attention(q.numpy(), d ** -0.5, np.arange(T, T + Tq), K[:, :, n_q:].numpy(),
                            V[:, :, n_q:].numpy(), np.arange(n_q, T + Tq), np.full(W + Tq, 1 << 40), tok)
    err = float(np.abs(out.cpu().numpy() - ref).max())
    assert err <= 2e-3, err


def test_decode_rejects_cpu_tensors_and_bad_shapes():
    import kvq
    with pytest.raises(kvq.KVQError):
        kvq.kivi_quant(torch.zeros(1, 1, 4, 128), 4, 32, True, 0)
    K = torch.randn(1, 2, 256, 64, device="cuda")
    with pytest.raises((kvq.KVQError, ValueError)):
        c = kvq.PackedKIVICache.from_context(K, K, window=32, group_k=32, group_v=32)
        kvq.kivi_decode(torch.randn(1, 2, 1, 64, device="cuda"), 0.1, c)
