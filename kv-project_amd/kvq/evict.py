"""Eviction path on the GPU: decode-time score accumulation, top-k retention, and the decode over
the retained set (SnapKV-style selection over a packed KIVI cache).

Reference behaviour (STRATA_KV.py):
  * ``snapkv_scores`` (932-954): scores are the softmax probabilities a window of queries gives each
    context token, averaged over those queries and over the query heads of each KV group; the
    recent window is always kept (it gets max + 1).
  * ``topk`` + ``sort`` (975, 1022-1023): the k best positions per KV head, in position order.
Here the queries are decode steps: ``kivi_decode(..., scores=...)`` adds each step's probabilities
of the packed tokens (mean over the group's query heads) to a per-(b, KV head) scores row;
``topk_retain`` keeps the k best packed positions; ``retained_cache`` turns them, dequantised,
plus the exact rows (the recent window, always kept) into a cache the same decode kernel reads.
"""
from __future__ import annotations

from dataclasses import replace

import torch

from . import _lib
from .decode import PackedKIVICache


@torch.no_grad()
def topk_retain(scores: torch.Tensor, k: int) -> torch.Tensor:
    """scores (..., n) float32 on the GPU -> int32 (..., k): the positions of the k largest scores of
    each row in increasing order (lowest positions kept among scores tied at the k-th)."""
    _lib.require_gpu(scores)
    if scores.dtype != torch.float32:
        raise TypeError("scores must be float32")
    n = scores.shape[-1]
    if not 0 <= k <= n:
        raise ValueError("need 0 <= k <= n")
    rows = scores.reshape(-1, n)
    if rows.stride(-1) != 1:
        rows = rows.contiguous()
    idx = torch.empty(rows.shape[0], k, dtype=torch.int32, device=scores.device)
    _lib.call("kvq_topk_retain", rows.data_ptr(), rows.shape[0], n, rows.stride(0), k, idx.data_ptr(), k,
              _lib.stream_of(scores))
    return idx.reshape(scores.shape[:-1] + (k,))


@torch.no_grad()
def gather_dequant(cache: PackedKIVICache, idx: torch.Tensor, dtype: torch.dtype):
    """Dequantised key / value rows (B, Hkv, k, d) of ``dtype`` at packed positions idx (B, Hkv, k)
    (code * scale + lo in fp32, as kivi_quant's xhat; STRATA_KV.py:855)."""
    _lib.require_gpu(idx)
    B, H = cache.kc.shape[:2]
    d = cache.kc.shape[3] * 2
    if idx.shape[:2] != (B, H) or idx.dtype != torch.int32:
        raise ValueError("idx must be int32 (B, Hkv, k)")
    idx = idx.contiguous()
    k = idx.shape[2]
    ko = torch.empty((B, H, k, d), dtype=dtype, device=idx.device)
    vo = torch.empty_like(ko)
    _lib.call("kvq_kivi_gather_dequant", cache.kc.data_ptr(), cache.k_lo.data_ptr(), cache.k_sc.data_ptr(),
              cache.vc.data_ptr(), cache.vmeta.data_ptr(), cache.cap_t, cache.n_q, cache.group_k, cache.group_v,
              B * H, d, idx.data_ptr(), k, k, ko.data_ptr(), vo.data_ptr(), _lib.DTYPE_CODE[dtype], k * d,
              _lib.stream_of(idx))
    return ko, vo


@torch.no_grad()
def retained_cache(cache: PackedKIVICache, idx: torch.Tensor) -> PackedKIVICache:
    """The cache after eviction: the retained packed positions idx (B, Hkv, k), dequantised, followed
    by the cache's exact rows (the recent window, always kept) -- all read as exact rows by the
    decode kernel (n_q = 0)."""
    ko, vo = gather_dequant(cache, idx, cache.k_exact.dtype)
    ke = torch.cat([ko, cache.k_exact[:, :, :cache.n_exact]], 2).contiguous()
    ve = torch.cat([vo, cache.v_exact[:, :, :cache.n_exact]], 2).contiguous()
    return replace(cache, n_q=0, k_exact=ke, v_exact=ve, n_exact=ke.shape[2], exact_pos=None, ring=False)
