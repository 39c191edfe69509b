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


SNAPKV_WINDOW, SNAPKV_KERNEL = 64, 5           # the reference's defaults (STRATA_KV.py:418-419)


def _window_rows(q, H: int, w: int) -> torch.Tensor:
    """The observation queries at positions H - w .. H - 1: q (B, Hq, >= H, d), or an object with
    the reference's QRows.at(positions) (q_at, STRATA_KV.py:3173-3175)."""
    pos = torch.arange(H - w, H)
    if hasattr(q, "at"):
        return q.at(pos)
    return q[:, :, H - w:H]


@torch.no_grad()
def snapkv_scores(q, k: torch.Tensor, H: int, scaling: float, cfg=None, out: torch.Tensor | None = None,
                  workspace: torch.Tensor | None = None) -> torch.Tensor:
    """SnapKV scores (STRATA_KV.py:932-954) on the device: q (B, Hq, >= H, d) (or QRows), k (B, Hkv, >= H, d)
    -> (B, Hkv, H) float32.  The last SNAPKV_WINDOW context queries attend causally to the keys [0, H);
    the probabilities of the non-window keys, averaged over those queries and over the query heads of
    each KV group and pooled by avg_pool1d(SNAPKV_KERNEL, padding // 2), are the scores; the window gets
    the largest score + 1.  ``cfg``: any object with SNAPKV_WINDOW / SNAPKV_KERNEL (the reference's
    Config), else the reference's defaults 64 / 5."""
    w = int(getattr(cfg, "SNAPKV_WINDOW", SNAPKV_WINDOW))
    kern = int(getattr(cfg, "SNAPKV_KERNEL", SNAPKV_KERNEL))
    qw = _window_rows(q, H, w)
    _lib.require_gpu(qw, k)
    B, Hq, _, d = qw.shape
    Hkv = k.shape[1]
    if k.shape[2] < H or qw.shape[2] != w or k.dtype != qw.dtype:
        raise ValueError("need k with >= H rows and the window queries in k's dtype")
    if qw.stride(-1) != 1:
        qw = qw.contiguous()
    if k.stride(-1) != 1:
        k = k.contiguous()
    dt = _lib.DTYPE_CODE[k.dtype]
    if out is None:
        out = torch.empty((B, Hkv, H), dtype=torch.float32, device=k.device)
    elif out.dtype != torch.float32 or tuple(out.shape) != (B, Hkv, H) or not out.is_contiguous():
        raise ValueError("out must be a contiguous float32 (B, Hkv, H) tensor")
    if workspace is None:
        need = _lib.load().kvq_snapkv_scores_workspace(B, Hq, Hkv, w, H, dt)
        if need < 0:
            raise _lib.KVQError("kvq_snapkv_scores_workspace rejected the shape")
        workspace = torch.empty((need,), dtype=torch.float32, device=k.device)
    _lib.call("kvq_snapkv_scores", qw.data_ptr(), dt, qw.stride(0), qw.stride(1), qw.stride(2), k.data_ptr(),
              k.stride(0), k.stride(1), k.stride(2), B, Hq, Hkv, d, w, H, float(scaling), kern, out.data_ptr(),
              workspace.data_ptr(), workspace.numel(), _lib.stream_of(k))
    return out


@torch.no_grad()
def topk_workspace_words(rows: int, n: int) -> int:
    """32-bit words of workspace the split selection needs for ``rows`` rows of n scores (0 when
    such rows take the one-workgroup kernels: n <= 4096, n > 2^24 or more than 65535 rows)."""
    return int(_lib.load().kvq_topk_retain_workspace(rows, n))


def topk_retain(scores: torch.Tensor, k: int, out: torch.Tensor | None = None, *,
                workspace: torch.Tensor | None = None, split: bool = True) -> torch.Tensor:
    """scores (..., n) float32 on the GPU -> int32 (..., k): the positions of the k largest scores of
    each row in increasing order (lowest positions kept among scores tied at the k-th).  ``out``: a
    contiguous int32 (..., k) tensor to write them into.  ``split`` (default) spreads each row over
    several workgroups (kvq_topk_retain_ws) where topk_workspace_words > 0, with ``workspace`` (a
    contiguous 32-bit tensor of at least that many elements, 256-byte aligned) or one from torch's
    allocator; False keeps one workgroup per row (kvq_topk_retain).  Both give the same result."""
    _lib.require_gpu(scores)
    if scores.dtype != torch.float32:
        raise TypeError("scores must be float32")
    n = scores.shape[-1]
    if not 0 <= k <= n:
        raise ValueError("need 0 <= k <= n")
    rows = scores.reshape(-1, n)
    if rows.stride(-1) != 1:
        rows = rows.contiguous()
    if out is None:
        idx = torch.empty(rows.shape[0], k, dtype=torch.int32, device=scores.device)
    else:
        if out.dtype != torch.int32 or out.shape != scores.shape[:-1] + (k,) or not out.is_contiguous():
            raise ValueError("out must be a contiguous int32 (..., k) tensor")
        idx = out.view(rows.shape[0], k)
    words = topk_workspace_words(rows.shape[0], n) if split else 0
    if words > 0:
        if workspace is None:
            workspace = torch.empty(words, dtype=torch.int32, device=scores.device)
        elif (workspace.element_size() != 4 or not workspace.is_contiguous() or workspace.numel() < words
              or workspace.device != scores.device):
            raise ValueError(f"workspace must be a contiguous 32-bit tensor of >= {words} elements on the scores' device")
        _lib.call("kvq_topk_retain_ws", rows.data_ptr(), rows.shape[0], n, rows.stride(0), k, idx.data_ptr(), k,
                  workspace.data_ptr(), workspace.numel(), _lib.stream_of(scores))
    else:
        _lib.call("kvq_topk_retain", rows.data_ptr(), rows.shape[0], n, rows.stride(0), k, idx.data_ptr(), k,
                  _lib.stream_of(scores))
    return idx.reshape(scores.shape[:-1] + (k,))


@torch.no_grad()
def gather_dequant(cache: PackedKIVICache, idx: torch.Tensor, dtype: torch.dtype, out=None):
    """Dequantised key / value rows (B, Hkv, k, d) of ``dtype`` at packed positions idx (B, Hkv, k)
    (code * scale + lo in fp32, as kivi_quant's xhat; STRATA_KV.py:855).  ``out`` = (ko, vo): rows
    [0, k) of the third axis of two (B, Hkv, >= k, d) tensors receive them instead."""
    _lib.require_gpu(idx)
    B, H = cache.kc.shape[:2]
    d = cache.kc.shape[3] * 2
    if idx.shape[:2] != (B, H) or idx.dtype != torch.int32:
        raise ValueError("idx must be int32 (B, Hkv, k)")
    idx = idx.contiguous()
    k = idx.shape[2]
    if out is None:
        ko = torch.empty((B, H, k, d), dtype=dtype, device=idx.device)
        vo = torch.empty_like(ko)
    else:
        ko, vo = out
        if (ko.shape[:2] != (B, H) or ko.shape[2] < k or ko.shape[3] != d or vo.shape != ko.shape
                or ko.dtype != dtype or vo.dtype != dtype or not ko.is_contiguous() or not vo.is_contiguous()):
            raise ValueError("out must be two contiguous (B, Hkv, >= k, d) tensors of dtype")
    _lib.call("kvq_kivi_gather_dequant", cache.kc.data_ptr(), cache.k_lo.data_ptr(), cache.k_sc.data_ptr(),
              cache.vc.data_ptr(), cache.vmeta.data_ptr(), cache.cap_t, cache.n_q, cache.group_k, cache.group_v,
              B * H, d, idx.data_ptr(), k, k, ko.data_ptr(), vo.data_ptr(), _lib.DTYPE_CODE[dtype],
              ko.shape[2] * d, _lib.stream_of(idx))
    return ko, vo


@torch.no_grad()
def retained_cache(cache: PackedKIVICache, idx: torch.Tensor) -> PackedKIVICache:
    """The cache after eviction: the retained packed positions idx (B, Hkv, k), dequantised, followed
    by the cache's exact rows (the recent window, always kept) -- all read as exact rows by the
    decode kernel (n_q = 0).  The gather writes straight into the combined rows."""
    B, H, k = idx.shape
    ne = cache.n_exact
    d = cache.kc.shape[3] * 2
    ke = torch.empty((B, H, k + ne, d), dtype=cache.k_exact.dtype, device=idx.device)
    ve = torch.empty_like(ke)
    gather_dequant(cache, idx, cache.k_exact.dtype, out=(ke, ve))
    if ne > 0:
        ke[:, :, k:].copy_(cache.k_exact[:, :, :ne])
        ve[:, :, k:].copy_(cache.v_exact[:, :, :ne])
    return replace(cache, n_q=0, k_exact=ke, v_exact=ve, n_exact=k + ne, exact_pos=None, ring=False)


@torch.no_grad()
def gather_rows(k: torch.Tensor, v: torch.Tensor | None, idx: torch.Tensor, out=None):
    """Rows of k (and v) (B, Hkv, T, d) at positions idx (B, Hkv, m) int32, in idx order ->
    (B, Hkv, m, d) of k's dtype (libkvq kvq_gather_rows; an index outside [0, T) gives a zero row).
    ``out`` = (ko, vo): rows [0, m) of two (B, Hkv, >= m, d) tensors receive them instead."""
    _lib.require_gpu(k, idx)
    B, H, T, d = k.shape
    if idx.dim() != 3 or idx.shape[:2] != (B, H) or idx.dtype != torch.int32:
        raise ValueError("idx must be int32 (B, Hkv, m)")
    k = k.contiguous()
    if v is not None:
        _lib.require_gpu(v)
        if v.shape != k.shape or v.dtype != k.dtype:
            raise ValueError("k and v must have one shape and dtype")
        v = v.contiguous()
    idx = idx.contiguous()
    m = idx.shape[2]
    if out is None:
        ko = torch.empty((B, H, m, d), dtype=k.dtype, device=k.device)
        vo = torch.empty_like(ko) if v is not None else None
    else:
        ko, vo = out
        for o in (ko, vo):
            if o is None:
                continue
            if (o.shape[:2] != (B, H) or o.shape[2] < m or o.shape[3] != d or o.dtype != k.dtype
                    or not o.is_contiguous()):
                raise ValueError("out must be contiguous (B, Hkv, >= m, d) tensors of k's dtype")
        if (vo is None) != (v is None):
            raise ValueError("out must hold a value buffer exactly when v is given")
    row = d * k.element_size()
    _lib.call("kvq_gather_rows", k.data_ptr(), _lib.ptr(v), B * H, T, T * row, row, idx.data_ptr(), m, m,
              ko.data_ptr(), _lib.ptr(vo), ko.shape[2] * row, _lib.stream_of(k))
    return ko, vo


@torch.no_grad()
def chunk_share(qref: torch.Tensor, k: torch.Tensor) -> torch.Tensor:
    """finalize_chunk's within-chunk attention share (STRATA_KV.py:581-583): qref (B, Hkv, nq, d) the
    scaled observed queries, k (B, Hkv, C, d) -> (B, Hkv, C) float32, the softmax over the chunk's
    keys of each query averaged over the queries (libkvq kvq_chunk_share)."""
    _lib.require_gpu(qref, k)
    B, H, nq, d = qref.shape
    C = k.shape[2]
    if k.shape[:2] != (B, H) or k.shape[3] != d:
        raise ValueError("qref (B, Hkv, nq, d) and k (B, Hkv, C, d) must agree")
    q32, k32 = qref.float().contiguous(), k.float().contiguous()
    share = torch.empty((B, H, C), dtype=torch.float32, device=k.device)
    ws = torch.empty((_lib.load().kvq_chunk_share_workspace(B * H, nq, C),), dtype=torch.float32, device=k.device)
    _lib.call("kvq_chunk_share", q32.data_ptr(), k32.data_ptr(), B * H, nq, C, d, share.data_ptr(), ws.data_ptr(),
              ws.numel(), _lib.stream_of(k))
    return share


@torch.no_grad()
def fake_quant_tokens(x: torch.Tensor, bits: int) -> torch.Tensor:
    """What a reader of a token stored at ``bits`` sees (fake_quant_tokens, STRATA_KV.py:556-563):
    bits >= 16 keeps x; otherwise absmax_quant's codes times its fp16 scale per vector (549-554), in
    float32 (libkvq kvq_absmax_fake_quant)."""
    if bits >= 16:
        return x
    _lib.require_gpu(x)
    xf = x.float().contiguous()
    out = torch.empty_like(xf)
    d = xf.shape[-1]
    _lib.call("kvq_absmax_fake_quant", xf.data_ptr(), xf.numel() // d, d, int(bits), out.data_ptr(),
              _lib.stream_of(xf))
    return out


@torch.no_grad()
def finalize_chunk(k: torch.Tensor, v: torch.Tensor, qref: torch.Tensor, method, plan, keep_bits: int, cfg=None):
    """Drop-in for finalize_chunk (STRATA_KV.py:573-592) of the top-k families: k, v (B, Hkv, C, d),
    qref (B, Hkv, nq, d) scaled observed queries; keeps plan["tokens"] tokens per (b, KV head) by
    their within-chunk attention share (``chunk_share``), in position order (``topk_retain``; among
    shares tied at the m-th the lowest positions), gathers them (``gather_rows``) and stores them at
    ``keep_bits`` (``fake_quant_tokens``).  Returns {k, v, b (zeros), idx (int64)}.  ``method``: an
    object with ``family`` (or the family name); attention matching ("am", a least-squares fit
    outside this path) is refused."""
    family = getattr(method, "family", method)
    if family == "am":
        raise NotImplementedError("attention matching (family 'am') is not part of the device path")
    m = int(plan["tokens"] if isinstance(plan, dict) else plan)
    B, H, C, d = k.shape
    if not 1 <= m <= C:
        raise ValueError("plan['tokens'] must be in [1, C]")
    share = chunk_share(qref, k)
    idx = topk_retain(share, m)                                          # (B, Hkv, m) int32, position order
    gk, gv = gather_rows(k.float(), v.float(), idx)
    return {"k": fake_quant_tokens(gk, keep_bits), "v": fake_quant_tokens(gv, keep_bits),
            "b": torch.zeros((B, H, m), device=k.device), "idx": idx.to(torch.int64)}


def retained_workspace_floats(q: torch.Tensor, cache: PackedKIVICache, idx: torch.Tensor) -> int:
    """Floats of workspace one retained_decode launch of q (B, Hq, Tq, d) over idx (B, Hkv, k) needs
    (Tq within one query-token piece)."""
    B, Hq, Tq, d = q.shape
    need = _lib.load().kvq_kivi_retained_workspace(B, Hq, cache.kc.shape[1], Tq, d, idx.shape[2], cache.n_exact)
    if need < 0:
        raise _lib.KVQError("kvq_kivi_retained_workspace rejected the shape")
    return int(need)


@torch.no_grad()
def retained_decode(q: torch.Tensor, scaling: float, cache: PackedKIVICache, idx: torch.Tensor, *,
                    q_pos: torch.Tensor | None = None, out: torch.Tensor | None = None,
                    workspace: torch.Tensor | None = None, chunk: int | None = None) -> torch.Tensor:
    """Attention of q (B, Hq, Tq, d) over the retained packed positions idx (B, Hkv, k) int32 of the
    cache and its exact rows (the recent window), read straight from the packed cache (libkvq
    kvq_kivi_decode_retained: each kept token dequantised in registers, no gathered copy) ->
    (B, Tq, Hq, d) in q's dtype.  The same attention as kivi_decode over retained_cache(cache, idx),
    with the kept rows in fp32 rather than rounded to the model dtype.  Exact rows are visible per
    q_pos / cache.exact_pos as in kivi_decode; any Tq (query-token pieces, kvq.query)."""
    from .query import decode_in_pieces, query_pieces
    _lib.require_gpu(q, idx)
    B, Hq, Tq, d = q.shape
    Hkv = cache.kc.shape[1]
    _lib.check_q_cache(q, cache.kc.shape[0], Hkv, cache.kc.shape[3] * 2, "retained_decode")
    if idx.dim() != 3 or idx.shape[:2] != (B, Hkv) or idx.dtype != torch.int32:
        raise ValueError("idx must be int32 (B, Hkv, k)")
    pieces = query_pieces(Hq // Hkv, Tq, chunk)
    if len(pieces) > 1:
        return decode_in_pieces(lambda qs, qp, o: retained_decode(qs, scaling, cache, idx, q_pos=qp, out=o,
                                                                  workspace=workspace), q, q_pos, out, pieces)
    if q.stride(-1) != 1:
        q = q.contiguous()
    if cache.k_exact.dtype != q.dtype:
        raise TypeError("q and the exact rows must share a dtype")
    idx = idx.contiguous()
    k = idx.shape[2]
    if workspace is None:
        workspace = torch.empty((retained_workspace_floats(q, cache, idx),), dtype=torch.float32, device=q.device)
    out = _lib.out_or_new(out, (B, Tq, Hq, d), q.dtype, q.device, "retained_decode")
    ep = cache.exact_pos if q_pos is not None else None
    qp = q_pos if ep is not None else None
    dt = _lib.DTYPE_CODE[q.dtype]
    _lib.call("kvq_kivi_decode_retained", q.data_ptr(), dt, q.stride(0), q.stride(1), q.stride(2), B, Hq, Hkv, Tq, d,
              float(scaling), cache.kc.data_ptr(), cache.k_lo.data_ptr(), cache.k_sc.data_ptr(), cache.vc.data_ptr(),
              cache.vmeta.data_ptr(), cache.cap_t, cache.n_q, cache.group_k, cache.group_v, idx.data_ptr(), k, k,
              cache.k_exact.data_ptr(), cache.v_exact.data_ptr(), dt, cache.cap_e, cache.n_exact, _lib.ptr(ep),
              _lib.ptr(qp), out.data_ptr(), dt, workspace.data_ptr(), workspace.numel(), _lib.stream_of(q))
    return out
