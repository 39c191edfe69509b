"""Decode states of the eviction families that keep exact rows, with the reference's selections.

* ``EvictedState`` -- the LayerState a SnapKV or StreamingLLM compression leaves (SnapKVMethod,
  STRATA_KV.py:955-981; StreamingLLMMethod, 1036-1060; LayerState, 682-719): per (b, KV head) a
  set of kept context rows, read exactly, plus appended rows.  The reference keeps every column
  some head reads and hides the others per head with ``hide``; here each (b, KV head) holds just
  its kept rows, gathered on the device (kvq_gather_rows), which is the same attention (hidden rows
  carry no weight) over fewer bytes.
* ``MTLPState`` -- "More Tokens, Lower Precision" (SnapKVQuantMethod, 984-1033): the last
  ``window`` context rows exact for every head, and the kept earlier rows, gathered in position
  order, KIVI-coded as one sequence (keys per channel over groups of ``group`` kept tokens, values
  per token over ``group`` channels; 1024-1027) and read through the packed decode.
* selections: ``snapkv_keep`` (top-k of snapkv_scores, 975), ``streaming_keep`` (sinks + recent,
  1048-1059), ``mtlp_select`` / ``mtlp_budget`` (1004-1023).

Both states follow the decode-state protocol (append, attend, check_kernel, n, n0, shared,
use_kernel, context_bytes) and run in libkvq's decode kernels only.
"""
from __future__ import annotations

import math
from dataclasses import replace
from typing import Optional

import torch

from . import _lib
from .decode import PackedKIVICache, exact_rows_cache
from .evict import SNAPKV_KERNEL, SNAPKV_WINDOW, gather_rows, snapkv_scores, topk_retain
from .state import PackedState

N_SINK = 4                               # the reference's attention sinks (STRATA_KV.py:354)
ALWAYS = -(1 << 62)                      # exact_pos of a row every decode query reads


def snapkv_keep(q, k: torch.Tensor, H: int, scaling: float, keep: int, cfg=None) -> torch.Tensor:
    """Kept positions of SnapKVMethod.entries (STRATA_KV.py:975-980): the ``keep`` largest
    snapkv_scores per (b, KV head), int32 (B, Hkv, keep) in position order (lowest positions among
    scores tied at the keep-th; torch.topk leaves that order unspecified)."""
    return topk_retain(snapkv_scores(q, k, H, scaling, cfg), keep)


def streaming_keep(B: int, Hkv: int, H: int, keep: int, n_sink: int = N_SINK, device="cuda") -> torch.Tensor:
    """Kept positions of a frozen StreamingLLMMethod (STRATA_KV.py:1048-1059): the sinks [0, n_sink)
    and the most recent max(1, keep - n_sink) context tokens, int32 (B, Hkv, m) in position order."""
    recent = max(1, keep - n_sink)
    pos = torch.arange(H, device=device)
    kept = pos[(pos < n_sink) | (pos >= H - recent)].to(torch.int32)
    return kept.expand(B, Hkv, -1).contiguous()


def mtlp_budget(keep: float, P: int, d: int, bits: int, group: int, window: int = SNAPKV_WINDOW) -> int:
    """Kept coded tokens of SnapKVQuantMethod (STRATA_KV.py:1004-1007): what keep x the fp16 context
    cache of P tokens holds once the exact window is paid, at 2 d (bits + 32 / group) bits a token."""
    per_tok = 2 * d * (bits + 32.0 / group)
    return int(math.floor((keep * P * 2 * d * 16.0 - min(window, P) * 2 * d * 16.0) / per_tok))


def mtlp_select(q, k: torch.Tensor, H: int, scaling: float, n_q: int, cfg=None) -> torch.Tensor:
    """Kept coded positions of SnapKVQuantMethod.entries (STRATA_KV.py:1016-1023): the n_q largest
    snapkv_scores among the positions before the window, int32 (B, Hkv, n_q) in position order."""
    w = int(getattr(cfg, "SNAPKV_WINDOW", SNAPKV_WINDOW))
    n_q = max(0, min(int(n_q), H - w))
    sc = snapkv_scores(q, k, H, scaling, cfg)[..., :H - w].contiguous()
    return topk_retain(sc, n_q)


def _positions(cap: int, held: int, device) -> torch.Tensor:
    pos = torch.full((cap,), 1 << 62, dtype=torch.int64, device=device)
    pos[:held] = ALWAYS
    return pos


class EvictedState(PackedState):
    """Exact kept rows per (b, KV head) as the decoder holds them after a SnapKV / StreamingLLM
    compression.  ``K, V`` (B, Hkv, H, d): the prefilled context; ``keep`` (B, Hkv, m) int32 kept
    positions (``snapkv_keep`` / ``streaming_keep``); ``extra`` rows of room for appended tokens."""

    def __init__(self, K: torch.Tensor, V: torch.Tensor, keep: torch.Tensor, *, extra: int,
                 shared: Optional[int] = None):
        _lib.require_gpu(K, V, keep)
        B, Hkv, H, d = K.shape
        m = keep.shape[2]
        ke = torch.empty((B, Hkv, m + extra, d), dtype=K.dtype, device=K.device)
        ve = torch.empty_like(ke)
        gather_rows(K, V, keep.to(torch.int32), out=(ke, ve))
        self.cache = exact_rows_cache(ke, ve, m, _positions(m + extra, m, K.device))
        self.H, self.n0, self.n, self.m = H, H, H, m
        self.shared, self.use_kernel = shared, True

    def context_bytes(self) -> int:
        """Bytes of the stored context: the kept exact rows of every (b, KV head) (state_bits counts
        the rows readable by each head, STRATA_KV.py:767-777)."""
        c = self.cache
        return 2 * c.k_exact.shape[0] * c.k_exact.shape[1] * self.m * c.k_exact.shape[3] * c.k_exact.element_size()


class MTLPState(PackedState):
    """SnapKVQuantMethod's cache as the decoder holds it: ``K, V`` (B, Hkv, H, d) the prefilled
    context, ``idx`` (B, Hkv, n_q) int32 kept positions before the window (``mtlp_select``), KIVI
    ``bits`` = 4 with groups of ``group`` (the reference's KIVI_GROUP) over the kept rows, the last
    ``window`` context rows exact, ``extra`` rows of room for appended tokens."""

    def __init__(self, K: torch.Tensor, V: torch.Tensor, idx: torch.Tensor, *, window: int = SNAPKV_WINDOW,
                 group: int = 32, extra: int, bits: int = 4, shared: Optional[int] = None):
        _lib.require_gpu(K, V, idx)
        if bits != 4:
            raise ValueError("the packed decode reads 4-bit codes")
        B, Hkv, H, d = K.shape
        n_q = idx.shape[2]
        w = min(window, H)
        if n_q:
            gk, gv = gather_rows(K, V, idx.to(torch.int32))                     # kept rows, position order
            cache = PackedKIVICache.from_context(gk, gv, window=0, group_k=group, group_v=group, bits=bits,
                                                 extra_exact=w + extra)
        else:
            cache = exact_rows_cache(torch.empty((B, Hkv, w + extra, d), dtype=K.dtype, device=K.device),
                                     torch.empty((B, Hkv, w + extra, d), dtype=K.dtype, device=K.device), 0)
        win = torch.arange(H - w, H, device=K.device, dtype=torch.int32).expand(B, Hkv, -1).contiguous()
        gather_rows(K, V, win, out=(cache.k_exact, cache.v_exact))
        self.cache = replace(cache, n_exact=w, exact_pos=_positions(cache.cap_e, w, K.device))
        self.H, self.n0, self.n, self.window = H, H, H, w
        self.shared, self.use_kernel = shared, True

    def context_bytes(self) -> int:
        """Bytes of the stored context: codes and fp16 metadata of the kept rows plus the exact
        window."""
        c = self.cache
        B, Hkv, _, d = c.k_exact.shape
        return c.packed_bytes() + 2 * B * Hkv * self.window * d * c.k_exact.element_size()
