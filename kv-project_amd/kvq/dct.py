"""Blockwise token-axis DCT coding of K/V and the decode over it (libkvq kvq_dct_*).

No DCT exists in the reference; the coder follows its conventions: symmetric absmax quantisation
of each (block, channel)'s 16 kept coefficients (absmax_quant, STRATA_KV.py:549-554) stored
offset-binary at 4 bits (TILT_KV.py:2621-2625), and attention over the reconstructed rows plus
exact rows (chunked_attention, STRATA_KV.py:641-675).
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional

import numpy as np
import torch

from . import _lib
from .query import decode_in_pieces, query_pieces

BLOCK = 64
KEEP = 16

_TABLES = {}


def dct_table(device="cuda") -> torch.Tensor:
    """(16, 64) float32: rows 0..15 of the orthonormal DCT-II, C[k, n] = a_k cos(pi (2n + 1) k / 128),
    a_0 = 1/8, a_k = sqrt(2)/8, rounded once from float64."""
    key = str(device)
    if key not in _TABLES:
        k = np.arange(KEEP)[:, None]
        n = np.arange(BLOCK)[None, :]
        C = np.cos(math.pi * (2 * n + 1) * k / (2 * BLOCK))
        C[0] *= math.sqrt(1.0 / BLOCK)
        C[1:] *= math.sqrt(2.0 / BLOCK)
        _TABLES[key] = torch.tensor(C.astype(np.float32), device=device)
    return _TABLES[key]


def dct_decode_table(device="cuda") -> torch.Tensor:
    """(2048,) float32: the table C (16, 64) followed by its transpose (64, 16), the decode's constant
    operands (each lane reads 16-byte runs of either)."""
    key = "dec:" + str(device)
    if key not in _TABLES:
        C = dct_table(device)
        _TABLES[key] = torch.cat([C.reshape(-1), C.t().contiguous().reshape(-1)])
    return _TABLES[key]


@torch.no_grad()
def dct_encode(x: torch.Tensor, for_values: bool = False):
    """x (B, Hkv, T, 128), T % 64 == 0 -> (codes (B, Hkv, T/64, 1024) uint8, scales (B, Hkv, T/64, 128)
    fp16) in the key layout (16 rows of 16 words by coefficient: word D holds channels 8D .. 8D+7, channel
    8D + e at nibble (0, 4, 1, 5, 2, 6, 3, 7)[e]; scales by channel) or, with
    ``for_values``, the value-tile layout the decode reads."""
    _lib.require_gpu(x)
    B, H, T, d = x.shape
    if d != 128 or T % BLOCK:
        raise ValueError("dct_encode needs head_dim 128 and T a multiple of 64")
    x = x.contiguous()
    nb = T // BLOCK
    codes = torch.empty((B, H, nb, 1024), dtype=torch.uint8, device=x.device)
    scales = torch.empty((B, H, nb, 128), dtype=torch.float16, device=x.device)
    _lib.call("kvq_dct_encode", x.data_ptr(), _lib.DTYPE_CODE[x.dtype], B * H, T, d, T * d,
              dct_table(x.device).data_ptr(), int(for_values), codes.data_ptr(), scales.data_ptr(),
              _lib.stream_of(x))
    return codes, scales


@dataclass
class DctCache:
    """DCT-coded context of one layer: T coded tokens (whole 64-token blocks) and exact rows (the
    remainder of the context, the recent window and appended tokens)."""
    T: int
    kc: torch.Tensor
    ks: torch.Tensor
    vc: torch.Tensor
    vs: torch.Tensor
    k_exact: torch.Tensor
    v_exact: torch.Tensor
    n_exact: int
    exact_pos: Optional[torch.Tensor] = None

    @classmethod
    @torch.no_grad()
    def from_context(cls, K: torch.Tensor, V: torch.Tensor, *, window: int, extra_exact: int = 0) -> "DctCache":
        """K, V (B, Hkv, T, d): the largest multiple of 64 tokens of [0, T - window) is coded, every
        later row stays exact (at least ``window`` of them)."""
        _lib.require_gpu(K, V)
        B, H, T, d = K.shape
        nc = max(0, (T - window) // BLOCK * BLOCK)
        kc, ks = dct_encode(K[:, :, :nc])
        vc, vs = dct_encode(V[:, :, :nc], for_values=True)
        ne = T - nc
        cap_e = max(ne + extra_exact, 1)
        ke = torch.zeros((B, H, cap_e, d), dtype=K.dtype, device=K.device)
        ve = torch.zeros_like(ke)
        ke[:, :, :ne] = K[:, :, nc:]
        ve[:, :, :ne] = V[:, :, nc:]
        return cls(nc, kc, ks, vc, vs, ke, ve, ne)

    def coded_bytes(self) -> int:
        """Bytes of the coded context one decode step reads (codes + fp16 scales)."""
        return sum(t.numel() * t.element_size() for t in (self.kc, self.ks, self.vc, self.vs))


def dct_workspace_floats(B: int, Hq: int, Hkv: int, Tq: int, d: int, T: int, n_exact: int) -> int:
    n = _lib.load().kvq_dct_decode_workspace(B, Hq, Hkv, Tq, d, T, n_exact)
    if n < 0:
        raise _lib.KVQError("kvq_dct_decode_workspace rejected the shape")
    return n


@torch.no_grad()
def dct_decode(q: torch.Tensor, scaling: float, cache: DctCache, *, q_pos: Optional[torch.Tensor] = None,
               out: Optional[torch.Tensor] = None, workspace: Optional[torch.Tensor] = None,
               phases: int = 3, chunk: Optional[int] = None) -> torch.Tensor:
    """Attention of q (B, Hq, Tq, d) over the coded blocks (all visible) and the exact rows (visible
    per q_pos / exact_pos when both are set) -> (B, Tq, Hq, d) of q's dtype.  ``phases`` 1 computes
    only the partials into ``workspace``, 2 only merges them (timing hooks), 3 both.  Any Tq (query-token
    pieces of at most 8 // rep tokens, and at most ``chunk``; kvq.query)."""
    _lib.require_gpu(q)
    B, Hq, Tq, d = q.shape
    Hkv = cache.k_exact.shape[1]
    _lib.check_q_cache(q, cache.k_exact.shape[0], Hkv, cache.k_exact.shape[3], "dct_decode")
    pieces = query_pieces(Hq // Hkv, Tq, chunk)
    if len(pieces) > 1:
        if phases != 3:
            raise ValueError("a chunked query step runs whole steps (phases 3)")
        return decode_in_pieces(lambda qs, qp, o: dct_decode(qs, scaling, cache, q_pos=qp, out=o, workspace=workspace),
                                q, q_pos, out, pieces)
    if q.stride(-1) != 1:
        q = q.contiguous()
    if cache.k_exact.dtype != q.dtype:
        raise TypeError("q and the exact rows must share a dtype")
    if workspace is None:                      # a caller's workspace is size-checked by the library
        workspace = torch.zeros((dct_workspace_floats(B, Hq, Hkv, Tq, d, cache.T, cache.n_exact),), dtype=torch.float32, device=q.device)
    out = _lib.out_or_new(out, (B, Tq, Hq, d), q.dtype, q.device, "dct_decode")
    ep = cache.exact_pos if q_pos is not None else None
    qp = q_pos if ep is not None else None
    _lib.call("kvq_dct_decode", q.data_ptr(), _lib.DTYPE_CODE[q.dtype], q.stride(0), q.stride(1), q.stride(2),
              B, Hq, Hkv, Tq, d, float(scaling), dct_decode_table(q.device).data_ptr(), cache.T, cache.kc.data_ptr(),
              cache.ks.data_ptr(), cache.vc.data_ptr(), cache.vs.data_ptr(), cache.k_exact.data_ptr(),
              cache.v_exact.data_ptr(), cache.k_exact.shape[2], cache.n_exact, _lib.ptr(ep), _lib.ptr(qp),
              out.data_ptr(), workspace.data_ptr(), workspace.numel(), int(phases), _lib.stream_of(q))
    return out
