"""Mixed-width KIVI cache: per-64-token-block code widths 2/4/8 with an offset table (libkvq
kvq_mixed_*).

Inside a block the codes and fp16 metadata are kivi_quant's (STRATA_KV.py:826-856) at the
block's width with group 32; the decode is chunked_attention (641-675) over the blocks' entries
plus exact rows.  The reference keeps one dense tensor per width (StrataState, 1782-1783); here
every block carries its width and the blocks of a (b, h) live in one variable-width region.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch

from . import _lib
from .query import decode_in_pieces, query_pieces

BLOCK = 64
UNIT = 2048                 # bytes; a block of width b occupies b + 1 units


def c3_widths(importance: torch.Tensor) -> torch.Tensor:
    """importance (B, H, nb) -> widths (B, H, nb) int8: the top floor(0.1 nb) blocks of each
    (b, h) by importance get 8 bits, the next floor(0.4 nb) - floor(0.1 nb) get 4, the rest 2."""
    nb = importance.shape[-1]
    n8 = int(0.1 * nb)
    n4 = int(0.4 * nb) - n8
    order = torch.argsort(-importance, dim=-1, stable=True)
    rank = torch.argsort(order, dim=-1, stable=True)
    w = torch.full(importance.shape, 2, dtype=torch.int8, device=importance.device)
    w[rank < n8 + n4] = 4
    w[rank < n8] = 8
    return w


def offset_table(widths: torch.Tensor):
    """widths (B, H, nb) in {2, 4, 8} -> (blk_bits (B, H, nb) uint8, blk_off (B, H, nb) int32 units
    from the (b, h) base, bh_base (B*H,) int64 units, seg (B*H, 4) int64 = (base, n8, n4, n2),
    total units).  Storage order within a (b, h): 8-bit blocks, then 4-bit, then 2-bit, each in
    token order."""
    B, H, nb = widths.shape
    w = widths.to(torch.int64).reshape(B * H, nb)
    if bool(((w != 2) & (w != 4) & (w != 8)).any()):
        raise ValueError("block widths must be 2, 4 or 8")
    order = torch.argsort(-w, dim=-1, stable=True)                   # storage order
    size = torch.gather(w + 1, 1, order)                              # units per stored block
    start = torch.cumsum(size, 1) - size                              # units from the (b, h) base
    off = torch.empty_like(start)
    off.scatter_(1, order, start)
    tot = size.sum(1)
    base = torch.cumsum(tot, 0) - tot
    seg = torch.stack([base, (w == 8).sum(1), (w == 4).sum(1), (w == 2).sum(1)], 1).contiguous()
    return (w.to(torch.uint8).reshape(B, H, nb).contiguous(), off.to(torch.int32).reshape(B, H, nb).contiguous(),
            base.contiguous(), seg, int(tot.sum()))


@dataclass
class MixedKIVICache:
    """Mixed-width coded context of one layer: nb 64-token blocks per (b, h) in ``buf`` (see
    offset_table for the layout) and exact rows (the remainder, the window, appended tokens)."""
    nb: int
    buf: torch.Tensor
    blk_bits: torch.Tensor
    blk_off: torch.Tensor
    bh_base: torch.Tensor
    seg: torch.Tensor
    k_exact: torch.Tensor
    v_exact: torch.Tensor
    n_exact: int
    exact_pos: Optional[torch.Tensor] = None

    @classmethod
    @torch.no_grad()
    def from_context(cls, K: torch.Tensor, V: torch.Tensor, widths: torch.Tensor, *, window: int,
                     extra_exact: int = 0) -> "MixedKIVICache":
        """K, V (B, Hkv, T, 128); widths (B, Hkv, nb) with nb = (T - window) // 64: block i covers
        tokens [64 i, 64 i + 64); every later row stays exact."""
        _lib.require_gpu(K, V)
        B, H, T, d = K.shape
        if d != 128:
            raise ValueError("the mixed-width cache needs head_dim 128")
        nb = max(0, (T - window) // BLOCK)
        if tuple(widths.shape) != (B, H, nb):
            raise ValueError(f"widths must be (B, Hkv, {nb})")
        nc = nb * BLOCK
        bits, off, base, seg, units = offset_table(widths.to(K.device))
        buf = torch.empty((max(units, 1) * UNIT,), dtype=torch.uint8, device=K.device)
        if nb:
            Kc, Vc = K[:, :, :nc].contiguous(), V[:, :, :nc].contiguous()
            _lib.call("kvq_mixed_encode", Kc.data_ptr(), Vc.data_ptr(), _lib.DTYPE_CODE[K.dtype], B * H, nb, d, nc * d,
                      bits.data_ptr(), off.data_ptr(), base.data_ptr(), buf.data_ptr(), _lib.stream_of(K))
        ne = T - nc
        cap_e = max(ne + extra_exact, 1)
        ke = torch.zeros((B, H, cap_e, d), dtype=K.dtype, device=K.device)
        ve = torch.zeros_like(ke)
        ke[:, :, :ne] = K[:, :, nc:]
        ve[:, :, :ne] = V[:, :, nc:]
        return cls(nb, buf, bits, off, base, seg, ke, ve, ne)

    def coded_bytes(self) -> int:
        """Bytes of the coded blocks one decode step reads (codes + fp16 metadata) plus the
        segment table."""
        return int((self.blk_bits.to(torch.int64) + 1).sum()) * UNIT + self.seg.numel() * 8

    def block_view(self, b: int, h: int, i: int) -> torch.Tensor:
        """The bytes of block i (token order) of (b, h)."""
        H = self.blk_bits.shape[1]
        bits = int(self.blk_bits[b, h, i])
        start = (int(self.bh_base[b * H + h]) + int(self.blk_off[b, h, i])) * UNIT
        return self.buf[start:start + (bits + 1) * UNIT]


def mixed_workspace_floats(B: int, Hq: int, Hkv: int, Tq: int, d: int, nb: int, n_exact: int) -> int:
    n = _lib.load().kvq_mixed_decode_workspace(B, Hq, Hkv, Tq, d, nb, n_exact)
    if n < 0:
        raise _lib.KVQError("kvq_mixed_decode_workspace rejected the shape")
    return n


@torch.no_grad()
def mixed_decode(q: torch.Tensor, scaling: float, cache: MixedKIVICache, *, q_pos: Optional[torch.Tensor] = None,
                 out: Optional[torch.Tensor] = None, workspace: Optional[torch.Tensor] = None,
                 phases: int = 3, chunk: Optional[int] = None) -> torch.Tensor:
    """Attention of q (B, Hq, Tq, d) over every coded block (all visible) and the exact rows
    (visible per q_pos / exact_pos when both are set) -> (B, Tq, Hq, d) of q's dtype.  ``phases`` 1 computes
    only the partials into ``workspace``, 2 only merges them (timing hooks), 3 both.  Any Tq (query-token
    pieces of at most 8 // rep tokens, and at most ``chunk``; kvq.query)."""
    _lib.require_gpu(q)
    B, Hq, Tq, d = q.shape
    Hkv = cache.k_exact.shape[1]
    _lib.check_q_cache(q, cache.k_exact.shape[0], Hkv, cache.k_exact.shape[3], "mixed_decode")
    pieces = query_pieces(Hq // Hkv, Tq, chunk)
    if len(pieces) > 1:
        if phases != 3:
            raise ValueError("a chunked query step runs whole steps (phases 3)")
        return decode_in_pieces(lambda qs, qp, o: mixed_decode(qs, scaling, cache, q_pos=qp, out=o, workspace=workspace),
                                q, q_pos, out, pieces)
    if q.stride(-1) != 1:
        q = q.contiguous()
    if cache.k_exact.dtype != q.dtype:
        raise TypeError("q and the exact rows must share a dtype")
    if workspace is None:                      # a caller's workspace is size-checked by the library
        workspace = torch.zeros((mixed_workspace_floats(B, Hq, Hkv, Tq, d, cache.nb, cache.n_exact),), dtype=torch.float32, device=q.device)
    out = _lib.out_or_new(out, (B, Tq, Hq, d), q.dtype, q.device, "mixed_decode")
    ep = cache.exact_pos if q_pos is not None else None
    qp = q_pos if ep is not None else None
    _lib.call("kvq_mixed_decode", q.data_ptr(), _lib.DTYPE_CODE[q.dtype], q.stride(0), q.stride(1), q.stride(2),
              B, Hq, Hkv, Tq, d, float(scaling), cache.buf.data_ptr(), cache.seg.data_ptr(), cache.nb,
              cache.k_exact.data_ptr(), cache.v_exact.data_ptr(), cache.k_exact.shape[2], cache.n_exact,
              _lib.ptr(ep), _lib.ptr(qp), out.data_ptr(), workspace.data_ptr(), workspace.numel(), int(phases),
              _lib.stream_of(q))
    return out
