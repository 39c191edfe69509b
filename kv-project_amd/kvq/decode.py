"""Packed KIVI cache on the GPU and its split-K flash-decoding call.

``PackedKIVICache`` holds one layer's cache in the decode layout of libkvq: 4-bit key codes in
pack_codes rows (STRATA_KV.py:2728-2732), per-channel fp16 key lo/scale per group of
``group_k`` tokens, 4-bit value codes in 32-token tiles, per-token fp16 value (scale, lo) per
channel group, and the exact rows (the residual window, model dtype).  ``kivi_decode`` is one
decode step of attention over it; it replaces chunked_attention over KIVI token entries
(STRATA_KV.py:641-675 via LayerState.attend 716-719) for a single step.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional

import torch

from . import _lib
from .kivi import kivi_quant_stored, v_tile, vmeta_tile
from .query import decode_in_pieces, query_pieces


def _round_up(x: int, m: int) -> int:
    return -(-x // m) * m


@dataclass
class PackedKIVICache:
    kc: torch.Tensor            # (B, Hkv, cap_t, d/2) uint8
    k_lo: torch.Tensor          # (B, Hkv, cap_t/group_k, d) fp16
    k_sc: torch.Tensor
    vc: torch.Tensor            # (B, Hkv, cap_t/32, 16*d) uint8
    vmeta: torch.Tensor         # (B, Hkv, cap_t/32, d/group_v, 32, 2) fp16 (scale, lo)
    n_q: int
    group_k: int
    group_v: int
    k_exact: torch.Tensor       # (B, Hkv, cap_e, d) model dtype
    v_exact: torch.Tensor
    n_exact: int
    exact_pos: Optional[torch.Tensor] = None    # (cap_e,) int64, positions of the exact rows
    bits: int = 4
    ring: bool = False          # exact rows form a ring: position p in slot p % cap_e
    next_pos: int = 0           # ring mode: position of the next appended token

    @property
    def cap_t(self) -> int:
        return self.kc.shape[2]

    @property
    def cap_e(self) -> int:
        return self.k_exact.shape[2]

    @classmethod
    @torch.no_grad()
    def from_context(cls, K: torch.Tensor, V: torch.Tensor, *, window: int, group_k: int,
                     group_v: int, bits: int = 4, extra_tokens: int = 0, extra_exact: int = 0,
                     dtype: Optional[torch.dtype] = None, ring: bool = False) -> "PackedKIVICache":
        """Compress a context cache K, V (B, Hkv, T, d) the way KIVIMethod leaves it at a horizon
        (STRATA_KV.py:801-823, no sinks): rows [0, T - window) are read from their codes, the last
        ``window`` rows stay exact.  Key groups are formed over all T rows (a group that straddles
        the window boundary takes its min/max over all of its rows, as kivi_quant over the whole
        tensor does).  ``extra_tokens`` / ``extra_exact`` reserve capacity for appends."""
        _lib.require_gpu(K, V)
        if bits != 4:
            raise ValueError("the decode kernel reads 4-bit codes")
        B, H, T, d = K.shape
        if window > T or window < 0:
            raise ValueError("window must be in [0, T]")
        n_q = T - window
        dtype = dtype or K.dtype
        dev = K.device
        cap_t = max(_round_up(max(n_q + extra_tokens, 1), math.lcm(group_k, 32)), math.lcm(group_k, 32))
        kq = kivi_quant_stored(K, bits, group_k, True, 0)
        vq = kivi_quant_stored(V, bits, group_v, False, 0)
        kc = torch.zeros((B, H, cap_t, d // 2), dtype=torch.uint8, device=dev)
        n_gq = -(-n_q // group_k)
        # a key group is quantised once, when its first token leaves the window: keep the codes of
        # every row of the groups that have started (later rows of the last group are masked at
        # decode until they leave the window themselves)
        rows_k = min(n_gq * group_k, T, cap_t)
        kc[:, :, :rows_k] = kq["packed"][:, :, :rows_k]
        k_lo = torch.zeros((B, H, cap_t // group_k, d), dtype=torch.float16, device=dev)
        k_sc = torch.zeros_like(k_lo)
        k_lo[:, :, :n_gq] = kq["lo"][:, :, :n_gq]
        k_sc[:, :, :n_gq] = kq["scale"][:, :, :n_gq]
        vc = v_tile(vq["packed"][:, :, :n_q].contiguous(), cap_t)
        vmeta = vmeta_tile(vq["lo"][:, :, :n_q].contiguous(), vq["scale"][:, :, :n_q].contiguous(), cap_t)
        cap_e = window if ring else max(window + extra_exact, 1)
        if ring and (window < group_k or window == 0):
            raise ValueError("the streaming window must hold at least one key group")
        k_ex = torch.zeros((B, H, cap_e, d), dtype=dtype, device=dev)
        v_ex = torch.zeros_like(k_ex)
        slots = (torch.arange(n_q, T, device=dev) % cap_e) if ring else torch.arange(window, device=dev)
        k_ex[:, :, slots] = K[:, :, n_q:].to(dtype)
        v_ex[:, :, slots] = V[:, :, n_q:].to(dtype)
        return cls(kc, k_lo, k_sc, vc, vmeta, n_q, group_k, group_v, k_ex, v_ex, window, ring=ring,
                   next_pos=T)

    @torch.no_grad()
    def append(self, k: torch.Tensor, v: torch.Tensor) -> None:
        """Streaming append of one token per sequence, k, v (B, Hkv, 1, d): the token leaving the
        window is quantised and packed in place (and its key group once it is complete), then the
        new rows enter the ring (libkvq kvq_kivi_append).  Raises when the packed capacity is
        exhausted, as LayerState.append does for its buffer (STRATA_KV.py:707-714)."""
        if not self.ring:
            raise ValueError("append() needs a ring-layout cache (from_context(..., ring=True))")
        _lib.require_gpu(k, v)
        if k.dtype != self.k_exact.dtype or v.dtype != self.k_exact.dtype:
            raise TypeError("appended rows must have the cache's exact-row dtype")
        B, H, t, d = k.shape
        if t != 1:
            raise ValueError("append() takes one token per sequence")
        W, pos = self.cap_e, self.next_pos
        if pos >= W and pos - W >= self.cap_t:          # token pos - W would take packed row >= cap_t
            raise RuntimeError("decode buffer exhausted")
        _lib.call("kvq_kivi_append", k.data_ptr(), v.data_ptr(), _lib.DTYPE_CODE[k.dtype], k.stride(0),
                  k.stride(1), v.stride(0), v.stride(1), B, H, d, pos, self.k_exact.data_ptr(),
                  self.v_exact.data_ptr(), W, self.kc.data_ptr(), self.k_lo.data_ptr(), self.k_sc.data_ptr(),
                  self.vc.data_ptr(), self.vmeta.data_ptr(), self.cap_t, self.group_k, self.group_v,
                  _lib.stream_of(k))
        self.next_pos = pos + 1
        self.n_q = max(0, self.next_pos - W)
        self.n_exact = min(self.next_pos, W)

    def packed_bytes(self) -> int:
        """Bytes of the n_q packed rows a decode step reads: 4-bit codes + fp16 metadata."""
        B, H = self.kc.shape[:2]
        d = self.kc.shape[3] * 2
        n_g = -(-self.n_q // self.group_k)
        codes = 2 * B * H * self.n_q * d // 2
        kmeta = B * H * n_g * d * 4
        vmeta = B * H * self.n_q * (d // self.group_v) * 4
        return codes + kmeta + vmeta

    def exact_bytes(self) -> int:
        """Bytes of the n_exact exact key/value rows a decode step reads."""
        B, H = self.kc.shape[:2]
        d = self.kc.shape[3] * 2
        return 2 * B * H * self.n_exact * d * self.k_exact.element_size()

    def payload_bytes(self) -> int:
        """Bytes a decode step reads: codes and metadata of the n_q packed rows + exact rows."""
        return self.packed_bytes() + self.exact_bytes()

    def _exact_window(self, n_exact: Optional[int]):
        n_exact = self.n_exact if n_exact is None else int(n_exact)
        if not 0 <= n_exact <= self.n_exact:
            raise ValueError("n_exact must be in [0, cache.n_exact]")
        # oldest exact row first: a ring holds position p in slot p % cap_e
        first = ((self.next_pos - self.n_exact) % self.cap_e) if self.ring else 0
        return n_exact, first

    def wire_bytes(self, n_exact: Optional[int] = None) -> int:
        """Size of the wire-format payload (``export``) without writing it."""
        n_ex, _ = self._exact_window(n_exact)
        B, H = self.kc.shape[:2]
        n = _lib.load().kvq_kivi_payload_bytes(B * H, self.n_q, self.kc.shape[3] * 2, self.group_k, self.group_v, n_ex,
                                              _lib.DTYPE_CODE[self.k_exact.dtype])
        if n < 0:
            raise _lib.KVQError("kvq_kivi_payload_bytes rejected the shape")
        return int(n)

    @torch.no_grad()
    def export(self, n_exact: Optional[int] = None, out: Optional[torch.Tensor] = None) -> torch.Tensor:
        """The layer's payload in the reference's storage format (payload_bytes, STRATA_KV.py:2736-2769),
        written on the device by libkvq kvq_kivi_export: pack_codes key codes, fp16 key lo / scale
        of every group, pack_codes value codes, fp16 value lo / scale, then the first ``n_exact``
        exact rows (all by default) oldest first as fp16, each section (b, h)-major.  Its length is
        the measured cache size."""
        n_ex, first = self._exact_window(n_exact)
        nbytes = self.wire_bytes(n_ex)
        if out is None:
            out = torch.empty((nbytes,), dtype=torch.uint8, device=self.kc.device)
        B, H = self.kc.shape[:2]
        _lib.call("kvq_kivi_export", self.kc.data_ptr(), self.k_lo.data_ptr(), self.k_sc.data_ptr(), self.vc.data_ptr(),
                  self.vmeta.data_ptr(), B * H, self.cap_t, self.n_q, self.kc.shape[3] * 2, self.group_k, self.group_v,
                  self.k_exact.data_ptr(), self.v_exact.data_ptr(), _lib.DTYPE_CODE[self.k_exact.dtype], self.cap_e,
                  n_ex, first, out.data_ptr(), out.numel(), _lib.stream_of(self.kc))
        return out[:nbytes]


def exact_rows_cache(k_exact: torch.Tensor, v_exact: torch.Tensor, n_exact: int,
                     exact_pos: Optional[torch.Tensor] = None) -> PackedKIVICache:
    """A cache of exact rows only (n_q = 0): k_exact, v_exact (B, Hkv, cap_e, d) of which the first
    ``n_exact`` rows are held, visible per ``exact_pos`` (all visible when None).  The packed fields
    are minimal placeholders the decode never reads (it reads no packed row when n_q = 0)."""
    B, H, _, d = k_exact.shape
    dev = k_exact.device
    z8 = lambda *s: torch.zeros(s, dtype=torch.uint8, device=dev)
    z16 = lambda *s: torch.zeros(s, dtype=torch.float16, device=dev)
    return PackedKIVICache(z8(B, H, 64, d // 2), z16(B, H, 1, d), z16(B, H, 1, d), z8(B, H, 2, 16 * d),
                           z16(B, H, 2, d // 64, 32, 2), 0, 64, 64, k_exact, v_exact, n_exact, exact_pos)


def workspace_floats(B: int, Hq: int, Hkv: int, Tq: int, d: int, n_q: int, n_exact: int,
                     group_k: int, group_v: int, split_tokens: int = 0) -> int:
    n = _lib.load().kvq_kivi_decode_workspace(B, Hq, Hkv, Tq, d, n_q, n_exact, group_k, group_v,
                                              split_tokens)
    if n < 0:
        raise _lib.KVQError("kvq_kivi_decode_workspace rejected the shape")
    return n


def score_workspace_floats(B: int, Hq: int, Hkv: int, Tq: int, d: int, n_q: int, n_exact: int,
                           group_k: int, group_v: int, split_tokens: int = 0) -> int:
    """Workspace floats of a scored step that spills its logits (kvq_kivi_score_workspace): the
    scores then come from the logits without a second pass over the keys."""
    n = _lib.load().kvq_kivi_score_workspace(B, Hq, Hkv, Tq, d, n_q, n_exact, group_k, group_v, split_tokens)
    if n < 0:
        raise _lib.KVQError("kvq_kivi_score_workspace rejected the shape")
    return n


@torch.no_grad()
def kivi_decode(q: torch.Tensor, scaling: float, cache: PackedKIVICache, *,
                q_pos: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None,
                workspace: Optional[torch.Tensor] = None, split_tokens: int = 0,
                phases: Optional[int] = None, scores: Optional[torch.Tensor] = None,
                score_weight: float = 1.0, chunk: Optional[int] = None,
                static_scratch: bool = False) -> torch.Tensor:
    """Attention of q (B, Hq, Tq, d) over the packed cache; returns (B, Tq, Hq, d) in q's dtype.

    Any Tq: a step with more than 8 // rep query tokens (or more than ``chunk``) runs as
    consecutive launches over query-token pieces (kvq.query), as chunked_attention takes query
    chunks (STRATA_KV.py:641-675).

    With ``q_pos`` (Tq,) int64 and ``cache.exact_pos`` set, exact row i is visible to query t iff
    exact_pos[i] <= q_pos[t] (the causal rule of chunked_attention among appended rows); every
    packed row is visible.  ``phases`` 1/2 run only the split / merge kernel (timing).

    ``scores`` (B, Hkv, >= n_q) float32 on the GPU: the step also adds ``score_weight`` times the
    probability mass each packed token received from the query heads of its KV group (the
    decode-time accumulation of the eviction path).  With a workspace of score_workspace_floats
    (the default here when scores are given) the split kernel spills its logits and the scores
    come from them; a workspace of workspace_floats makes the score pass read the keys again.

    ``static_scratch``: run through kvq_kivi_decode_noalloc, which keeps the split partials in the
    library's static per-GPU scratch instead of a workspace (no device allocation in the call;
    pass ``out`` too for a step that allocates nothing -- a step split into query-token pieces
    allocates nothing at batch 1, and one staging tensor of a piece's output at a larger batch).
    Steps on one GPU that use it must not overlap in time."""
    _lib.require_gpu(q)
    B, Hq, Tq, d = q.shape
    Hkv = cache.kc.shape[1]
    _lib.check_q_cache(q, cache.kc.shape[0], Hkv, cache.kc.shape[3] * 2, "kivi_decode")
    pieces = query_pieces(Hq // Hkv, Tq, chunk)
    if len(pieces) > 1:
        if phases not in (None, 3, 7):
            raise ValueError("a chunked query step runs whole steps (phases 3 or 7)")
        return decode_in_pieces(
            lambda qs, qp, o: kivi_decode(qs, scaling, cache, q_pos=qp, out=o, workspace=workspace,
                                          split_tokens=split_tokens, phases=phases, scores=scores,
                                          score_weight=score_weight, static_scratch=static_scratch),
            q, q_pos, out, pieces)
    if q.stride(-1) != 1:
        q = q.contiguous()
    if cache.k_exact.dtype != q.dtype:
        raise TypeError("q and the exact rows must share a dtype")
    out = _lib.out_or_new(out, (B, Tq, Hq, d), q.dtype, q.device, "kivi_decode")
    if static_scratch and workspace is not None:
        raise ValueError("static_scratch takes no workspace")
    if workspace is None and not static_scratch:   # a caller's workspace is size-checked by the library
        size = workspace_floats if scores is None else score_workspace_floats
        need = size(B, Hq, Hkv, Tq, d, cache.n_q, cache.n_exact, cache.group_k, cache.group_v,
                                split_tokens)
        workspace = torch.zeros((need,), dtype=torch.float32, device=q.device)
    if phases is None:
        phases = 7 if scores is not None else 3
    if scores is not None:
        _lib.require_gpu(scores)
        if scores.dtype != torch.float32 or scores.shape[:2] != (B, Hkv) or scores.stride(-1) != 1 \
                or scores.stride(0) != Hkv * scores.stride(1) or scores.shape[2] < cache.n_q:
            raise ValueError("scores must be float32 (B, Hkv, >= n_q) with contiguous rows")
    ep = cache.exact_pos if q_pos is not None else None
    qp = q_pos if ep is not None else None
    dt = _lib.DTYPE_CODE[q.dtype]
    if static_scratch:
        _lib.call("kvq_kivi_decode_noalloc", q.data_ptr(), dt, q.stride(0), q.stride(1), q.stride(2),
                  B, Hq, Hkv, Tq, d, float(scaling),
                  cache.kc.data_ptr(), cache.k_lo.data_ptr(), cache.k_sc.data_ptr(), cache.vc.data_ptr(),
                  cache.vmeta.data_ptr(), cache.cap_t, cache.n_q, cache.group_k, cache.group_v,
                  cache.k_exact.data_ptr(), cache.v_exact.data_ptr(), dt, cache.cap_e, cache.n_exact,
                  _lib.ptr(ep), _lib.ptr(qp), out.data_ptr(), dt,
                  _lib.ptr(scores), scores.stride(1) if scores is not None else 0, float(score_weight),
                  split_tokens, phases, _lib.stream_of(q))
        return out
    _lib.call("kvq_kivi_decode", q.data_ptr(), dt, q.stride(0), q.stride(1), q.stride(2),
              B, Hq, Hkv, Tq, d, float(scaling),
              cache.kc.data_ptr(), cache.k_lo.data_ptr(), cache.k_sc.data_ptr(), cache.vc.data_ptr(),
              cache.vmeta.data_ptr(), cache.cap_t, cache.n_q, cache.group_k, cache.group_v,
              cache.k_exact.data_ptr(), cache.v_exact.data_ptr(), dt, cache.cap_e, cache.n_exact,
              _lib.ptr(ep), _lib.ptr(qp), out.data_ptr(), dt, workspace.data_ptr(), workspace.numel(),
              _lib.ptr(scores), scores.stride(1) if scores is not None else 0, float(score_weight),
              split_tokens, phases, _lib.stream_of(q))
    return out


def _unpack_rows(rows: torch.Tensor) -> torch.Tensor:
    """pack_codes rows (..., d/2) uint8 -> codes (..., d) int: channel 2i in the high nibble."""
    hi, lo = (rows >> 4).to(torch.int32), (rows & 15).to(torch.int32)
    return torch.stack([hi, lo], -1).flatten(-2)


def _dequant_keys(c: PackedKIVICache) -> torch.Tensor:
    """Dequantised keys of the n_q packed rows, float32 (B, Hkv, n_q, d): code * scale + lo."""
    codes = _unpack_rows(c.kc[:, :, :c.n_q]).float()
    g = torch.arange(c.n_q, device=c.kc.device) // c.group_k
    sc = c.k_sc[:, :, g].float()
    lo = c.k_lo[:, :, g].float()
    return codes * sc + lo


# token of each of the 32 metadata slots of a value tile: slot 8g + j holds token
# 16 * (j >> 2) + 4g + (j & 3)
_SLOT_TOKEN = [16 * (j >> 2) + 4 * g + (j & 3) for g in range(4) for j in range(8)]


def _dequant_values(c: PackedKIVICache) -> torch.Tensor:
    """Dequantised values of the n_q packed rows, float32 (B, Hkv, n_q, d)."""
    from .kivi import v_untile
    B, H = c.kc.shape[:2]
    d = c.kc.shape[3] * 2
    codes = _unpack_rows(v_untile(c.vc, c.n_q)).float()                     # (B, H, n_q, d)
    ngv = d // c.group_v
    inv = torch.empty(32, dtype=torch.long)
    inv[torch.tensor(_SLOT_TOKEN)] = torch.arange(32)
    vm = c.vmeta[:, :, :, :, inv.to(c.vmeta.device)]                          # token order
    vm = vm.permute(0, 1, 2, 4, 3, 5).reshape(B, H, -1, ngv, 2)[:, :, :c.n_q].float()
    sc = vm[..., 0].repeat_interleave(c.group_v, -1)
    lo = vm[..., 1].repeat_interleave(c.group_v, -1)
    return codes * sc + lo
