"""STRATA codec and planar packing on the GPU (STRATA_KV.py:1110-1189, 1546-1548).

``rotation_signs`` and ``uniform_step`` restate the reference's host-side constants
(rotation_matrix's seeded sign draw, 1119-1124 with _rng 306-307; the golden-section quantiser
step, 1132-1155); everything per token runs in libkvq.
"""
from __future__ import annotations

import math
import zlib
from functools import lru_cache
from typing import Optional, Tuple

import numpy as np
import torch

from . import _lib
from .query import decode_in_pieces, query_pieces


@lru_cache(maxsize=None)
def _signs_np(d: int, key: str) -> np.ndarray:
    g = np.random.default_rng([42, zlib.crc32(b"rotation"), zlib.crc32(key.encode())])
    return g.choice([-1.0, 1.0], d)


def rotation_signs(d: int, key: str = "strata", device="cuda") -> torch.Tensor:
    """The +-1 vector s of rotation_matrix(d, key) = H_d diag(s) / sqrt(d) (float32 on the device)."""
    if d & (d - 1):
        raise ValueError("the Hadamard rotation needs a power-of-two head_dim")
    return torch.tensor(_signs_np(d, key), dtype=torch.float32, device=device)


@lru_cache(maxsize=None)
def uniform_step(bits: int) -> Tuple[float, float]:
    """(step, mse): the step (in RMS units) of the MSE-optimal mid-rise uniform quantiser of N(0, 1)
    with 2^bits levels and its mean squared error -- the reference's golden-section search on a
    360001-point grid (STRATA_KV.py:1132-1155), same return shape."""
    x = np.linspace(-9.0, 9.0, 360001)
    w = np.exp(-0.5 * x * x)
    w /= w.sum()
    half = (2 ** bits - 1) / 2.0

    def mse(step):
        c = np.clip(np.round(x / step + half), 0, 2 ** bits - 1)
        return float((w * (x - (c - half) * step) ** 2).sum())
    lo, hi = 1e-4, 4.0
    g = (math.sqrt(5) - 1) / 2
    for _ in range(200):
        a, b = hi - g * (hi - lo), lo + g * (hi - lo)
        lo, hi = (lo, b) if mse(a) < mse(b) else (a, hi)
    step = 0.5 * (lo + hi)
    return step, mse(step)


@torch.no_grad()
def pack_planar(codes: torch.Tensor, bits: int) -> torch.Tensor:
    """(..., d) uint8 codes -> (..., d*bits/8) planar bytes (STRATA_KV.py:1171-1182)."""
    _lib.require_gpu(codes)
    d = codes.shape[-1]
    c = codes.reshape(-1, d).contiguous()
    out = torch.empty((c.shape[0], d * bits // 8), dtype=torch.uint8, device=codes.device)
    _lib.call("kvq_pack_planar", c.data_ptr(), c.shape[0], d, bits, out.data_ptr(), _lib.stream_of(codes))
    return out.reshape(*codes.shape[:-1], d * bits // 8)


@torch.no_grad()
def unpack_planar(packed: torch.Tensor, bits: int) -> torch.Tensor:
    """Inverse of pack_planar (STRATA_KV.py:1185-1189): (..., d*bits/8) uint8 -> (..., d) int32 codes,
    the reference's return type."""
    return unpack_planar_u8(packed, bits).to(torch.int32)


@torch.no_grad()
def unpack_planar_u8(packed: torch.Tensor, bits: int) -> torch.Tensor:
    """unpack_planar with the codes left as uint8 (the library's output, one byte per code)."""
    _lib.require_gpu(packed)
    d = packed.shape[-1] * 8 // bits
    p = packed.reshape(-1, packed.shape[-1]).contiguous()
    out = torch.empty((p.shape[0], d), dtype=torch.uint8, device=packed.device)
    _lib.call("kvq_unpack_planar", p.data_ptr(), p.shape[0], d, bits, out.data_ptr(), _lib.stream_of(packed))
    return out.reshape(*packed.shape[:-1], d)


@torch.no_grad()
def strata_center_rotate(x: torch.Tensor, signs: Optional[torch.Tensor] = None):
    """x (B, Hkv, n, d) -> (mu (B, Hkv, d) fp16, y (B, Hkv, n, d) float32 = (x - mu) R^T)."""
    _lib.require_gpu(x)
    B, H, n, d = x.shape
    signs = rotation_signs(d, device=x.device) if signs is None else signs
    x = x.contiguous()
    mu = torch.empty((B, H, d), dtype=torch.float16, device=x.device)
    y = torch.empty((B, H, n, d), dtype=torch.float32, device=x.device)
    _lib.call("kvq_strata_center_rotate", x.data_ptr(), _lib.DTYPE_CODE[x.dtype], B * H, n, d, n * d,
              signs.data_ptr(), mu.data_ptr(), y.data_ptr(), _lib.stream_of(x))
    return mu, y


@torch.no_grad()
def strata_quantize(Y: torch.Tensor, bits: int):
    """Drop-in for strata_quantize (STRATA_KV.py:1158-1168): rotated, centred vectors Y (..., 128) on
    the GPU -> (codes uint8 (..., 128), s (...), y_hat (..., 128)), s the fp16-stored scale and
    y_hat = s (c - (2^bits - 1) / 2), both in float32 (the library quantises float32 rows; Y of
    another dtype is converted first).  The codes and scales come from kvq_strata_quantize, the
    kernel the compressor uses (planar form: ``strata_quantize_planar``)."""
    _lib.require_gpu(Y)
    d = Y.shape[-1]
    y = Y.reshape(1, 1, -1, d).to(torch.float32)
    planar, s16 = strata_quantize_planar(y, bits)
    codes = unpack_planar_u8(planar, bits).reshape(Y.shape)
    s = s16.float().reshape(Y.shape[:-1])
    y_hat = (codes.float() - (2 ** bits - 1) / 2.0) * s[..., None]
    return codes, s, y_hat


@torch.no_grad()
def strata_quantize_planar(y: torch.Tensor, bits: int, idx: Optional[torch.Tensor] = None):
    """Rotated rows y (B, Hkv, n, d) float32 (rows idx (B, Hkv, m) int32 if given) -> (planar codes
    (B, Hkv, m, d*bits/8) uint8, scales (B, Hkv, m) fp16): strata_quantize (STRATA_KV.py:1158-1168)
    followed by pack_planar (1171-1182), the stored form of a stratum, in one launch."""
    _lib.require_gpu(y)
    B, H, n, d = y.shape
    y = y.contiguous()
    if idx is not None:
        idx = idx.to(torch.int32).contiguous()
        if idx.shape[:2] != (B, H) or bool(((idx < 0) | (idx >= n)).any()):
            raise ValueError("idx must be (B, Hkv, m) positions in [0, n)")
    m = n if idx is None else idx.shape[2]
    codes = torch.empty((B, H, m, d * bits // 8), dtype=torch.uint8, device=y.device)
    scales = torch.empty((B, H, m), dtype=torch.float16, device=y.device)
    _lib.call("kvq_strata_quantize", y.data_ptr(), B * H, n, d, _lib.ptr(idx), m, bits, uniform_step(bits)[0],
              codes.data_ptr(), scales.data_ptr(), _lib.stream_of(y))
    return codes, scales


@torch.no_grad()
def strata_v_tile(rows: torch.Tensor, vs: torch.Tensor, bits: int, cap_t: int):
    """Planar value rows (B, Hkv, n, d*bits/8) and fp16 scales (B, Hkv, n) -> (tiles
    (B, Hkv, cap_t/32, 512*bits) uint8, slot-ordered scales (B, Hkv, cap_t/32, 32) fp16)."""
    _lib.require_gpu(rows, vs)
    B, H, n, rb = rows.shape
    rows, vs = rows.contiguous(), vs.contiguous()
    tiles = torch.empty((B, H, cap_t // 32, 512 * bits), dtype=torch.uint8, device=rows.device)
    vsl = torch.empty((B, H, cap_t // 32, 32), dtype=torch.float16, device=rows.device)
    _lib.call("kvq_strata_v_tile", rows.data_ptr(), B * H, n, n * rb, bits, cap_t, tiles.data_ptr(), vs.data_ptr(),
              n, vsl.data_ptr(), _lib.stream_of(rows))
    return tiles, vsl


from dataclasses import dataclass, field
from typing import List, Sequence, Tuple


@dataclass
class StrataTier:
    """One stratum of a STRATA cache on the GPU (the tier dict of STRATA_KV.py:1615-1623 plus the
    decode kernel's value tiles): planar key rows (B, Hkv, n, d*bits/8), fp16 key scales
    (B, Hkv, cap) zero past n, value tiles and slot-ordered value scales of capacity cap
    (multiple of 32)."""
    bits: int
    n: int
    kc: torch.Tensor
    ks: torch.Tensor
    vt: torch.Tensor
    vsl: torch.Tensor
    cap: int
    vc: torch.Tensor = None          # planar value rows (kept for byte accounting / repacking)
    vs: torch.Tensor = None


@dataclass
class StrataCache:
    """STRATA-coded context of one layer (StrataState, STRATA_KV.py:1710-1760): per-head fp16 means,
    the rotation signs, strata of 2/4/8-bit codes, and exact rows (window + appended tokens)."""
    mu_k: torch.Tensor
    mu_v: torch.Tensor
    signs: torch.Tensor
    tiers: List[StrataTier]
    k_exact: torch.Tensor
    v_exact: torch.Tensor
    n_exact: int
    exact_pos: Optional[torch.Tensor] = None

    @classmethod
    @torch.no_grad()
    def from_context(cls, K: torch.Tensor, V: torch.Tensor, *, window: int,
                     assign: Sequence[Tuple[int, torch.Tensor]], extra_exact: int = 0) -> "StrataCache":
        """K, V (B, Hkv, T, d): rows [0, T - window) are coded, the last ``window`` stay exact.
        ``assign`` = [(bits, idx (B, Hkv, m) positions in [0, T - window))]: the tokens of each
        stratum (a token in no stratum is dropped, as the reference's level 0).  The means are
        taken over all coded rows (STRATA_KV.py:1546)."""
        _lib.require_gpu(K, V)
        B, H, T, d = K.shape
        nc = T - window
        signs = rotation_signs(d, device=K.device)
        mu_k, yk = strata_center_rotate(K[:, :, :nc], signs)
        mu_v, yv = strata_center_rotate(V[:, :, :nc], signs)
        tiers = []
        for bits, idx in assign:
            idx = idx.to(device=K.device, dtype=torch.int32)
            m = idx.shape[2]
            kc, ks = strata_quantize_planar(yk, bits, idx)
            vc, vs = strata_quantize_planar(yv, bits, idx)
            cap = max(32, -(-m // 32) * 32)
            vt, vsl = strata_v_tile(vc, vs, bits, cap)
            ksp = torch.zeros((B, H, cap), dtype=torch.float16, device=K.device)
            ksp[:, :, :m] = ks
            tiers.append(StrataTier(bits, m, kc, ksp, vt, vsl, cap, vc, vs))
        cap_e = max(window + extra_exact, 1)
        ke = torch.zeros((B, H, cap_e, d), dtype=K.dtype, device=K.device)
        ve = torch.zeros_like(ke)
        ke[:, :, :window] = K[:, :, nc:]
        ve[:, :, :window] = V[:, :, nc:]
        return cls(mu_k, mu_v, signs, tiers, ke, ve, window)

    def coded_bytes(self) -> int:
        """Bytes of the coded context a decode step reads: codes + fp16 scales of every stratum and
        the fp16 means (context_bytes' coded part, STRATA_KV.py:1729-1735)."""
        tot = self.mu_k.numel() * 2 + self.mu_v.numel() * 2
        for t in self.tiers:
            tot += 2 * t.kc.numel() + 2 * t.n * t.kc.shape[0] * t.kc.shape[1] * 2
        return tot


def strata_workspace_floats(B: int, Hq: int, Hkv: int, Tq: int, d: int, n_exact: int, tier_n: Sequence[int],
                            tier_bits: Sequence[int]) -> int:
    import ctypes
    arr = (ctypes.c_int64 * max(1, len(tier_n)))(*tier_n)
    bits = (ctypes.c_int * max(1, len(tier_bits)))(*tier_bits)
    n = _lib.load().kvq_strata_decode_workspace(B, Hq, Hkv, Tq, d, n_exact, len(tier_n), bits, arr)
    if n < 0:
        raise _lib.KVQError("kvq_strata_decode_workspace rejected the shape")
    return n


@torch.no_grad()
def strata_decode(q: torch.Tensor, scaling: float, cache: StrataCache, *, q_pos: Optional[torch.Tensor] = None,
                  out: Optional[torch.Tensor] = None, workspace: Optional[torch.Tensor] = None,
                  chunk: Optional[int] = None) -> torch.Tensor:
    """StrataState.attend (STRATA_KV.py:1762-1795) for q (B, Hq, Tq, d) -> (B, Tq, Hq, d): the exact
    rows (visible per q_pos / exact_pos when both are set) and every stratum, merged exactly, the
    coded part rotated back once and the value mean added.  Any Tq (query-token pieces of at most
    8 // rep tokens, and at most ``chunk``; kvq.query)."""
    import ctypes
    _lib.require_gpu(q)
    B, Hq, Tq, d = q.shape
    Hkv = cache.k_exact.shape[1]
    _lib.check_q_cache(q, cache.k_exact.shape[0], Hkv, cache.k_exact.shape[3], "strata_decode")
    pieces = query_pieces(Hq // Hkv, Tq, chunk)
    if len(pieces) > 1:
        return decode_in_pieces(lambda qs, qp, o: strata_decode(qs, scaling, cache, q_pos=qp, out=o, workspace=workspace),
                                q, q_pos, out, pieces)
    if q.stride(-1) != 1:
        q = q.contiguous()
    if cache.k_exact.dtype != q.dtype:
        raise TypeError("q and the exact rows must share a dtype")
    tiers = [t for t in cache.tiers if t.n > 0]
    nt = len(tiers)
    if workspace is None:                      # a caller's workspace is size-checked by the library
        need = strata_workspace_floats(B, Hq, Hkv, Tq, d, cache.n_exact, [t.n for t in tiers], [t.bits for t in tiers])
        workspace = torch.zeros((need,), dtype=torch.float32, device=q.device)
    out = _lib.out_or_new(out, (B, Tq, Hq, d), q.dtype, q.device, "strata_decode")
    P = ctypes.c_void_p
    bits = (ctypes.c_int * max(1, nt))(*[t.bits for t in tiers])
    tn = (ctypes.c_int64 * max(1, nt))(*[t.n for t in tiers])
    cap = (ctypes.c_int64 * max(1, nt))(*[t.cap for t in tiers])
    kc = (P * max(1, nt))(*[t.kc.data_ptr() for t in tiers])
    ks = (P * max(1, nt))(*[t.ks.data_ptr() for t in tiers])
    vt = (P * max(1, nt))(*[t.vt.data_ptr() for t in tiers])
    vsl = (P * max(1, nt))(*[t.vsl.data_ptr() for t in tiers])
    ep = cache.exact_pos if q_pos is not None else None
    qp = q_pos if ep is not None else None
    dt = _lib.DTYPE_CODE[q.dtype]
    _lib.call("kvq_strata_decode", q.data_ptr(), dt, q.stride(0), q.stride(1), q.stride(2), B, Hq, Hkv, Tq, d,
              float(scaling), cache.signs.data_ptr(), cache.mu_k.data_ptr(), cache.mu_v.data_ptr(), nt, bits, tn,
              cap, kc, ks, vt, vsl, cache.k_exact.data_ptr(), cache.v_exact.data_ptr(), cache.k_exact.shape[2],
              cache.n_exact, _lib.ptr(ep), _lib.ptr(qp), out.data_ptr(), workspace.data_ptr(), workspace.numel(),
              _lib.stream_of(q))
    return out
