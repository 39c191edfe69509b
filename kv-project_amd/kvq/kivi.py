"""KIVI quantisation and bit packing on the GPU: drop-ins for the reference's codec functions.

* ``kivi_quant``  — same signature, semantics and return dict as STRATA_KV.py:826-856.
* ``pack_codes``  — same bytes as STRATA_KV.py:2728-2732 (MSB-first packing), on the device.
* ``kivi_quant_stored`` — the storage form the decode state keeps: fp16 metadata and packed codes.
"""
from __future__ import annotations

import torch

from . import _lib


def _check_x(x: torch.Tensor) -> None:
    _lib.require_gpu(x)
    if x.dim() != 4:
        raise ValueError("x must be (B, H, T, d)")
    if x.dtype not in _lib.DTYPE_CODE:
        raise TypeError(f"unsupported dtype {x.dtype}")
    if x.stride(-1) != 1:
        raise ValueError("x must have contiguous channels")


def _meta_shape(B, H, n, d, group, along_tokens):
    if along_tokens:
        n_g = -(-n // group)
        return (B, H, n_g, d), n_g * d
    width = group if d % group == 0 else d
    return (B, H, n, d // width), n * (d // width)


@torch.no_grad()
def kivi_quant_stored(x: torch.Tensor, bits: int, group: int, along_tokens: bool, n_sink: int,
                      *, want_codes: bool = False, want_packed: bool = True,
                      want_xhat: bool = False) -> dict:
    """KIVI quantisation returning the stored representation: fp16 ``lo``/``scale`` (keys
    (B,H,n_g,d), values (B,H,n,d/width)), optional uint8 ``codes`` (B,H,n,d), optional
    ``packed`` (B,H,n,d*bits/8) pack_codes rows, optional float32 ``xhat`` (B,H,T,d)."""
    _check_x(x)
    B, H, T, d = x.shape
    n = T - n_sink
    if n < 0:
        raise ValueError("n_sink > T")
    dev = x.device
    mshape, mbh = _meta_shape(B, H, n, d, group, along_tokens)
    lo = torch.empty(mshape, dtype=torch.float16, device=dev)
    sc = torch.empty(mshape, dtype=torch.float16, device=dev)
    codes = torch.empty((B, H, n, d), dtype=torch.uint8, device=dev) if want_codes else None
    packed = None
    if want_packed:
        if (d * bits) % 8:
            raise ValueError("packed rows need d*bits divisible by 8")
        packed = torch.empty((B, H, n, d * bits // 8), dtype=torch.uint8, device=dev)
    xhat = torch.empty((B, H, T, d), dtype=torch.float32, device=dev) if want_xhat else None
    _lib.call("kvq_kivi_quant", x.data_ptr(), _lib.DTYPE_CODE[x.dtype], B, H, T, d,
              x.stride(0), x.stride(1), x.stride(2), bits, group, int(bool(along_tokens)), n_sink,
              _lib.ptr(codes), n * d, _lib.ptr(packed), n * (d * bits // 8), lo.data_ptr(),
              sc.data_ptr(), mbh, _lib.ptr(xhat), _lib.stream_of(x))
    return {"lo": lo, "scale": sc, "codes": codes, "packed": packed, "xhat": xhat}


@torch.no_grad()
def kivi_quant(x: torch.Tensor, bits: int, group: int, along_tokens: bool, n_sink: int) -> dict:
    """Drop-in for kivi_quant (STRATA_KV.py:826-856): {xhat (float32, sinks exact), codes (uint8,
    rows n_sink..), lo, scale (float32 holding fp16 values; keys (B,H,n_g,1,d), values
    (B,H,n,d/width,1))}.  Bit-exact with the reference."""
    st = kivi_quant_stored(x, bits, group, along_tokens, n_sink, want_codes=True,
                           want_packed=False, want_xhat=True)
    lo, sc = st["lo"].float(), st["scale"].float()
    if along_tokens:
        lo, sc = lo.unsqueeze(3), sc.unsqueeze(3)
    else:
        lo, sc = lo.unsqueeze(4), sc.unsqueeze(4)
    return {"xhat": st["xhat"], "codes": st["codes"], "lo": lo, "scale": sc}


@torch.no_grad()
def pack_codes(codes: torch.Tensor, bits: int) -> torch.Tensor:
    """Drop-in for pack_codes (STRATA_KV.py:2728-2732): flat uint8 tensor of the MSB-first packed
    codes (zero-padded last byte), computed on the codes' GPU."""
    _lib.require_gpu(codes)
    c = codes.reshape(-1)
    if c.dtype != torch.uint8:
        c = c.to(torch.uint8)
    c = c.contiguous()
    out = torch.empty(((c.numel() * bits + 7) // 8,), dtype=torch.uint8, device=c.device)
    _lib.call("kvq_pack_codes", c.data_ptr(), c.numel(), bits, out.data_ptr(), _lib.stream_of(c))
    return out


@torch.no_grad()
def unpack_codes(packed: torch.Tensor, bits: int, count: int) -> torch.Tensor:
    """Inverse of pack_codes: the first ``count`` codes as uint8."""
    _lib.require_gpu(packed)
    p = packed.reshape(-1).contiguous()
    out = torch.empty((count,), dtype=torch.uint8, device=p.device)
    _lib.call("kvq_unpack_codes", p.data_ptr(), count, bits, out.data_ptr(), _lib.stream_of(p))
    return out


@torch.no_grad()
def pack_rows(codes: torch.Tensor, bits: int) -> torch.Tensor:
    """Drop-in for pack_rows (QUASAR_KV.py:1185-1190): codes (..., w) < 2^bits -> uint8
    (..., w * bits / 8), first code of each byte in its most significant bits.  For rows of whole
    bytes these are pack_codes' bytes row by row, computed on the codes' GPU."""
    if bits not in (1, 2, 4, 8):
        raise ValueError("bits in {1, 2, 4, 8}")
    w = codes.shape[-1]
    if (w * bits) % 8:
        raise ValueError("a row must fill whole bytes (w * bits % 8 == 0)")
    return pack_codes(codes, bits).reshape(*codes.shape[:-1], w * bits // 8)


@torch.no_grad()
def unpack_rows(packed: torch.Tensor, bits: int, levels: torch.Tensor) -> torch.Tensor:
    """Decode of pack_rows bytes through the byte table of QUASAR_KV.py:1194-1202: float32
    (..., nbytes * 8 / bits) with every code replaced by levels[code] (levels: 2^bits float32)."""
    _lib.require_gpu(packed, levels)
    if bits not in (1, 2, 4, 8):
        raise ValueError("bits in {1, 2, 4, 8}")
    lv = levels.to(torch.float32).reshape(-1).contiguous()
    if lv.numel() != 1 << bits:
        raise ValueError("levels must hold 2^bits entries")
    p = packed.contiguous()
    out = torch.empty(p.shape[:-1] + (p.shape[-1] * (8 // bits),), dtype=torch.float32, device=p.device)
    _lib.call("kvq_unpack_rows_lut", p.data_ptr(), p.numel(), bits, lv.data_ptr(), out.data_ptr(),
              _lib.stream_of(p))
    return out


@torch.no_grad()
def v_tile(rows: torch.Tensor, cap_t: int) -> torch.Tensor:
    """4-bit value rows (B, H, n, d/2) (pack_codes order) -> decode tiles (B, H, cap_t/32, 16*d)."""
    _lib.require_gpu(rows)
    B, H, n, db = rows.shape
    d = db * 2
    rows = rows.contiguous()
    tiles = torch.empty((B, H, cap_t // 32, 16 * d), dtype=torch.uint8, device=rows.device)
    _lib.call("kvq_v_tile", rows.data_ptr(), B * H, n, n * db, d, cap_t, tiles.data_ptr(),
              _lib.stream_of(rows))
    return tiles


@torch.no_grad()
def v_untile(tiles: torch.Tensor, n: int) -> torch.Tensor:
    """Inverse of v_tile: (B, H, cap_t/32, 16*d) -> (B, H, n, d/2) pack_codes rows."""
    _lib.require_gpu(tiles)
    B, H, nc, w = tiles.shape
    d = w // 16
    tiles = tiles.contiguous()
    rows = torch.empty((B, H, n, d // 2), dtype=torch.uint8, device=tiles.device)
    _lib.call("kvq_v_untile", tiles.data_ptr(), B * H, n, d, nc * 32, rows.data_ptr(), n * d // 2,
              _lib.stream_of(tiles))
    return rows


@torch.no_grad()
def vmeta_tile(lo: torch.Tensor, scale: torch.Tensor, cap_t: int) -> torch.Tensor:
    """Value metadata (B, H, n, ngv) fp16 lo/scale -> (B, H, cap_t/32, ngv, 32, 2) fp16 pairs
    (scale, lo) in the decode kernel's token-slot order."""
    _lib.require_gpu(lo, scale)
    B, H, n, ngv = lo.shape
    lo, scale = lo.contiguous(), scale.contiguous()
    vm = torch.empty((B, H, cap_t // 32, ngv, 32, 2), dtype=torch.float16, device=lo.device)
    _lib.call("kvq_vmeta_tile", lo.data_ptr(), scale.data_ptr(), B * H, n, ngv, n * ngv, cap_t,
              vm.data_ptr(), _lib.stream_of(lo))
    return vm
