"""KIVI group quantiser, fp16 storage rounding and MSB-first bit packing (numpy restatement).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Reference:
  * ``as_stored``   STRATA_KV.py:539-542
  * ``kivi_quant``  STRATA_KV.py:826-856 (byte-identical twins QUASAR_KV.py:840, HEDGE_KV.py:856)
  * ``pack_codes``  STRATA_KV.py:2728-2732

Pinning (tests/test_oracle_kivi.py):
  * ``kivi_quant`` by its closed form: every code is checked against a brute-force argmin over
    all 2^b levels (round-half-even tie rule included), lo against fp16(min) of the group, scale
    against fp16((max - lo) / qmax) clamped at 2^-24, and hand-computed known answers; the
    padding rule (last row replicated) against explicit small cases.
  * ``pack_codes`` against ``numpy.packbits(bitorder='big')``, the library routine the reference
    calls (STRATA_KV.py:2731-2732), and by round trip through ``unpack_codes``.
"""
from __future__ import annotations

import numpy as np

FP16_MAX = 65504.0          # STRATA_KV.py:536


def as_stored(x: np.ndarray) -> np.ndarray:
    """Saturating round to fp16 and back to x's dtype (STRATA_KV.py:539-542)."""
    return np.clip(x, -FP16_MAX, FP16_MAX).astype(np.float16).astype(x.dtype)


def kivi_quant(x: np.ndarray, bits: int, group: int, along_tokens: bool, n_sink: int) -> dict:
    """KIVI asymmetric min/max quantisation (STRATA_KV.py:826-856).

    x (B, H, T, d).  Keys (along_tokens=True): per channel over groups of ``group`` consecutive
    tokens, the last partial group padded by replicating the last row (842-843).  Values: per token
    over groups of ``group`` channels, or the whole row when d % group != 0 (847-849).  Returns
    xhat (float32, sinks exact), codes (uint8, rows n_sink..), lo and scale (float32 holding fp16
    values) with the reference's shapes: K (B,H,n_g,1,d), V (B,H,n,d/width,1).
    """
    qmax = 2 ** bits - 1
    y = np.asarray(x, dtype=np.float32)
    body = y[:, :, n_sink:]
    B, H, n, d = body.shape
    if along_tokens:
        n_g = -(-n // group)
        pad = n_g * group - n
        if pad:
            body = np.concatenate([body, np.broadcast_to(body[:, :, -1:], (B, H, pad, d))], 2)
        g = body.reshape(B, H, n_g, group, d)
        red = 3
    else:
        width = group if d % group == 0 else d
        g = body.reshape(B, H, n, d // width, width)
        red = 4
    lo = as_stored(g.min(axis=red, keepdims=True))
    # (max - lo) / qmax in float32, rounded to fp16, then clamp_min(2^-24) (850)
    sc = np.maximum(as_stored((g.max(axis=red, keepdims=True) - lo) / np.float32(qmax)),
                    np.float32(2.0 ** -24))
    codes = np.clip(np.round((g - lo) / sc), 0, qmax)                # half-to-even, as torch.round
    deq = (codes * sc + lo).reshape(B, H, -1, d)[:, :, :n]           # two roundings, no FMA
    return {"xhat": np.concatenate([y[:, :, :n_sink], deq], 2).astype(np.float32),
            "codes": codes.reshape(B, H, -1, d)[:, :, :n].astype(np.uint8),
            "lo": lo.astype(np.float32), "scale": sc.astype(np.float32)}


def kivi_dequant(codes: np.ndarray, lo: np.ndarray, scale: np.ndarray, group: int,
                 along_tokens: bool) -> np.ndarray:
    """xhat of stored codes exactly as kivi_quant computes it: codes * scale + lo in float32,
    two roundings (STRATA_KV.py:853).  codes (B,H,n,d); lo/scale in kivi_quant's shapes."""
    B, H, n, d = codes.shape
    c = codes.astype(np.float32)
    if along_tokens:
        n_g = lo.shape[2]
        pad = n_g * group - n
        if pad:
            c = np.concatenate([c, np.zeros((B, H, pad, d), np.float32)], 2)
        g = c.reshape(B, H, n_g, group, d)
    else:
        width = d // lo.shape[3]
        g = c.reshape(B, H, n, d // width, width)
    out = (g * scale.astype(np.float32)) + lo.astype(np.float32)
    return out.reshape(B, H, -1, d)[:, :, :n]


def pack_codes(codes: np.ndarray, bits: int) -> np.ndarray:
    """Bit-pack non-negative integer codes (< 2^bits) into uint8, MSB first (STRATA_KV.py:2728-2732).

    The reference flattens row-major, expands every code into ``bits`` big-endian bit planes and
    calls np.packbits (zero padding of the last byte).  Restated here with shifts on the
    concatenated bit string so that the numpy routine stays an independent check.
    """
    c = np.asarray(codes).reshape(-1).astype(np.uint64)
    nbits = c.size * bits
    out = np.zeros((nbits + 7) // 8, dtype=np.uint8)
    if bits in (1, 2, 4, 8):
        per = 8 // bits
        pad = (-c.size) % per
        cc = np.concatenate([c, np.zeros(pad, np.uint64)]).reshape(-1, per)
        acc = np.zeros(cc.shape[0], np.uint64)
        for i in range(per):                          # first code in the most significant bits
            acc |= (cc[:, i] & np.uint64((1 << bits) - 1)) << np.uint64(bits * (per - 1 - i))
        out[:] = acc.astype(np.uint8)
        return out
    for i in range(bits):                             # general widths: bit i of every code, MSB first
        bit = ((c >> np.uint64(bits - 1 - i)) & np.uint64(1)).astype(np.uint8)
        pos = np.arange(c.size, dtype=np.int64) * bits + i
        np.bitwise_or.at(out, pos // 8, (bit << (7 - (pos % 8))).astype(np.uint8))
    return out


def pack_rows(codes: np.ndarray, bits: int) -> np.ndarray:
    """QUASAR_KV.py:1185-1190: codes (..., w) -> uint8 (..., w * bits / 8), the 8/bits codes of a
    byte placed from its most significant bits down (w * bits must be a multiple of 8)."""
    c = np.asarray(codes).astype(np.uint32)
    per = 8 // bits
    g = c.reshape(*c.shape[:-1], c.shape[-1] // per, per)
    shifts = (np.arange(per - 1, -1, -1) * bits).astype(np.uint32)
    return (g << shifts).sum(-1).astype(np.uint8)


def byte_lut(levels: np.ndarray, bits: int) -> np.ndarray:
    """QUASAR_KV.py:1194-1202: the (256, 8/bits) table taking one stored byte to the levels of its
    codes, first code first."""
    per = 8 // bits
    byte = np.arange(256)[:, None]
    shifts = np.arange(per - 1, -1, -1)[None, :] * bits
    return np.asarray(levels)[(byte >> shifts) & ((1 << bits) - 1)]


def unpack_rows_lut(packed: np.ndarray, bits: int, levels: np.ndarray) -> np.ndarray:
    """Decode of pack_rows bytes by one gather per byte through byte_lut."""
    p = np.asarray(packed, dtype=np.uint8)
    return byte_lut(levels, bits)[p].reshape(*p.shape[:-1], p.shape[-1] * (8 // bits))


def unpack_codes(packed: np.ndarray, bits: int, count: int) -> np.ndarray:
    """Inverse of pack_codes: the first ``count`` codes (uint8)."""
    p = np.asarray(packed, dtype=np.uint8)
    bitsarr = np.unpackbits(p)[:count * bits].reshape(count, bits).astype(np.uint16)
    w = (1 << np.arange(bits - 1, -1, -1)).astype(np.uint16)
    return (bitsarr * w).sum(1).astype(np.uint8)


def kivi_state_bits(n_q: int, n_exact: int, d: int, bits: int, group: int) -> float:
    """Analytic stored bits of one (b, h) pair of a KIVI layer (LayerMethod.state_bits,
    STRATA_KV.py:773-783, with KIVIMethod.entry_bits 798-799 and kivi_effective_bits 465-466):
    2 d (bits + 32 / group) per quantised token, 2 d 16 per exact row."""
    return n_q * 2 * d * (bits + 32.0 / group) + n_exact * 2 * d * 16.0


def kivi_payload_sections(K: np.ndarray, V: np.ndarray, bits: int, group_k: int, group_v: int, n_q: int):
    """The quantised part of the KIVI payload (payload_bytes, STRATA_KV.py:2736-2769) of K, V
    (B, H, T, d) float32 whose first n_q rows are read quantised: per section, the bytes of every
    (b, h) in order -- pack_codes of the key codes, fp16 key lo, fp16 key scale (the ceil(n_q /
    group_k) groups that hold those rows), pack_codes of the value codes, fp16 value lo and scale
    of the n_q rows.  Keys are grouped over all T rows, as kivi_quant over the whole tensor does."""
    B, H, T, d = K.shape
    kq = kivi_quant(K, bits, group_k, True, 0)
    vq = kivi_quant(V, bits, group_v, False, 0)
    n_g = -(-n_q // group_k)
    sec = [b"", b"", b"", b"", b"", b""]
    for b in range(B):
        for h in range(H):
            sec[0] += pack_codes(kq["codes"][b, h, :n_q], bits).tobytes()
            sec[1] += kq["lo"][b, h, :n_g].astype(np.float16).tobytes()
            sec[2] += kq["scale"][b, h, :n_g].astype(np.float16).tobytes()
            sec[3] += pack_codes(vq["codes"][b, h, :n_q], bits).tobytes()
            sec[4] += vq["lo"][b, h, :n_q].astype(np.float16).tobytes()
            sec[5] += vq["scale"][b, h, :n_q].astype(np.float16).tobytes()
    return sec
