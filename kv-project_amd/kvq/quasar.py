"""QUASAR compressed-domain decode: ``QuasarState`` over an embedded spectral code (libkvq
kvq_quasar_*).

Mirrors QuasarState (QUASAR_KV.py:1854-1990): exact rows in a buffer with room for appended tokens,
and the embedded code of the coded tokens -- per side one flat uint8 buffer holding every step's
(Hkv, n_s, bytes) block of pack_rows codes plus a step table [offset, n_s, bytes per row, a, w,
bits, level offset] (1883-1898).  ``attend`` reads only those bytes: the query is mapped into each
head's coefficient space once (q T_K), every K step adds q~[band] . level[code] for the tokens
owning it, one softmax covers exact rows and coded tokens, and the coded tokens' weighted levels
are lifted back once (acc T_V^T + P mu_V).  The kernel path is the only path; ``reference_attend``
(dense attention over the stored code decoded back to rows, ``reconstruct``) exists for
``check_kernel``.
"""
from __future__ import annotations

import ctypes as C
from functools import lru_cache
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np
import torch

from . import _lib
from .query import decode_in_pieces, query_pieces

MAX_SPLITS = 1024


# ---- codebooks (host-side set-up, computed once per stage tuple) --------------------------------

@lru_cache(maxsize=None)
def lloyd_max_gaussian(bits: int) -> np.ndarray:
    """Lloyd-Max levels of N(0, 1) with 2^bits cells (STRATA_KV.py:1082-1098)."""
    from scipy import stats
    n = 2 ** bits
    x = np.linspace(-9.0, 9.0, 360001)
    w = np.exp(-0.5 * x * x)
    w /= w.sum()
    c = stats.norm.ppf((np.arange(n) + 0.5) / n)
    for _ in range(500):
        cell = np.searchsorted((c[1:] + c[:-1]) / 2, x)
        mass = np.bincount(cell, w, n)
        c = np.bincount(cell, w * x, n) / np.maximum(mass, 1e-300)
    return c.astype(np.float32)


@lru_cache(maxsize=None)
def stage_codebooks(stage_bits: Tuple[int, ...]) -> List[np.ndarray]:
    """Embedded residual Lloyd-Max levels of every stage (QUASAR_KV.py:1143-1169), float32."""
    from scipy import stats
    x = stats.norm.ppf((np.arange(200000) + 0.5) / 200000)
    cur, out = np.zeros_like(x), []
    for t, b in enumerate(stage_bits):
        r = x - cur
        if t == 0:
            c = lloyd_max_gaussian(b).astype(np.float64)
        else:
            n = 2 ** b
            c = np.quantile(r, (np.arange(n) + 0.5) / n)
            for _ in range(150):
                cell = np.searchsorted((c[1:] + c[:-1]) / 2, r)
                c = np.bincount(cell, r, n) / np.maximum(np.bincount(cell, None, n), 1)
        cur = cur + c[np.searchsorted((c[1:] + c[:-1]) / 2, r)]
        out.append(c.astype(np.float32))
    return out


def band_edges(d: int, fractions: Sequence[float]) -> List[Tuple[int, int]]:
    """Bands of the coefficient basis, leading first (QUASAR_KV.py:1205-1215)."""
    widths = [max(4, int(round(d * f / 4)) * 4) for f in fractions[:-1]]
    widths.append(d - sum(widths))
    if widths[-1] < 4 or any(w % 4 for w in widths):
        raise ValueError(f"bands {tuple(fractions)} do not split head_dim {d} into multiples of 4")
    out, a = [], 0
    for w in widths:
        out.append((a, a + w))
        a += w
    return out


def pack_rows_np(codes: np.ndarray, bits: int) -> np.ndarray:
    """(..., w) codes -> (..., w bits / 8) uint8, first code in the most significant bits
    (QUASAR_KV.py:1185-1190), on the host (the compressor's side)."""
    per = 8 // bits
    c = codes.astype(np.int32).reshape(*codes.shape[:-1], codes.shape[-1] // per, per)
    shifts = np.arange(per - 1, -1, -1, dtype=np.int32) * bits
    return (c << shifts).sum(-1).astype(np.uint8)


# ---- the stored code, as the decoder holds it -----------------------------------------------

def _side_buffers(packed: Dict, side: int, stages: Tuple[int, ...], device) -> Dict:
    """Flat code buffer and step table of one side (QuasarState.__init__, 1883-1898), with the
    checks the kernel relies on: rows of 4k bytes, a power of two <= 64; n_s non-increasing."""
    books = stage_codebooks(tuple(stages))
    lvl_off = np.cumsum([0] + [len(b_) for b_ in books])[:-1]
    rows, flats, off, prev = [], [], 0, None
    for st in packed["steps"]:
        if st["side"] != side:
            continue
        codes = torch.as_tensor(st["codes"])
        if codes.dtype != torch.uint8 or codes.dim() != 3:
            raise ValueError("step codes must be uint8 (Hkv, n_s, bytes)")
        b = int(stages[st["stage"]])
        w = int(st["b"]) - int(st["a"])
        nb = int(codes.shape[-1])
        if b not in (1, 2, 4, 8) or nb * 8 != w * b or nb % 4 or nb > 64 or nb & (nb - 1):
            raise ValueError(f"step band of {w} codes at {b} bits: rows must be 4, 8, 16, 32 or 64 bytes")
        n_s = int(st["n"])
        if codes.shape[1] != n_s or (prev is not None and n_s > prev):
            raise ValueError("steps must own non-increasing token prefixes (n_s) in step order")
        prev = n_s
        rows.append([off, n_s, nb, int(st["a"]), w, b, int(lvl_off[st["stage"]])])
        flats.append(codes.reshape(-1))
        off += codes.numel()
    if not rows:
        return {"table_np": np.zeros((0, 7), np.int32), "flat": None, "table": None}
    if sum(r_[2] for r_ in rows) > 128:
        raise ValueError("at most 128 code bytes per token and side (d = 128 coefficients at 8 bits)")
    if off >= 1 << 31:
        raise ValueError("a side's code buffer must stay under 2 GiB")
    table = np.asarray(rows, dtype=np.int32)
    flat = torch.cat(flats).to(device)
    return {"table_np": table, "flat": flat, "table": torch.from_numpy(table).to(device)}


class QuasarState:
    """Compressed cache of one layer as a decoder holds it (QUASAR_KV.py:1854-1990).

    ``Ke``, ``Ve`` (1, Hkv, n0, d): the exact rows (model dtype, on the GPU); ``packed``: the stored
    code (QuasarMethod.pack, 1786-1808): steps [{side, a, b, stage, n, codes}], n_c, counts, rho_k /
    rho_v (Hkv, n_c), T_k / T_v (Hkv, d, R), mu_k / mu_v (Hkv, d); ``stages`` the stage bits;
    ``extra`` rows of room for appended tokens; ``H`` the position of the first appended token."""

    def __init__(self, Ke: torch.Tensor, Ve: torch.Tensor, packed: Optional[Dict], stages, extra: int, H: int):
        _lib.require_gpu(Ke, Ve)
        B, Hkv, n0, d = Ke.shape
        if B != 1:
            raise ValueError("QuasarState holds one sequence (batch 1), as the reference does")
        if d != 128:
            raise ValueError("the QUASAR decode needs head_dim 128")
        dev = Ke.device
        self.K = Ke.new_zeros((B, Hkv, n0 + extra, d))
        self.V = Ve.new_zeros((B, Hkv, n0 + extra, d))
        self.K[:, :, :n0], self.V[:, :, :n0] = Ke, Ve
        self.n0 = self.n = n0
        self.H, self.shared, self.p = H, None, packed
        self.dtype = Ke.dtype
        self.use_kernel = True
        self.stages = tuple(int(b) for b in stages)
        self.exact_pos = torch.full((n0 + extra,), -(1 << 62), dtype=torch.int64, device=dev)
        self.exact_pos[n0:] = H + torch.arange(extra, device=dev)
        self.n_c = int(packed["n_c"]) if packed is not None else 0
        self.sides = [None, None]
        if self.n_c > 0:
            books = stage_codebooks(self.stages)
            self.levels = torch.from_numpy(np.concatenate(books).astype(np.float32)).to(dev)
            self.sides = [_side_buffers(packed, s, self.stages, dev) for s in (0, 1)]
            for sd in self.sides:                  # a side dict as the reference's kernel wrappers take it
                sd["levels"] = self.levels
            if self.sides[0]["flat"] is None or self.sides[1]["flat"] is None:
                raise ValueError("a coded layer needs steps on both sides")
            f16 = lambda x: torch.as_tensor(x).to(dev, torch.float16).contiguous()
            f32 = lambda x: torch.as_tensor(x).to(dev, torch.float32).contiguous()
            self.rho_k, self.rho_v = f16(packed["rho_k"]), f16(packed["rho_v"])
            # T_V is taken at fp16 (its stored precision) by the lift and by the torch path alike
            self.T_k, self.T_v = f32(packed["T_k"]), f32(torch.as_tensor(packed["T_v"]).to(torch.float16))
            # (Hkv, R_v, d) fp16: the lift reads it by channel; fp16 is the precision the code stores
            self.T_vt = torch.as_tensor(packed["T_v"]).to(dev, torch.float16).transpose(1, 2).contiguous()
            self.mu_k, self.mu_v = f32(packed["mu_k"]), f32(packed["mu_v"])
            for nm, t, shape in (("rho_k", self.rho_k, (Hkv, self.n_c)), ("rho_v", self.rho_v, (Hkv, self.n_c)),
                                 ("mu_k", self.mu_k, (Hkv, d)), ("mu_v", self.mu_v, (Hkv, d))):
                if tuple(t.shape) != shape:
                    raise ValueError(f"{nm} must be {shape}")
            if self.T_k.shape[:2] != (Hkv, d) or self.T_v.shape[:2] != (Hkv, d):
                raise ValueError("T_k, T_v must be (Hkv, d, R)")
            if self.T_k.shape[-1] % 4 or self.T_v.shape[-1] % 4:
                raise ValueError("the read-out matrices' R must be a multiple of 4")
            for side, T in ((0, self.T_k), (1, self.T_v)):
                tab = self.sides[side]["table_np"]
                if int((tab[:, 3] + tab[:, 4]).max()) > T.shape[-1]:
                    raise ValueError("a step's band ends past the read-out matrix's R columns")
                if int(tab[:, 1].max()) > self.n_c:
                    raise ValueError("a step owns more tokens than n_c")
            self.bounds, self.splits = self._plan(Hkv)
        self._ws = None

    def _plan(self, Hkv: int):
        """Makespan-balanced token splits and the slot table (kvq_quasar_plan, host memory), uploaded."""
        kt, vt = self.sides[0]["table_np"], self.sides[1]["table_np"]
        bounds = np.zeros(MAX_SPLITS + 1, dtype=np.int32)
        slots = np.zeros((2, 32, 8), dtype=np.int32)
        n_slots = np.zeros(2, dtype=np.int32)
        n_splits = C.c_int32(0)
        _lib.call("kvq_quasar_plan", kt.ctypes.data, kt.shape[0], vt.ctypes.data, vt.shape[0], self.n_c, Hkv,
                  MAX_SPLITS, bounds.ctypes.data, C.addressof(n_splits), slots.ctypes.data, n_slots.ctypes.data)
        S = int(n_splits.value)
        self.slots = torch.from_numpy(slots).to(self.K.device)
        self.n_slots = (int(n_slots[0]), int(n_slots[1]))
        return torch.from_numpy(bounds[:S + 1].copy()).to(self.K.device), S

    def context_bytes(self) -> int:
        """Bytes of the stored context: exact rows + the packed code (QUASAR_KV.py:1900-1905): the
        flat code buffers, the level histogram, rho, T and mu as stored (2 bytes each)."""
        exact = 2 * self.K[:, :, :self.n0].numel() * self.K.element_size()
        if self.n_c == 0:
            return exact
        p = self.p
        counts = torch.as_tensor(p["counts"]).numel() * 4 if "counts" in p else 0
        flats = sum(s_["flat"].numel() for s_ in self.sides)
        mats = 2 * (self.rho_k.numel() + self.rho_v.numel() + self.T_k.numel() + self.T_v.numel() +
                    self.mu_k.numel() + self.mu_v.numel())
        return exact + counts + flats + mats

    def append(self, k: torch.Tensor, v: torch.Tensor, pos) -> None:
        """Append t exact rows (QUASAR_KV.py:1907-1913)."""
        t = k.shape[2]
        if self.n + t > self.K.shape[2]:
            raise RuntimeError("decode buffer exhausted")
        self.K[:, :, self.n:self.n + t], self.V[:, :, self.n:self.n + t] = k, v
        self.n += t

    def _workspace(self, Hq: int, Tq: int) -> torch.Tensor:
        Hkv, d = self.K.shape[1], self.K.shape[3]
        Rk = self.T_k.shape[-1] if self.n_c > 0 else 1
        need = _lib.load().kvq_quasar_decode_workspace(Hq, Hkv, Tq, d, Rk, self.K.shape[2], max(self.splits, 1)
                                                       if self.n_c > 0 else 1)
        if need < 0:
            raise _lib.KVQError("kvq_quasar_decode_workspace rejected the shape")
        if self._ws is None or self._ws.numel() < need:
            self._ws = torch.empty((need,), dtype=torch.float32, device=self.K.device)
        return self._ws

    @torch.no_grad()
    def attend(self, q: torch.Tensor, scaling: float, qpos, chunk=None, out: Optional[torch.Tensor] = None,
               phases: int = 7) -> torch.Tensor:
        """One decode step (QUASAR_KV.py:1945-1968): q (1, Hq, Tq, d) -> (1, Tq, Hq, d) in q's dtype.
        Appended rows are causal (row at position H + i visible to query t iff H + i <= qpos[t]).
        ``phases`` (timing hooks): mask of 1 (query coefficients), 2 (split launch), 4 (merge).
        Any Tq: query-token pieces of at most 8 // rep tokens, and at most ``chunk`` (kvq.query)."""
        _lib.require_gpu(q)
        B, Hq, Tq, d = q.shape
        if B != 1:
            raise ValueError("QuasarState.attend takes batch 1")
        pieces = query_pieces(Hq // self.K.shape[1], Tq, chunk)
        if len(pieces) > 1:
            if phases != 7:
                raise ValueError("a chunked query step runs whole steps (phases 7)")
            qp_all = torch.as_tensor(qpos, dtype=torch.int64).reshape(-1)
            if qp_all.numel() != Tq:
                raise ValueError("qpos needs one position per query row")
            return decode_in_pieces(lambda qs, qp, o: self.attend(qs, scaling, qp, out=o), q, qp_all, out, pieces)
        if q.dtype != self.dtype:
            q = q.to(self.dtype)
        if q.stride(-1) != 1:
            q = q.contiguous()
        Hkv = self.K.shape[1]
        qp = torch.as_tensor(qpos, dtype=torch.int64).reshape(-1).to(q.device)
        if qp.numel() != Tq:
            raise ValueError("qpos needs one position per query row")
        ws = self._workspace(Hq, Tq)
        out = _lib.out_or_new(out, (1, Tq, Hq, d), q.dtype, q.device, "QuasarState.attend")
        coded = self.n_c > 0
        k_s, v_s = (self.sides[0], self.sides[1]) if coded else ({}, {})
        P = _lib.ptr
        _lib.call("kvq_quasar_decode", q.data_ptr(), _lib.DTYPE_CODE[q.dtype], q.stride(1), q.stride(2), Hq, Hkv, Tq, d,
                  float(scaling), self.K.data_ptr(), self.V.data_ptr(), self.K.shape[2], self.n,
                  self.exact_pos.data_ptr(), qp.data_ptr(),
                  P(k_s.get("flat")), k_s["flat"].numel() if coded else 0,
                  P(v_s.get("flat")), v_s["flat"].numel() if coded else 0, P(self.slots) if coded else None,
                  self.n_slots[0] if coded else 0, self.n_slots[1] if coded else 0,
                  P(self.levels) if coded else None, self.levels.numel() if coded else 0,
                  P(self.rho_k) if coded else None, P(self.rho_v) if coded else None, self.n_c,
                  P(self.T_k) if coded else None, P(self.T_vt) if coded else None,
                  self.T_k.shape[-1] if coded else 0, self.T_v.shape[-1] if coded else 0,
                  P(self.mu_k) if coded else None, P(self.mu_v) if coded else None,
                  P(self.bounds) if coded else None, self.splits if coded else 0,
                  out.data_ptr(), ws.data_ptr(), ws.numel(), int(phases), _lib.stream_of(q))
        return out

    @torch.no_grad()
    def reconstruct(self):
        """The coded tokens decoded back to key and value rows, float32 (Hkv, n_c, d): each side's
        coefficients summed over the steps that own a token (every step's pack_rows bytes read through
        its stage's level table, kvq.unpack_rows), then lifted out of the coefficient basis, x = rho c T^T
        + mu -- the rows whose attention the compressed-domain decode computes (QUASAR_KV.py:1952-1966)."""
        from .kivi import unpack_rows
        Hkv, d = self.K.shape[1], self.K.shape[-1]
        dev = self.K.device
        if self.n_c == 0:
            z = torch.zeros((Hkv, 0, d), device=dev)
            return z, z.clone()
        books = [torch.from_numpy(x).to(dev) for x in stage_codebooks(self.stages)]
        rows = []
        for side, T, rho, mu in ((0, self.T_k, self.rho_k, self.mu_k), (1, self.T_v, self.rho_v, self.mu_v)):
            coef = torch.zeros((Hkv, self.n_c, T.shape[-1]), device=dev)
            for st in self.p["steps"]:
                if st["side"] != side or int(st["n"]) == 0:
                    continue
                b = self.stages[st["stage"]]
                lv = unpack_rows(torch.as_tensor(st["codes"]).to(dev), b, books[st["stage"]])   # (Hkv, n_s, w)
                coef[:, :int(st["n"]), st["a"]:st["b"]] += lv
            rows.append(rho.float()[..., None] * torch.matmul(coef, T.transpose(-1, -2)) + mu[:, None, :])
        return rows[0], rows[1]

    @torch.no_grad()
    def reference_attend(self, q: torch.Tensor, scaling: float, qpos) -> torch.Tensor:
        """The gate check_kernel holds the kernel to: one dense float32 softmax over the exact rows
        (appended ones causal) and the coded tokens' reconstructed rows (``reconstruct``) -- the
        attention the compressed-domain decode must reproduce."""
        B, Hq, Tq, d = q.shape
        Hkv = self.K.shape[1]
        rep = Hq // Hkv
        qp = torch.as_tensor(qpos, device=q.device).reshape(-1)
        kr, vr = self.reconstruct()
        keys = torch.cat([self.K[0, :, :self.n].float(), kr], 1)          # (Hkv, n + n_c, d)
        vals = torch.cat([self.V[0, :, :self.n].float(), vr], 1)
        vis = torch.cat([self.exact_pos[None, :self.n] <= qp[:, None],
                         torch.ones((Tq, kr.shape[1]), dtype=torch.bool, device=q.device)], 1)
        qg = q[0].float().reshape(Hkv, rep, Tq, d)
        s = torch.matmul(qg, keys[:, None].transpose(-1, -2)) * scaling
        o = torch.matmul(s.masked_fill(~vis, float("-inf")).softmax(-1), vals[:, None])
        return o.reshape(Hq, Tq, d).transpose(0, 1)[None].to(q.dtype).contiguous()

    @torch.no_grad()
    def check_kernel(self, tol: float = 2e-2) -> Dict:
        """Relative max error of the kernel against reference_attend on seeded random queries
        (QUASAR_KV.py:1970-1990).  Raises when it exceeds ``tol``: there is no other path."""
        g = torch.Generator(device="cpu").manual_seed(42)
        Hq = self.K.shape[1] * 4
        q = torch.randn(1, Hq, 2, self.K.shape[-1], generator=g).to(self.K.device, self.dtype)
        qpos = torch.tensor([self.H, self.H + 1])
        ref = self.reference_attend(q, self.K.shape[-1] ** -0.5, qpos).float()
        out = self.attend(q, self.K.shape[-1] ** -0.5, qpos).float()
        err = float((out - ref).abs().max() / ref.abs().max().clamp_min(1e-30))
        if err > tol:
            raise RuntimeError(f"QuasarState.check_kernel: relative error {err:.3e} > {tol}")
        return {"kernel": True, "kernel_rel_err": err}


# ---- the reference's kernel-wrapper call shapes (QUASAR_KV.py:1556-1577) --------------------

def _host_table(side: Dict) -> np.ndarray:
    t = side.get("table_np")
    if t is None:                                  # the reference keeps its table on the device
        t = torch.as_tensor(side["table"]).detach().cpu().numpy()
    return np.ascontiguousarray(np.asarray(t, dtype=np.int32).reshape(-1, 7))


def _side_parts(side: Dict, device):
    flat = side["flat"]
    levels = torch.as_tensor(side["levels"]).to(device, torch.float32).contiguous()
    if flat is not None:
        _lib.require_gpu(flat)
    return flat, levels


@torch.no_grad()
def quasar_scores(qt: torch.Tensor, side: Dict, n_c: int) -> torch.Tensor:
    """Drop-in for quasar_scores (QUASAR_KV.py:1556-1564): qt (Hkv, rows, R) the query's coefficients
    -> (Hkv, rows, n_c) float32, the sum over the key side's steps owning each coded token of
    qt[band] . levels[codes] (libkvq kvq_quasar_scores).  ``side``: a QuasarState side ({flat, table
    (or table_np), levels}), the reference's or this package's."""
    _lib.require_gpu(qt)
    Hkv, rows, R = qt.shape
    tab = _host_table(side)
    flat, levels = _side_parts(side, qt.device)
    q32 = qt.float().contiguous()
    out = torch.empty((Hkv, rows, int(n_c)), dtype=torch.float32, device=qt.device)
    _lib.call("kvq_quasar_scores", q32.data_ptr(), Hkv, rows, R, _lib.ptr(flat), 0 if flat is None else flat.numel(),
              tab.ctypes.data, tab.shape[0], levels.data_ptr(), levels.numel(), int(n_c), out.data_ptr(),
              _lib.stream_of(qt))
    return out


@torch.no_grad()
def quasar_values(pv: torch.Tensor, side: Dict, R: int) -> torch.Tensor:
    """Drop-in for quasar_values (QUASAR_KV.py:1567-1577): pv (Hkv, rows, n_c) weighted probabilities
    of the coded tokens -> (Hkv, rows, R) float32, per coefficient the sum over the value side's
    steps covering it of pv . levels[codes] (libkvq kvq_quasar_values)."""
    _lib.require_gpu(pv)
    Hkv, rows, n_c = pv.shape
    tab = _host_table(side)
    flat, levels = _side_parts(side, pv.device)
    p32 = pv.float().contiguous()
    out = torch.empty((Hkv, rows, int(R)), dtype=torch.float32, device=pv.device)
    ws = torch.empty((_lib.load().kvq_quasar_values_workspace(Hkv, rows, int(R), n_c),), dtype=torch.float32,
                     device=pv.device)
    _lib.call("kvq_quasar_values", p32.data_ptr(), Hkv, rows, n_c, _lib.ptr(flat), 0 if flat is None else flat.numel(),
              tab.ctypes.data, tab.shape[0], levels.data_ptr(), levels.numel(), int(R), out.data_ptr(), ws.data_ptr(),
              ws.numel(), _lib.stream_of(pv))
    return out


# ---- synthetic stored codes (tests and the benchmark) -------------------------------------

def default_plan(n_bands: int, n_stages: int) -> List[List[Tuple[int, int, int]]]:
    """Steps each level adds, (side, band, stage): stage 0 of every band (leading band first), then
    stage 1 of every band, ...; each level adds the same (band, stage) on both sides."""
    return [[(s, kk, t) for s in (0, 1)] for t in range(n_stages) for kk in range(n_bands)]


def synthetic_packed(Hkv: int, d: int, n_c: int, *, stages=(2, 2, 4), bands=(0.125, 0.125, 0.25, 0.5),
                     fractions: Optional[Sequence[float]] = None, seed: int = 0) -> Dict:
    """A stored code of the reference's format (QuasarMethod.pack, 1786-1808) from synthetic
    coefficients: u ~ N(0, 1) per (head, token, coefficient) and side, embedded-quantised with the
    stage codebooks; level lv keeps the fraction ``fractions[lv - 1]`` of the coded tokens (a
    non-increasing prefix); T random orthonormal, rho and mu random; all stored as fp16."""
    rng = np.random.default_rng(seed)
    edges = band_edges(d, bands)
    plan = default_plan(len(edges), len(stages))
    if fractions is None:
        fractions = np.linspace(1.0, 0.1, len(plan))
    fractions = np.asarray(fractions, dtype=np.float64)
    if len(fractions) != len(plan) or np.any(np.diff(fractions) > 0):
        raise ValueError("one non-increasing fraction per level")
    n_s = np.maximum(0, np.minimum(n_c, np.round(fractions * n_c).astype(np.int64)))
    n_s[0] = n_c
    books = stage_codebooks(tuple(stages))
    sides = []
    for s in (0, 1):
        u = rng.standard_normal((Hkv, n_c, d)).astype(np.float32)
        codes, cur = [], np.zeros_like(u)
        for cb in books:
            c = np.searchsorted((cb[1:] + cb[:-1]) / 2, u - cur, side="left")
            cur = cur + cb[c]
            codes.append(c.astype(np.uint8))
        sides.append(codes)
    steps = []
    for lv, adds in enumerate(plan):
        for s, kk, t in adds:
            a, b = edges[kk]
            steps.append({"side": s, "a": a, "b": b, "stage": t, "n": int(n_s[lv]),
                          "codes": torch.from_numpy(pack_rows_np(sides[s][t][:, :n_s[lv], a:b], stages[t]))})
    counts = np.zeros(len(plan) + 2, np.int32)
    counts[1:len(plan) + 1] = -np.diff(np.concatenate([n_s, [0]]))
    out = {"steps": steps, "counts": torch.from_numpy(counts), "n_c": int(n_c)}
    for nm in ("k", "v"):
        T = np.linalg.qr(rng.standard_normal((Hkv, d, d)))[0]
        out[f"T_{nm}"] = torch.from_numpy(T.astype(np.float16))
        out[f"rho_{nm}"] = torch.from_numpy((np.abs(rng.standard_normal((Hkv, n_c))) * 0.5 + 0.3).astype(np.float16))
        out[f"mu_{nm}"] = torch.from_numpy((rng.standard_normal((Hkv, d)) * 0.2).astype(np.float16))
    return out
