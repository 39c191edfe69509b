"""STRATA decoder state and kernel wrapper with the reference's call shapes.

* ``StrataState(Ke, Ve, packed, extra, H, R)`` -- StrataState (STRATA_KV.py:1710-1818): the exact
  rows of a layer (sinks, exact-level tokens, window; model dtype) with room for ``extra``
  appended rows, and ``packed`` = StrataMethod.pack's stored code (1611-1627).  ``append``,
  ``attend``, ``context_bytes``, ``check_kernel``, fields ``n``, ``n0``, ``H``, ``shared``,
  ``use_kernel``, ``p``, ``R``; DecodeCtl drives it like any layer state.  ``attend`` runs every
  stratum and the exact rows in one libkvq launch plus the merge (kvq_strata_decode); there is no
  second implementation, so a failed ``check_kernel`` raises instead of switching paths.
* ``strata_tier_kernel(qr, qb, t, target_programs=512) -> (m, l, acc, z)`` -- the reference's
  kernel wrapper (1450-1469): flash-decoding partials of one stratum for a pre-rotated query, in
  its output layout and units (libkvq kvq_strata_tier_partials).
* ``strata_pack(cache, counts=None)`` -- a StrataCache's code as StrataMethod.pack's dict.

The tier dict is the reference's: ``{bits, n, kc, ks, vc, vs}`` with planar key / value rows
(Hkv, n, d*bits/8) uint8 and fp16 scales (Hkv, n).  The decode reads the key rows as they are and
the values through their decode tiles (kvq_strata_v_tile), built once per state (and, for
``strata_tier_kernel``, once per tier dict: kept in the dict under ``"_kvq_layout"``).
"""
from __future__ import annotations

import math
from typing import Dict, List, Optional

import torch

from . import _lib
from .strata import StrataCache, StrataTier, rotation_signs, strata_decode, strata_v_tile, unpack_planar


def _signs_of(R: torch.Tensor) -> torch.Tensor:
    """The +-1 vector s of a rotation R = H_d diag(s) / sqrt(d) (row 0 of H_d is all ones), checked
    against the whole matrix: the decode kernel rotates by that Hadamard form only."""
    d = R.shape[-1]
    Rf = R.detach().float().cpu()
    s = torch.sign(Rf[0])
    if bool((s == 0).any()):
        raise ValueError("R is not a signed Hadamard rotation H diag(s) / sqrt(d)")
    Hm = torch.ones((1, 1))
    while Hm.shape[0] < d:
        Hm = torch.cat([torch.cat([Hm, Hm], 1), torch.cat([Hm, -Hm], 1)], 0)
    # R may come rounded to the model dtype (native_state passes rot(d).to(dtype))
    tol = 4e-3 / math.sqrt(d)
    if float((Rf - Hm / math.sqrt(d) * s[None, :]).abs().max()) > tol:
        raise ValueError("R is not a signed Hadamard rotation H diag(s) / sqrt(d)")
    return s


def _tier_layout(t: Dict, device) -> Dict:
    """Decode layout of a reference tier dict (batch 1 or a leading batch dim): padded key scales
    and value tiles, built once and kept in the dict."""
    key = (t["kc"].data_ptr(), t["vc"].data_ptr(), t["ks"].data_ptr(), t["vs"].data_ptr(), int(t["n"]),
           int(t["bits"]))
    lay = t.get("_kvq_layout")
    if lay is not None and lay["key"] == key:
        return lay
    bits, n = int(t["bits"]), int(t["n"])
    kc = t["kc"].to(device)
    vc = t["vc"].to(device)
    ks = torch.as_tensor(t["ks"]).to(device, torch.float16)
    vs = torch.as_tensor(t["vs"]).to(device, torch.float16)
    if kc.dim() == 3:
        kc, vc, ks, vs = kc[None], vc[None], ks[None], vs[None]
    B, Hkv = kc.shape[:2]
    if tuple(kc.shape[2:]) != (n, 16 * bits) or tuple(vc.shape[2:]) != (n, 16 * bits) or \
            tuple(ks.shape[2:]) != (n,) or tuple(vs.shape[2:]) != (n,):
        raise ValueError("tier tensors must be kc, vc (Hkv, n, d*bits/8) and ks, vs (Hkv, n) with d = 128")
    cap = max(32, -(-n // 32) * 32)
    vt, vsl = strata_v_tile(vc.contiguous(), vs.contiguous(), bits, cap)
    ksp = torch.zeros((B, Hkv, cap), dtype=torch.float16, device=device)
    ksp[:, :, :n] = ks
    lay = {"key": key, "tier": StrataTier(bits, n, kc.contiguous(), ksp, vt, vsl, cap, vc, vs)}
    t["_kvq_layout"] = lay
    return lay


@torch.no_grad()
def strata_tier_kernel(qr: torch.Tensor, qb: torch.Tensor, t: Dict, target_programs: int = 512):
    """Partials of one stratum (STRATA_KV.py:1450-1469): qr (Hkv, rows, d) rotated, scaled query,
    qb (Hkv, rows) logit of the mean key.  Returns m, l (Hkv, S, rows), acc (Hkv, S, rows, d) in the
    rotated value basis and z (Hkv, S, rows), natural exponent; the value offset is folded into acc
    (z = 0), which StrataState.attend's merge sums the same way.  S follows the reference's split
    rule (64-token units, about ``target_programs`` programs of 16 rows)."""
    _lib.require_gpu(qr, qb)
    Hkv, rows, d = qr.shape
    n, bits = int(t["n"]), int(t["bits"])
    if n <= 0:
        raise ValueError("empty stratum")
    BR, BN = 16, 64
    cdiv = lambda a, b: -(-a // b)
    rb = cdiv(rows, BR)
    n_split = max(1, min(cdiv(n, BN), cdiv(target_programs, Hkv * rb)))
    per = cdiv(cdiv(n, n_split), BN) * BN
    n_split = cdiv(n, per)
    tier = _tier_layout(t, qr.device)["tier"]
    if tier.kc.shape[0] != 1 or tier.kc.shape[1] != Hkv:
        raise ValueError("the tier must hold the query's Hkv heads (batch 1)")
    dev = qr.device
    m = torch.empty((Hkv, n_split, rows), dtype=torch.float32, device=dev)
    l, z = torch.empty_like(m), torch.empty_like(m)
    acc = torch.empty((Hkv, n_split, rows, d), dtype=torch.float32, device=dev)
    qr = qr.float().contiguous()
    qb = qb.float().contiguous()
    _lib.call("kvq_strata_tier_partials", qr.data_ptr(), qb.data_ptr(), Hkv, rows, d, bits, n, tier.kc.data_ptr(),
              tier.ks.data_ptr(), tier.vt.data_ptr(), tier.vsl.data_ptr(), tier.cap, n_split, m.data_ptr(),
              l.data_ptr(), acc.data_ptr(), z.data_ptr(), _lib.stream_of(qr))
    return m, l, acc, z


def strata_pack(cache: StrataCache, counts: Optional[List[int]] = None) -> Dict:
    """The code of a StrataCache as StrataMethod.pack returns it (STRATA_KV.py:1611-1627): tiers best
    precision first, each {bits, n, kc, ks, vc, vs} (planar rows (Hkv, n, d*bits/8), fp16 scales
    (Hkv, n)), the level histogram ``counts`` (int32; given, or [dropped = 0, per width 2/4/8,
    exact = 0]), n_c and the fp16 means (Hkv, d).  A batch-1 cache gives the reference's shapes; a
    larger batch keeps a leading batch dim on every tensor (StrataState takes both)."""
    one = cache.mu_k.shape[0] == 1
    sq = (lambda x: x[0].contiguous()) if one else (lambda x: x.contiguous())
    tiers = []
    for t in sorted((t for t in cache.tiers if t.n > 0), key=lambda t: -t.bits):
        tiers.append({"bits": t.bits, "n": t.n, "kc": sq(t.kc), "ks": sq(t.ks[:, :, :t.n]), "vc": sq(t.vc),
                      "vs": sq(t.vs)})
    n_c = sum(t["n"] for t in tiers)
    if counts is None:
        by_bits = {t["bits"]: t["n"] for t in tiers}
        counts = [0] + [by_bits.get(b, 0) for b in (2, 4, 8)] + [0]
    out = {"tiers": tiers, "counts": torch.tensor(counts, dtype=torch.int32), "n_c": n_c}
    if n_c:
        out["mu_k"], out["mu_v"] = sq(cache.mu_k), sq(cache.mu_v)
    return out


def _tensor_bytes(xs) -> int:
    """Bytes of a nested list of tensors (tensor_bytes, STRATA_KV.py:2718-2725)."""
    if isinstance(xs, torch.Tensor):
        return xs.numel() * xs.element_size()
    return sum(_tensor_bytes(x) for x in xs)


class StrataState:
    """Compressed cache of one layer as the decoder holds it (StrataState, STRATA_KV.py:1710-1818).

    ``Ke``, ``Ve`` (B, Hkv, n0, d): exact rows; ``packed``: StrataMethod.pack's dict (or None: exact
    rows only); ``extra`` rows of room for appended tokens; ``H`` the position of the first
    appended token; ``R`` the rotation (rotation_matrix(d, "strata"), possibly in the model dtype).
    The reference holds batch 1; here B >= 1 with tier tensors carrying a leading batch dim when
    B > 1 (every sequence with the same stratum sizes)."""

    def __init__(self, Ke: torch.Tensor, Ve: torch.Tensor, packed: Optional[Dict], extra: int, H: int,
                 R: torch.Tensor):
        _lib.require_gpu(Ke, Ve)
        B, Hkv, n0, d = Ke.shape
        dev = Ke.device
        self.K = Ke.new_zeros((B, Hkv, n0 + extra, d))
        self.V = Ve.new_zeros((B, Hkv, n0 + extra, d))
        self.K[:, :, :n0], self.V[:, :, :n0] = Ke, Ve
        self.n0 = self.n = n0
        self.dtype = Ke.dtype
        if packed is not None and packed["n_c"]:
            # as the reference: the stored fp16 means are read in the model dtype
            packed = {**packed, "mu_k": packed["mu_k"].to(self.dtype), "mu_v": packed["mu_v"].to(self.dtype)}
        self.H, self.shared, self.p, self.R = H, None, packed, R
        self.use_kernel = True
        # exact rows: the first n0 always visible, appended row i at position H + i (causal)
        self.exact_pos = torch.full((n0 + extra,), -(1 << 62), dtype=torch.int64, device=dev)
        self.exact_pos[n0:] = H + torch.arange(extra, device=dev)
        signs = _signs_of(R).to(dev) if packed is not None and packed["n_c"] else rotation_signs(d, device=dev)
        tiers = []
        if packed is not None and packed["n_c"]:
            for t in packed["tiers"]:
                if int(t["n"]) > 0:
                    tiers.append(_tier_layout(t, dev)["tier"])
            mu = lambda x: (x if x.dim() == 3 else x[None]).to(dev).to(torch.float16).contiguous()
            mu_k, mu_v = mu(packed["mu_k"]), mu(packed["mu_v"])
        else:
            mu_k = mu_v = torch.zeros((B, Hkv, d), dtype=torch.float16, device=dev)
        for t in tiers:
            if t.kc.shape[:2] != (B, Hkv):
                raise ValueError("tier tensors must hold the exact rows' (B, Hkv)")
        self.cache = StrataCache(mu_k, mu_v, signs, tiers, self.K, self.V, n0, self.exact_pos)

    def context_bytes(self) -> int:
        """Bytes of the stored context: exact rows + the packed strata (STRATA_KV.py:1729-1735)."""
        p = self.p
        coded = 0
        if p is not None:
            coded = _tensor_bytes([[[t[x] for x in ("kc", "vc", "ks", "vs")] for t in p["tiers"]], p["counts"]] +
                                  [p[x] for x in ("mu_k", "mu_v") if x in p])
        return _tensor_bytes([self.K[:, :, :self.n0], self.V[:, :, :self.n0]]) + coded

    def append(self, k: torch.Tensor, v: torch.Tensor, pos) -> None:
        """Append t exact rows (STRATA_KV.py:1743-1748)."""
        t = k.shape[2]
        if self.n + t > self.K.shape[2]:
            raise RuntimeError("decode buffer exhausted")
        self.K[:, :, self.n:self.n + t], self.V[:, :, self.n:self.n + t] = k, v
        self.n += t
        self.cache.n_exact = self.n

    def attend(self, q: torch.Tensor, scaling: float, qpos, chunk=None) -> torch.Tensor:
        """q (B, Hq, Tq, d) at positions ``qpos`` -> (B, Tq, Hq, d) in q's dtype (STRATA_KV.py:1762-1795):
        the exact rows (appended ones causal), every stratum read from its packed bytes, merged, the
        coded sum rotated back once and (sum p) mu_V added.  Any Tq (query pieces of at most
        8 // rep tokens, and at most ``chunk``)."""
        if not self.use_kernel:
            raise RuntimeError("StrataState: the HIP decode kernel is disabled (check_kernel failed)")
        qp = torch.as_tensor(qpos, dtype=torch.int64).reshape(-1).to(q.device)
        if qp.numel() != q.shape[2]:
            raise ValueError("qpos must hold one position per query token")
        return strata_decode(q.to(self.dtype), scaling, self.cache, q_pos=qp, chunk=chunk).to(q.dtype)

    @torch.no_grad()
    def reconstruct(self, b: int = 0):
        """The coded tokens of sequence b decoded back to key and value rows, float32 (Hkv, n_c, d):
        every stratum's stored code read through unpack_planar and its per-vector scales, then taken
        out of the rotated basis and re-centred, x = s (c - (2^bits - 1) / 2) R + mu (the inverse of
        compress_layer's Y = (X - mu) R^T, STRATA_KV.py:1546-1548).  Strata in storage order."""
        p, d = self.p, self.K.shape[-1]
        Hkv = self.K.shape[1]
        if p is None or not p["n_c"]:
            z = torch.zeros((Hkv, 0, d), device=self.K.device)
            return z, z.clone()
        one = lambda x: x if x.dim() == (3 if x.dtype == torch.uint8 else 2) else x[b]
        Rf = self.R.float().to(self.K.device)
        mu_k = (p["mu_k"] if p["mu_k"].dim() == 2 else p["mu_k"][b]).float().to(self.K.device)
        mu_v = (p["mu_v"] if p["mu_v"].dim() == 2 else p["mu_v"][b]).float().to(self.K.device)
        ks_rows, vs_rows = [], []
        for t in p["tiers"]:
            n, bits = int(t["n"]), int(t["bits"])
            if n == 0:
                continue
            mid = (2 ** bits - 1) / 2.0
            for src, scale, mu, acc in ((t["kc"], t["ks"], mu_k, ks_rows), (t["vc"], t["vs"], mu_v, vs_rows)):
                codes = unpack_planar(one(src).to(self.K.device), bits).float()            # (Hkv, n, d)
                y = (codes - mid) * one(torch.as_tensor(scale)).to(self.K.device).float()[..., None]
                acc.append(y @ Rf + mu[:, None, :])
        return torch.cat(ks_rows, 1), torch.cat(vs_rows, 1)

    @torch.no_grad()
    def reference_attend(self, q: torch.Tensor, scaling: float, qpos) -> torch.Tensor:
        """The gate check_kernel holds the kernel to: one dense float32 softmax, per sequence, over the
        exact rows (appended ones causal) and the coded tokens' reconstructed rows (``reconstruct``).
        The reference's decode identity (STRATA_KV.py:1983-1985) states that its compressed-domain
        decode equals attention over the reconstruction; this computes the right-hand side."""
        B, Hq, Tq, d = q.shape
        Hkv = self.K.shape[1]
        rep = Hq // Hkv
        qp = torch.as_tensor(qpos, device=q.device).reshape(-1)
        pos = self.exact_pos[:self.n]                                   # (n,) -2^62 for the first n0
        outs = []
        for b in range(B):
            kr, vr = self.reconstruct(b)
            keys = torch.cat([self.K[b, :, :self.n].float(), kr], 1)   # (Hkv, n + n_c, d)
            vals = torch.cat([self.V[b, :, :self.n].float(), vr], 1)
            # visibility per query token: exact row i iff pos[i] <= qpos[t]; every coded token
            vis = torch.cat([pos[None, :] <= qp[:, None],
                             torch.ones((Tq, kr.shape[1]), dtype=torch.bool, device=q.device)], 1)
            qg = q[b].float().reshape(Hkv, rep, Tq, d)
            s = torch.matmul(qg, keys[:, None].transpose(-1, -2)) * scaling              # (Hkv, rep, Tq, N)
            s = s.masked_fill(~vis, float("-inf"))
            o = torch.matmul(s.softmax(-1), vals[:, None])                               # (Hkv, rep, Tq, d)
            outs.append(o.reshape(Hq, Tq, d).transpose(0, 1))
        return torch.stack(outs).to(q.dtype).contiguous()

    @torch.no_grad()
    def check_kernel(self, tol: float = 2e-2) -> Dict:
        """Relative max error of the kernel against reference_attend on seeded random queries
        (STRATA_KV.py:1797-1817).  Raises when it exceeds ``tol``: there is no other path."""
        g = torch.Generator(device="cpu").manual_seed(42)
        B, Hkv, d = self.K.shape[0], self.K.shape[1], self.K.shape[-1]
        q = torch.randn(B, Hkv * 4, 2, d, generator=g).to(self.K.device, self.dtype)
        qpos = torch.tensor([self.H, self.H + 1])
        ref = self.reference_attend(q, d ** -0.5, qpos).float()
        out = self.attend(q, d ** -0.5, qpos).float()
        err = float((out - ref).abs().max() / ref.abs().max().clamp_min(1e-30))
        self.use_kernel = err <= tol
        if not self.use_kernel:
            raise RuntimeError(f"StrataState.check_kernel: relative error {err:.3e} > {tol}")
        return {"kernel": True, "kernel_rel_err": err}
