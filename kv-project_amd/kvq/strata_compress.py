"""STRATA compression of one layer on the device, end to end, in the reference's call shapes.

Reference (STRATA_KV.py, StrataMethod):
  * ``compress_layer(li, q, k, v, scaling, H)`` 1528-1581: coverage statistics of the layer's own
    queries (1540), metrics in the code basis (1546), each side centred, rotated and quantised at
    every width with its per-token error e^T M e (1547-1555), the distortion table D (1556-1558),
    the allocation (1559-1571) and the report (1572-1581);
  * ``strata(al)`` 1583-1590: the coded strata, best precision first, after the exact-level tokens;
  * ``pack(al)`` 1611-1627: the stored code (planar codes and fp16 scales per stratum, fp16 means,
    the int32 level histogram);
  * ``payload(li)`` 1667-1671: measured bytes of that code (tensor_bytes, 2718-2725);
  * ``native_state(li, K, V, extra, dtype)`` 1673-1687: the decoder's StrataState.

Every step with arithmetic runs on the GPU: ``kvq.coverage_stats`` (kvq_coverage_stats),
``kvq.strata_distortion`` (centring, rotation, metrics, per-width errors, D), ``kvq.allocate_layer``
(kvq_strata_allocate: order, head sum, Lagrangian search, lev, histogram, distortion ratio) and
``kvq.strata_quantize_planar`` (quantise + planar packing) of each stratum's rows (the order's rows of that width).
The one host synchronisation is the histogram's, as in the reference (1571).  Batch 1, as the
reference's compression (1533).
"""
from __future__ import annotations

from typing import Dict, List, Optional, Tuple

import torch

from .alloc import AllocWorkspace, allocate_layer, strata_distortion
from .coverage import coverage_stats
from .strata import rotation_signs, strata_quantize_planar
from .strata_state import StrataState, _tensor_bytes

# the Config fields compress_layer reads beyond coverage_stats', with the reference's defaults
_DEFAULTS = {"N_SINK": 4, "WINDOW": 32, "STRATA_BITS": (2, 4, 8), "STRATA_ROUNDS": 4}


def _cfg(cfg, name):
    return getattr(cfg, name, _DEFAULTS[name]) if cfg is not None else _DEFAULTS[name]


def rotation_matrix(d: int, key: str = "strata", device="cuda") -> torch.Tensor:
    """rotation_matrix(d, key) (STRATA_KV.py:1110-1128): H_d diag(s) / sqrt(d), float32."""
    s = rotation_signs(d, key, device="cpu").to(torch.float64)
    Hm = torch.ones((1, 1), dtype=torch.float64)
    while Hm.shape[0] < d:
        Hm = torch.cat([torch.cat([Hm, Hm], 1), torch.cat([Hm, -Hm], 1)], 0)
    return (Hm * s[None, :] / d ** 0.5).to(torch.float32).to(device)


class StrataCompressor:
    """The compression side of StrataMethod for one model: ``keep`` the kept fraction of the exact
    context's bits (STRATA_KV.py:1564), ``cfg`` any object with the reference's Config fields
    (N_SINK, WINDOW, STRATA_BITS, STRATA_ROUNDS and those coverage_stats reads; defaults otherwise),
    ``window_only`` / ``uniform`` the reference's variants (1488-1491).  The reference's rotate=False
    control (identity basis) has no device path: the decode kernels read the Hadamard basis only."""

    def __init__(self, keep: float, cfg=None, window_only: bool = False, uniform: bool = False,
                 rotate: bool = True):
        if not rotate:
            raise NotImplementedError("rotate=False: the device codec and decode use the Hadamard basis only")
        bits = tuple(_cfg(cfg, "STRATA_BITS"))
        if not set(bits) <= {2, 4, 8} or sorted(set(bits)) != list(bits):
            raise ValueError("STRATA_BITS must be increasing and drawn from {2, 4, 8} (planar byte packing)")
        self.keep, self.cfg, self.bits = float(keep), cfg, bits
        self.window_only, self.uniform = window_only, uniform
        self._ws: Dict[Tuple, AllocWorkspace] = {}

    @torch.no_grad()
    def compress_layer(self, q, k: torch.Tensor, v: torch.Tensor, scaling: float, H: int,
                       M: torch.Tensor) -> Optional[Dict]:
        """The allocation of one layer and what its code is cut from, or None when nothing is
        compressible (STRATA_KV.py:1528-1581).  q (1, Hq, T, d) or QRows, k, v (1, Hkv, T, d) on the
        GPU, M (Hq, d, d) the output metric W_O,a^T W_O,a of every query head (out_metric, 1519-1526).
        The dict carries the reference's keys (H, rs, re, order, lev, lev_cpu, counts, n_ex, n_c,
        bits, fixed, cost_tok, distortion) plus mu / y: the fp16 means and rotated rows of both
        sides, from which ``pack`` quantises each stratum."""
        c = self.cfg
        rs, re = _cfg(c, "N_SINK"), H - _cfg(c, "WINDOW")
        if re - rs <= 0 or k.shape[0] != 1:
            return None
        Hkv, d = k.shape[1], k.shape[-1]
        st = coverage_stats(q, k, v, scaling, H, rs, re, M, c, self.window_only)
        A, W, DD = st["A"], st["W"], st["DD"]
        if self.uniform:                    # importance-free control: one price per position (1542-1544)
            A, W = torch.full_like(A, float(A.mean())), torch.full_like(W, float(W.mean()))
            DD = torch.full_like(DD, float("inf"))
        dist = strata_distortion(k[0, :, rs:re], v[0, :, rs:re], A, W, DD, st["S"], st["Mbar"], self.bits)
        n, nlev = re - rs, len(self.bits) + 2
        ws = self._ws.get((Hkv, n, nlev))
        if ws is None:
            ws = self._ws[(Hkv, n, nlev)] = AllocWorkspace(Hkv, n, nlev, k.device)
        al = allocate_layer(dist["D"], self.bits, d, H, self.keep, rs, re, _cfg(c, "STRATA_ROUNDS"), workspace=ws)
        al["lev_cpu"] = al["lev"].cpu().numpy()
        al["mu"] = [dist["mu_k"], dist["mu_v"]]
        al["y"] = [dist["y_k"], dist["y_v"]]
        return al

    def strata(self, al: Dict) -> List[Tuple[int, int, int]]:
        """(option index, first sorted position, count) of every coded stratum, best precision
        first, after the exact-level tokens (STRATA_KV.py:1583-1590)."""
        nb, cnt = len(self.bits), al["counts"]
        out, start = [], cnt[nb + 1]
        for o in range(nb, 0, -1):
            if cnt[o]:
                out.append((o, start, cnt[o]))
            start += cnt[o]
        return out

    @torch.no_grad()
    def pack(self, al: Dict) -> Dict:
        """The stored code of one layer (STRATA_KV.py:1611-1627): per stratum the planar codes
        (Hkv, m, d b / 8) uint8 and fp16 scales (Hkv, m) of keys and values, rows in the order's
        ranks; the int32 histogram ``counts`` (host); n_c; the fp16 means (Hkv, d) when anything is
        coded.  Each stratum's rows are quantised at its own width only (quantisation is per row,
        so the codes equal the reference's all-rows quantisation gathered by the order)."""
        tiers = []
        for o, a, m in self.strata(al):
            idx = al["order"][:, a:a + m][None]
            b = self.bits[o - 1]
            t = {"bits": b, "n": m}
            for s, nm in ((0, "k"), (1, "v")):
                codes, scales = strata_quantize_planar(al["y"][s][None], b, idx)
                t[f"{nm}c"], t[f"{nm}s"] = codes[0], scales[0]
            tiers.append(t)
        out = {"tiers": tiers, "counts": torch.tensor(al["counts"], dtype=torch.int32), "n_c": al["n_c"]}
        if al["n_c"]:
            out["mu_k"], out["mu_v"] = al["mu"][0], al["mu"][1]
        return out

    @staticmethod
    def payload(packed: Dict) -> int:
        """Measured bytes of a stored code (StrataMethod.payload, STRATA_KV.py:1667-1671)."""
        return _tensor_bytes([[[t[x] for x in ("kc", "vc", "ks", "vs")] for t in packed["tiers"]], packed["counts"]] +
                             [packed[x] for x in ("mu_k", "mu_v") if x in packed])

    @torch.no_grad()
    def native_state(self, al: Optional[Dict], packed: Optional[Dict], K: torch.Tensor, V: torch.Tensor, extra: int,
                     dtype) -> StrataState:
        """The decoder's state of the layer (STRATA_KV.py:1673-1687): exact rows (sinks, the
        exact-level tokens of every head, the window) in ``dtype`` plus the packed strata.  K, V
        (1, Hkv, H, d): the layer's context cache."""
        H, d = K.shape[2], K.shape[-1]
        R = rotation_matrix(d, device=K.device).to(dtype)
        if al is None:
            return StrataState(K.to(dtype), V.to(dtype), None, extra, H, R)
        rs, re, n_ex = al["rs"], al["re"], al["n_ex"]
        Hkv = K.shape[1]
        dev = K.device
        ex_ids = torch.cat([torch.arange(rs, device=dev).expand(Hkv, rs), al["order"][:, :n_ex].long() + rs,
                            torch.arange(re, H, device=dev).expand(Hkv, H - re)], 1)
        Ke = K[0].gather(1, ex_ids[..., None].expand(Hkv, ex_ids.shape[1], d))[None].to(dtype)
        Ve = V[0].gather(1, ex_ids[..., None].expand(Hkv, ex_ids.shape[1], d))[None].to(dtype)
        return StrataState(Ke, Ve, packed, extra, H, R)
