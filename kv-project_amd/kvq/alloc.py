"""STRATA rate allocation on the GPU: the allocation steps of the compression side of one layer.

Reference behaviour (STRATA_KV.py):
  * ``StrataMethod.compress_layer`` (1528-1581): from the distortion table D (Hkv, n, nb + 2) of
    every coded token under each option [drop | b_1 .. b_nb bits | exact], the per-head importance
    order (1560), the head-summed table in rank order (1561), the per-token costs, fixed bits and
    budget (1562-1567), the search (1569; nothing but drops when the budget cannot pay the level
    histogram, 1567-1568), the monotone allocation ``lev`` and its histogram (1570-1571), the bits
    and distortion ratio it reports (1573-1581).
  * ``head_sync_allocate`` (1307-1351): Lagrangian relaxation (Everett, 1963) with the multiplier
    bracketed by ``rounds`` batched passes of 32 log-spaced multipliers.
``strata_allocate`` runs the table-to-allocation steps in one call of kvq_strata_allocate (search
in float64 on the device); ``allocate_layer`` adds the host bookkeeping of compress_layer.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import torch

from . import _lib


def layer_costs(bits, d: int, Hkv: int, H: int, keep: float, rs: int, re: int):
    """(cost (nb + 2,), fixed (nb + 1,), budget, hist_bits, cost_tok) in float64, as
    compress_layer computes them (STRATA_KV.py:1562-1567): cost_tok = [0, 2 (b d + 16) per width,
    2 d 16]; cost = cost_tok Hkv; fixed = histogram bits (+ fp16 means of both sides once
    anything is coded); budget = keep H Hkv 2 d 16 minus the sinks' and window's exact rows."""
    nb = len(bits)
    cost_tok = np.array([0.0] + [2.0 * (b * d + 16) for b in bits] + [2.0 * d * 16])
    hist_bits = (nb + 2) * 32.0
    fixed = np.where(np.arange(nb + 1) > 0, Hkv * 2 * d * 16.0, 0.0) + hist_bits
    budget = keep * H * Hkv * 2 * d * 16.0 - (rs + (H - re)) * Hkv * 2 * d * 16.0
    return cost_tok * Hkv, fixed, float(budget), hist_bits, cost_tok


class AllocWorkspace:
    """Device scratch of kvq_strata_allocate for one (Hkv, n, nlev), reusable across calls."""

    def __init__(self, Hkv: int, n: int, nlev: int, device):
        nbytes = _lib.load().kvq_strata_allocate_workspace(Hkv, n, nlev)
        if nbytes < 0:
            raise _lib.KVQError(f"kvq_strata_allocate_workspace: bad shape (Hkv={Hkv}, n={n}, nlev={nlev})")
        self.key = (Hkv, n, nlev)
        self.buf = torch.empty(int(nbytes), dtype=torch.uint8, device=device)


@torch.no_grad()
def strata_allocate(D: torch.Tensor, cost, fixed, budget: float, rounds: int = 4, search: bool = True,
                    workspace: AllocWorkspace | None = None) -> dict:
    """D (Hkv, n, nlev) float32 on the GPU -> dict of device tensors order (Hkv, n), dsort (n, nlev),
    choice (n,), lev (n,), counts (nlev,) and summary [bits, cap, distortion] (float64).
    ``search`` False gives the all-drop allocation (no search)."""
    _lib.require_gpu(D)
    if D.dtype != torch.float32 or D.dim() != 3:
        raise TypeError("D must be float32 (Hkv, n, nlev)")
    D = D.contiguous()
    Hkv, n, nlev = D.shape
    cost = np.ascontiguousarray(cost, dtype=np.float64)
    fixed = np.ascontiguousarray(fixed, dtype=np.float64)
    if cost.shape != (nlev,) or fixed.shape != (nlev - 1,):
        raise ValueError(f"cost must have nlev = {nlev} entries and fixed nlev - 1")
    if workspace is None or workspace.key != (Hkv, n, nlev):
        workspace = AllocWorkspace(Hkv, n, nlev, D.device)
    dev = D.device
    i32 = dict(dtype=torch.int32, device=dev)
    out = {"order": torch.empty((Hkv, n), **i32), "dsort": torch.empty((n, nlev), dtype=torch.float32, device=dev),
           "choice": torch.empty(n, **i32), "lev": torch.empty(n, **i32), "counts": torch.empty(nlev, **i32),
           "summary": torch.empty(3, dtype=torch.float64, device=dev)}
    dp = C.POINTER(C.c_double)
    _lib.call("kvq_strata_allocate", D.data_ptr(), Hkv, n, nlev, cost.ctypes.data_as(dp), fixed.ctypes.data_as(dp),
              float(budget), int(rounds) if search else -1, out["order"].data_ptr(), out["dsort"].data_ptr(),
              out["choice"].data_ptr(), out["lev"].data_ptr(), out["counts"].data_ptr(), out["summary"].data_ptr(),
              workspace.buf.data_ptr(), workspace.buf.numel(), _lib.stream_of(D))
    return out


@torch.no_grad()
def strata_distortion(K: torch.Tensor, V: torch.Tensor, A: torch.Tensor, W: torch.Tensor, DD: torch.Tensor,
                      S: torch.Tensor, Mbar: torch.Tensor, bits) -> dict:
    """The distortion table of compress_layer (STRATA_KV.py:1541-1559) from the coverage statistics:
    K, V (Hkv, n, 128) the coded rows [rs, re) of one layer (any float dtype); A, W, DD (Hkv, n) and
    S, Mbar (Hkv, 128, 128) float32 as ``coverage_stats`` returns them.  Returns D (Hkv, n,
    len(bits) + 2) float32 [drop | widths | exact] and the centred, rotated rows (mu_k, y_k, mu_v,
    y_v) the code is then cut from (``kvq.strata_quantize_planar`` with the allocation's order)."""
    from .strata import rotation_signs, strata_center_rotate, uniform_step
    _lib.require_gpu(K, V, A, W, DD, S, Mbar)
    Hkv, n, d = K.shape
    if V.shape != K.shape or d != 128:
        raise ValueError("K, V must be (Hkv, n, 128)")
    for nm, t, shape in (("A", A, (Hkv, n)), ("W", W, (Hkv, n)), ("DD", DD, (Hkv, n)), ("S", S, (Hkv, d, d)),
                         ("Mbar", Mbar, (Hkv, d, d))):
        if t.dtype != torch.float32 or tuple(t.shape) != shape:
            raise ValueError(f"{nm} must be float32 {shape}")
    signs = rotation_signs(d, device=K.device)
    mu_k, yk = strata_center_rotate(K[None], signs)
    mu_v, yv = strata_center_rotate(V[None], signs)
    nb = len(bits)
    D = torch.empty((Hkv, n, nb + 2), dtype=torch.float32, device=K.device)
    ws = torch.empty(int(_lib.load().kvq_strata_distortion_workspace(Hkv, n, nb)) // 4 + 1, dtype=torch.float32,
                     device=K.device)
    b_arr = (C.c_int * nb)(*bits)
    s_arr = (C.c_float * nb)(*[uniform_step(b)[0] for b in bits])
    c = lambda t: t.contiguous()
    S_, M_, A_, W_, DD_ = c(S), c(Mbar), c(A), c(W), c(DD)
    _lib.call("kvq_strata_distortion", yk.data_ptr(), yv.data_ptr(), Hkv, n, d, S_.data_ptr(), M_.data_ptr(),
              signs.data_ptr(), A_.data_ptr(), W_.data_ptr(), DD_.data_ptr(), nb, b_arr, s_arr, D.data_ptr(),
              ws.data_ptr(), ws.numel() * 4, _lib.stream_of(K))
    return {"D": D, "mu_k": mu_k[0], "y_k": yk[0], "mu_v": mu_v[0], "y_v": yv[0]}


@torch.no_grad()
def allocate_layer(D: torch.Tensor, bits, d: int, H: int, keep: float, rs: int, re: int, rounds: int = 4,
                   workspace: AllocWorkspace | None = None) -> dict:
    """The allocation part of compress_layer (STRATA_KV.py:1559-1581) for a layer whose table D
    (Hkv, re - rs, nb + 2) is given: order, lev (device), counts (host list, the one host
    synchronisation, as in the reference), n_ex, n_c, bits, fixed, cost_tok, distortion."""
    Hkv, n, nlev = D.shape
    nb = len(bits)
    if nlev != nb + 2 or n != re - rs:
        raise ValueError("D must be (Hkv, re - rs, len(bits) + 2)")
    cost, fixed_np, budget, hist_bits, cost_tok = layer_costs(bits, d, Hkv, H, keep, rs, re)
    out = strata_allocate(D, cost, fixed_np, budget, rounds, search=budget >= hist_bits, workspace=workspace)
    cnt = out["counts"].tolist()
    coded = [o for o in range(1, nb + 1) if cnt[o]]
    cap = max(coded) if coded else 0
    bits_f = float(sum(cnt[o] * cost_tok[o] * Hkv for o in coded) + fixed_np[min(cap, 1)])
    return {"H": H, "rs": rs, "re": re, "order": out["order"], "lev": out["lev"], "counts": cnt,
            "n_ex": cnt[nb + 1], "n_c": int(sum(cnt[1:nb + 1])), "bits": bits_f, "fixed": float(fixed_np[min(cap, 1)]),
            "cost_tok": cost_tok, "distortion": float(out["summary"][2]), "search_bits": float(out["summary"][0])}
