"""STRATA coverage statistics on the device: coverage_groups + coverage_stats (STRATA_KV.py:1206-1298).

``coverage_groups`` draws the observation positions on the host exactly as the reference does
(numpy's PCG64 seeded by CRC32 keys; the draws are pinned by golden vectors of the reference).
``coverage_stats`` builds the row plan of those groups once per shape (int32 tables on the device)
and runs ``kvq_coverage_stats``: eleven launches, no host synchronisation, deterministic sums.
"""
from __future__ import annotations

import zlib
from dataclasses import dataclass
from typing import Dict, List, Tuple

import numpy as np
import torch

from . import _lib

# the Config fields coverage_groups / coverage_stats read, with the reference's defaults
_DEFAULTS = {"N_SINK": 4, "STRATA_LOCAL": 64, "W_OBS": 32, "STRATA_SEGMENT": 512, "STRATA_QUERIES": 16,
             "STRATA_FLOOR": 1e-3}


def _cfg(cfg, name):
    return getattr(cfg, name, _DEFAULTS[name]) if cfg is not None else _DEFAULTS[name]


def _rng(*keys) -> np.random.Generator:
    """The reference's _rng: default_rng([42, crc32(str(key)) ...])."""
    return np.random.default_rng([42] + [zlib.crc32(str(k).encode()) for k in keys])


def coverage_groups(H: int, cfg=None) -> List[np.ndarray]:
    """Observation positions (STRATA_KV.py:1206-1222): one group per STRATA_SEGMENT context positions
    from N_SINK + STRATA_LOCAL (min(len, STRATA_QUERIES) positions drawn without replacement, sorted),
    then the last W_OBS positions (the window group, always last); empty groups dropped."""
    lo = _cfg(cfg, "N_SINK") + _cfg(cfg, "STRATA_LOCAL")
    win = max(lo, H - _cfg(cfg, "W_OBS"))
    seg_len, nq_max = _cfg(cfg, "STRATA_SEGMENT"), _cfg(cfg, "STRATA_QUERIES")
    groups = []
    for s in range(lo, win, seg_len):
        seg = np.arange(s, min(s + seg_len, win))
        groups.append(np.sort(_rng("cover_group", H, s).choice(seg, min(len(seg), nq_max), replace=False)))
    groups.append(np.arange(win, H))
    return [g for g in groups if len(g)]


@dataclass
class CoveragePlan:
    """Row plan of the kept groups (device int32 tables) for one (H, rs, re, rep, cfg, window_only)."""
    groups: List[np.ndarray]          # every group of coverage_groups (after window_only)
    kept: List[int]                   # indices into groups of those reaching [rs, re)
    positions: torch.Tensor           # (npos,) int64: sorted union of the kept groups' positions
    row_r: torch.Tensor               # (NR,) int64: query head of each row within its KV head
    row_p: torch.Tensor               # (NR,) int64: index into positions (0 for padding)
    NR: int
    n_rlist: int
    gtab: torch.Tensor
    rowpos: torch.Tensor
    rowgrp: torch.Tensor
    rlist: torch.Tensor
    items: torch.Tensor


_PLANS: Dict[Tuple, CoveragePlan] = {}


def coverage_plan(H: int, rs: int, re: int, rep: int, cfg=None, window_only: bool = False,
                  device: torch.device | str = "cuda") -> CoveragePlan:
    """The group table, row positions / groups, per-head row lists and 64-row work items of the groups
    of coverage_groups(H) that reach the coded range (the reference skips the others:
    STRATA_KV.py:1259-1261), cached per shape and device."""
    key = (H, rs, re, rep, window_only, str(device)) + tuple(_cfg(cfg, k) for k in sorted(_DEFAULTS))
    plan = _PLANS.get(key)
    if plan is not None:
        return plan
    groups = coverage_groups(H, cfg)
    if window_only:
        groups = groups[-1:]
    kept = [gi for gi, P in enumerate(groups) if min(re, int(P.max()) + 1) > rs]
    if not kept:
        raise ValueError("no coverage group reaches the coded range [rs, re)")
    positions = np.unique(np.concatenate([groups[gi] for gi in kept]))
    where = {int(p): i for i, p in enumerate(positions)}
    gtab, rowpos, rowgrp, row_r, row_p, items = [], [], [], [], [], []
    rlist = [[] for _ in range(rep)]
    row_base = 0
    local_far = _cfg(cfg, "STRATA_LOCAL")
    for gk, gi in enumerate(kept):
        P = groups[gi]
        nq = len(P)
        nq_pad = -(-nq // 16) * 16
        mmax = int(P.max()) + 1
        local = 1 if gi == len(groups) - 1 else local_far
        gtab.append([row_base, nq, nq_pad, mmax, min(re, mmax), local, 0, 0])
        for r in range(rep):
            for i in range(nq_pad):
                row = row_base + r * nq_pad + i
                real = i < nq
                rowpos.append(int(P[i]) if real else -1)
                rowgrp.append(gk)
                row_r.append(r)
                row_p.append(where[int(P[i])] if real else 0)
                rlist[r].append(row if real else -1)
        items.extend([gk, rb] for rb in range(-(-(rep * nq_pad) // 64)))
        row_base += rep * nq_pad
    dev = torch.device(device)
    i32 = lambda x: torch.tensor(np.asarray(x, dtype=np.int32), device=dev).contiguous()
    plan = CoveragePlan(groups=groups, kept=kept, positions=torch.as_tensor(positions, dtype=torch.long),
                        row_r=torch.tensor(row_r, dtype=torch.long, device=dev),
                        row_p=torch.tensor(row_p, dtype=torch.long, device=dev), NR=row_base,
                        n_rlist=row_base // rep, gtab=i32(gtab), rowpos=i32(rowpos), rowgrp=i32(rowgrp),
                        rlist=i32(rlist), items=i32(items))
    _PLANS[key] = plan
    return plan


def _rows_at(q, positions: torch.Tensor) -> torch.Tensor:
    """q_at (STRATA_KV.py:3173-3175): rows of q (B, Hq, T, d) or of a QRows-like object (``.at``)."""
    if hasattr(q, "at"):
        return q.at(positions)
    return q[:, :, positions.to(q.device)]


@torch.no_grad()
def coverage_stats(q, k: torch.Tensor, v: torch.Tensor, scaling: float, H: int, rs: int, re: int, M: torch.Tensor,
                   cfg=None, window_only: bool = False, workspace: torch.Tensor | None = None) -> Dict:
    """coverage_stats (STRATA_KV.py:1225-1298) on the device.  q (B, Hq, T, d) or QRows holding the
    groups' positions, k / v (B, Hkv, T, d) (batch element 0 is used, as in the reference), M (Hq, d, d)
    the per-query-head output metric.  Returns A, W, DD (Hkv, re - rs), S, Mbar (Hkv, d, d) float32 and
    the groups.  q, k, v share one dtype (fp32, fp16 or bf16); d = 128."""
    _lib.require_gpu(k, v, M)
    Hkv, T, d = k.shape[1], k.shape[2], k.shape[3]
    Hq = M.shape[0]
    if Hq % Hkv or tuple(M.shape) != (Hq, d, d):
        raise ValueError("M must be (Hq, d, d) with Hq a multiple of Hkv")
    rep = Hq // Hkv
    if v.shape[1:] != k.shape[1:] or v.dtype != k.dtype:
        raise ValueError("k and v must match in shape and dtype")
    if not 0 <= rs < re <= min(T, H):
        raise ValueError("need 0 <= rs < re <= min(H, T)")
    plan = coverage_plan(H, rs, re, rep, cfg, window_only, k.device)
    qg = _rows_at(q, plan.positions)[0]                                   # (Hq, npos, d)
    if qg.dtype != k.dtype or qg.shape[0] != Hq or qg.shape[-1] != d:
        raise ValueError("q must hold Hq query heads of k's dtype and head size")
    qg = qg.reshape(Hkv, rep, qg.shape[1], d)
    qr = qg[:, plan.row_r, plan.row_p].contiguous()                       # (Hkv, NR, d)
    k0, v0 = k[0], v[0]
    if k0.stride(-1) != 1:
        k0 = k0.contiguous()
    if v0.stride(-1) != 1:
        v0 = v0.contiguous()
    Mc = M.float().contiguous()
    dev = k.device
    n = re - rs
    A = torch.empty((Hkv, n), dtype=torch.float32, device=dev)
    W = torch.empty_like(A)
    DD = torch.empty_like(A)
    S = torch.empty((Hkv, d, d), dtype=torch.float32, device=dev)
    Mbar = torch.empty_like(S)
    G = len(plan.kept)
    need = _lib.load().kvq_coverage_stats_workspace(Hkv, rep, n, plan.NR, G)
    if need < 0:
        raise _lib.KVQError("kvq_coverage_stats_workspace rejected the shape")
    if workspace is None:
        workspace = torch.empty((need,), dtype=torch.float32, device=dev)
    elif (workspace.numel() < need or workspace.dtype != torch.float32 or not workspace.is_contiguous()
          or workspace.device != dev):
        # a caller who preallocated (e.g. for graph capture) gets an error, never a silent allocation
        raise ValueError(f"workspace must be a contiguous float32 tensor of >= {need} elements on {dev}")
    _lib.call("kvq_coverage_stats", qr.data_ptr(), _lib.DTYPE_CODE[k.dtype], plan.NR, plan.rowpos.data_ptr(),
              plan.rowgrp.data_ptr(), plan.rlist.data_ptr(), plan.n_rlist, plan.gtab.data_ptr(), G,
              plan.items.data_ptr(), plan.items.shape[0], k0.data_ptr(), k0.stride(0), k0.stride(1), v0.data_ptr(),
              v0.stride(0), v0.stride(1), T, Mc.data_ptr(), Hkv, rep, d, rs, re, float(scaling),
              float(_cfg(cfg, "STRATA_FLOOR")), A.data_ptr(), W.data_ptr(), DD.data_ptr(), S.data_ptr(),
              Mbar.data_ptr(), workspace.data_ptr(), workspace.numel(), _lib.stream_of(k))
    return {"A": A, "W": W, "DD": DD, "S": S, "Mbar": Mbar, "groups": plan.groups}
