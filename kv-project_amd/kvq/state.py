"""Drop-in decode boundary: attention router, decode controller and the KIVI layer state.

Mirrors the reference's Python call shapes for the decode path so its call sites reach the HIP
kernels unchanged:

* ``router_attention(module, query, key, value, attention_mask, *args, **kwargs)`` and
  ``routed(controller)`` -- STRATA_KV.py:495-523.  With no active controller the call is plain
  SDPA (the registered "sdpa" attention); sliding-window and soft-capped attention are refused.
* ``DecodeCtl(states).begin(positions)`` / ``.attend(module, q, k, v, mask, kwargs)`` --
  STRATA_KV.py:2817-2834: append the step's keys/values to the layer's state, then attend.
* ``KIVIState`` -- the decode-state protocol of LayerState / StrataState
  (STRATA_KV.py:682-719, 1710-1818): ``append(k, v, pos)``, ``attend(q, scaling, qpos,
  chunk=None)``, fields ``n``, ``n0``, ``shared``, ``use_kernel``, ``context_bytes()``,
  ``check_kernel(tol)``; raises ``RuntimeError("decode buffer exhausted")`` when full.

KIVIState holds the cache KIVIMethod leaves after prefill (STRATA_KV.py:801-823, no sinks):
context tokens older than the window are read from their 4-bit codes, the last ``window``
context tokens and every appended token exactly.  Attention runs in libkvq's split-K kernel; there
is no second implementation to fall back to, so a failed ``check_kernel`` raises instead of
switching paths.
"""
from __future__ import annotations

from contextlib import contextmanager
from typing import Dict, Optional

import torch

from . import _lib
from .decode import PackedKIVICache, kivi_decode

ROUTER_ATTN = "kvq_router"


class Router:
    active = None


def _sdpa(module, query, key, value, attention_mask, *args, **kwargs):
    from transformers.integrations.sdpa_attention import sdpa_attention_forward
    return sdpa_attention_forward(module, query, key, value, attention_mask, *args, **kwargs)


def router_attention(module, query, key, value, attention_mask, *args, **kwargs):
    """Attention entry registered with transformers' AttentionInterface (STRATA_KV.py:499-510):
    plain SDPA without a controller, the controller's attend() with one."""
    ctl = Router.active
    if ctl is None:
        return _sdpa(module, query, key, value, attention_mask, *args, **kwargs)
    if kwargs.get("sliding_window") or getattr(module, "sliding_window", None) or kwargs.get("softcap"):
        raise RuntimeError(f"layer {getattr(module, 'layer_idx', '?')}: sliding-window / soft-capped "
                           "attention is not supported")
    return ctl.attend(module, query, key, value, attention_mask, kwargs)


def register(name: str = ROUTER_ATTN) -> str:
    """Register router_attention (and the SDPA mask) under ``name`` (STRATA_KV.py:513-514)."""
    from transformers import AttentionInterface
    from transformers.masking_utils import AttentionMaskInterface, sdpa_mask
    AttentionInterface.register(name, router_attention)
    AttentionMaskInterface.register(name, sdpa_mask)
    return name


@contextmanager
def routed(controller):
    """Make ``controller`` the active one for the duration (STRATA_KV.py:517-523)."""
    previous = Router.active
    Router.active = controller
    try:
        yield controller
    finally:
        Router.active = previous


def payload_bytes(states: Dict[int, "KIVIState"]) -> int:
    """MEASURED bytes of the compressed context over the layers (payload_bytes, STRATA_KV.py:
    2736-2769): the wire-format size of every state that owns its cache (shared ones excluded)."""
    return sum(st.payload_bytes() for st in states.values() if st.shared is None)


class DecodeCtl:
    """Single- or multi-token decode steps against per-layer states (STRATA_KV.py:2817-2834)."""

    def __init__(self, states: Dict[int, "KIVIState"], chunk: Optional[int] = None):
        self.states, self.chunk = states, chunk
        self.pos = None

    def begin(self, positions):
        self.pos = positions

    def attend(self, module, q, k, v, mask, kwargs):
        st = self.states[module.layer_idx]
        scaling = kwargs.get("scaling") or module.scaling
        if st.shared is None:
            st.append(k, v, self.pos)
            src = st
        else:
            src = self.states[st.shared]          # the source layer already appended this step
        return src.attend(q, scaling, self.pos, self.chunk), None


class PackedState:
    """The decode-state protocol (LayerState / StrataState, STRATA_KV.py:682-719, 1710-1818) over one
    ``PackedKIVICache`` ``self.cache`` whose exact rows carry positions (``cache.exact_pos``): append,
    attend, reference_attend and check_kernel.  Subclasses build the cache (KIVIState: KIVIMethod's
    cache; kvq.evict_state: the eviction families') and count their stored bytes."""

    cache: PackedKIVICache
    n: int
    n0: int
    shared: Optional[int] = None
    use_kernel: bool = True

    def append(self, k: torch.Tensor, v: torch.Tensor, pos) -> None:
        """Append t tokens (B, Hkv, t, d) at positions ``pos`` exactly (STRATA_KV.py:707-714)."""
        c = self.cache
        t = k.shape[2]
        if c.n_exact + t > c.cap_e:
            raise RuntimeError("decode buffer exhausted")
        c.k_exact[:, :, c.n_exact:c.n_exact + t] = k.to(c.k_exact.dtype)
        c.v_exact[:, :, c.n_exact:c.n_exact + t] = v.to(c.v_exact.dtype)
        p = torch.as_tensor(pos, dtype=torch.int64).reshape(-1).to(c.k_exact.device)
        c.exact_pos[c.n_exact:c.n_exact + t] = p
        c.n_exact += t
        self.n += t

    def attend(self, q: torch.Tensor, scaling: float, qpos, chunk=None) -> torch.Tensor:
        """q (B, Hq, Tq, d) at positions ``qpos`` (Tq,) -> (B, Tq, Hq, d) in q's dtype.  Query t
        reads every quantised row, the window rows and the appended rows at positions <= qpos[t]
        (chunked_attention's visibility, STRATA_KV.py:641-675).  Any Tq: the step runs in
        query-token pieces of at most 8 // rep tokens, and at most ``chunk`` when it is given
        (the reference's ATTN_CHUNK query chunks)."""
        if not self.use_kernel:
            raise RuntimeError(f"{type(self).__name__}: the HIP decode kernel is disabled (check_kernel failed)")
        c = self.cache
        qp = torch.as_tensor(qpos, dtype=torch.int64).reshape(-1).to(q.device)
        if qp.numel() != q.shape[2]:
            raise ValueError("qpos must hold one position per query token")
        return kivi_decode(q.to(c.k_exact.dtype), scaling, c, q_pos=qp, chunk=chunk).to(q.dtype)

    @torch.no_grad()
    def reference_attend(self, q: torch.Tensor, scaling: float, qpos) -> torch.Tensor:
        """The same attention in float32 torch ops from the dequantised cache (for check_kernel):
        one softmax over the dequantised rows and the visible exact rows."""
        c = self.cache
        B, Hkv, _, d = c.k_exact.shape
        from .decode import _dequant_keys, _dequant_values
        if c.n_q > 0:
            kh = _dequant_keys(c)                                 # (B, Hkv, n_q, d) fp32
            vh = _dequant_values(c)
        else:
            kh = vh = torch.zeros((B, Hkv, 0, d), device=c.k_exact.device)
        ke = c.k_exact[:, :, :c.n_exact].float()
        ve = c.v_exact[:, :, :c.n_exact].float()
        rep = q.shape[1] // Hkv
        K = torch.cat([kh, ke], 2).repeat_interleave(rep, 1)
        V = torch.cat([vh, ve], 2).repeat_interleave(rep, 1)
        qp = torch.as_tensor(qpos, dtype=torch.int64).reshape(-1).to(q.device)
        s = (q.float() * scaling) @ K.transpose(-1, -2)             # (B, Hq, Tq, n)
        vis_e = c.exact_pos[:c.n_exact][None, :] <= qp[:, None]     # (Tq, n_exact)
        mask = torch.cat([torch.ones((qp.numel(), c.n_q), dtype=torch.bool, device=q.device), vis_e], 1)
        s = s.masked_fill(~mask, float("-inf"))
        o = s.softmax(-1) @ V
        return o.transpose(1, 2).to(q.dtype).contiguous()

    @torch.no_grad()
    def check_kernel(self, tol: float = 2e-2) -> Dict:
        """Relative max error of the kernel against reference_attend on seeded random queries
        (STRATA_KV.py:1797-1817).  Raises when it exceeds ``tol``: there is no other path."""
        c = self.cache
        g = torch.Generator(device="cpu").manual_seed(42)
        Hkv, d = c.k_exact.shape[1], c.k_exact.shape[3]
        q = torch.randn(c.k_exact.shape[0], Hkv * 4, 2, d, generator=g).to(c.k_exact.device, c.k_exact.dtype)
        qpos = torch.tensor([self.n, self.n + 1])
        ref = self.reference_attend(q, d ** -0.5, qpos).float()
        out = self.attend(q, d ** -0.5, qpos).float()
        err = float((out - ref).abs().max() / ref.abs().max().clamp_min(1e-30))
        self.use_kernel = err <= tol
        if not self.use_kernel:
            raise RuntimeError(f"{type(self).__name__}.check_kernel: relative error {err:.3e} > {tol}")
        return {"kernel": True, "kernel_rel_err": err}


class KIVIState(PackedState):
    """One layer's KIVI cache as the decoder holds it (LayerState protocol).

    ``K, V`` (B, Hkv, H, d): the prefilled context (post-RoPE, model dtype, on the GPU).
    Context rows [0, H - window) are quantised (keys per channel over ``group_k`` tokens,
    values per token over ``group_v`` channels, ``bits`` = 4), rows [H - window, H) stay exact,
    and ``extra`` rows of room are kept for appended tokens (the question and the answer)."""

    def __init__(self, K: torch.Tensor, V: torch.Tensor, *, window: int, group_k: int, group_v: int,
                 extra: int, bits: int = 4, shared: Optional[int] = None):
        _lib.require_gpu(K, V)
        B, Hkv, H, d = K.shape
        self.H = H
        self.cache = PackedKIVICache.from_context(K, V, window=window, group_k=group_k, group_v=group_v,
                                                  bits=bits, extra_exact=extra)
        self.cache.exact_pos = torch.full((self.cache.cap_e,), 1 << 62, dtype=torch.int64, device=K.device)
        self.cache.exact_pos[:window] = torch.arange(H - window, H, device=K.device)
        self.n0 = self.n = H                      # tokens held (context + appended)
        self.shared = shared
        self.use_kernel = True

    def context_bytes(self) -> int:
        """Bytes of the stored context: packed codes and fp16 metadata of the quantised rows plus
        the exact window rows (STRATA_KV.py:1729-1735 counts a state the same way)."""
        c = self.cache
        B, Hkv = c.kc.shape[:2]
        d = c.kc.shape[3] * 2
        window = self.n0 - c.n_q
        return c.packed_bytes() + 2 * B * Hkv * window * d * c.k_exact.element_size()

    def payload(self) -> torch.Tensor:
        """The stored context in the reference's storage format (payload_bytes, STRATA_KV.py:
        2736-2769), written on the device: codes and fp16 metadata of the quantised rows, then the
        context's exact rows (the window; appended tokens are not context)."""
        c = self.cache
        return c.export(n_exact=self.n0 - c.n_q)

    def payload_bytes(self) -> int:
        """MEASURED bytes of the stored context: the length of ``payload()``."""
        c = self.cache
        return c.wire_bytes(n_exact=self.n0 - c.n_q)
