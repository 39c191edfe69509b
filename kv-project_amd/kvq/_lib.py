"""ctypes binding of libkvq.so (the C ABI declared in include/kvq.h).

The library is loaded lazily and only from this package directory.  There is no fallback:
every product entry point raises ``KVQError`` when the library is missing or a call fails, so a
silent CPU path can never stand in for the HIP kernels.
"""
from __future__ import annotations

import ctypes as C
import threading
from pathlib import Path

import torch

import os

# the in-tree build; KVQ_LIBRARY may name another build of the same sources (A/B comparisons)
LIB_PATH = Path(os.environ.get("KVQ_LIBRARY") or (Path(__file__).resolve().parent / "libkvq.so"))

KVQ_F32, KVQ_F16, KVQ_BF16 = 0, 1, 2
DTYPE_CODE = {torch.float32: KVQ_F32, torch.float16: KVQ_F16, torch.bfloat16: KVQ_BF16}

i64, i32, f32, vp = C.c_int64, C.c_int, C.c_float, C.c_void_p

# name -> (restype, argtypes); mirrors include/kvq.h
SIGNATURES = {
    "kvq_last_error": (C.c_char_p, []),
    "kvq_abi_version": (i32, []),
    "kvq_kivi_quant": (i32, [vp, i32, i64, i64, i64, i64, i64, i64, i64, i32, i32, i32, i32,
                             vp, i64, vp, i64, vp, vp, i64, vp, vp]),
    "kvq_pack_codes": (i32, [vp, i64, i32, vp, vp]),
    "kvq_unpack_codes": (i32, [vp, i64, i32, vp, vp]),
    "kvq_unpack_rows_lut": (i32, [vp, i64, i32, vp, vp, vp]),
    "kvq_v_tile": (i32, [vp, i64, i64, i64, i64, i64, vp, vp]),
    "kvq_v_untile": (i32, [vp, i64, i64, i64, i64, vp, i64, vp]),
    "kvq_vmeta_tile": (i32, [vp, vp, i64, i64, i64, i64, i64, vp, vp]),
    "kvq_kivi_decode_workspace": (i64, [i64, i64, i64, i64, i64, i64, i64, i32, i32, i64]),
    "kvq_kivi_score_workspace": (i64, [i64, i64, i64, i64, i64, i64, i64, i32, i32, i64]),
    "kvq_kivi_decode": (i32, [vp, i32, i64, i64, i64, i64, i64, i64, i64, i64, f32,
                              vp, vp, vp, vp, vp, i64, i64, i32, i32, vp, vp, i32, i64, i64,
                              vp, vp, vp, i32, vp, i64, vp, i64, f32, i64, i32, vp]),
    "kvq_kivi_decode_noalloc": (i32, [vp, i32, i64, i64, i64, i64, i64, i64, i64, i64, f32,
                                      vp, vp, vp, vp, vp, i64, i64, i32, i32, vp, vp, i32, i64, i64,
                                      vp, vp, vp, i32, vp, i64, f32, i64, i32, vp]),
    "kvq_snapkv_scores_workspace": (i64, [i64, i64, i64, i64, i64, i32]),
    "kvq_coverage_stats_workspace": (i64, [i64, i64, i64, i64, i64]),
    "kvq_coverage_stats": (i32, [vp, i32, i64, vp, vp, vp, i64, vp, i64, vp, i64, vp, i64, i64, vp, i64, i64, i64,
                                 vp, i64, i64, i64, i64, i64, f32, f32, vp, vp, vp, vp, vp, vp, i64, vp]),
    "kvq_snapkv_scores": (i32, [vp, i32, i64, i64, i64, vp, i64, i64, i64, i64, i64, i64, i64, i64, i64, f32, i32,
                                vp, vp, i64, vp]),
    "kvq_topk_retain": (i32, [vp, i64, i64, i64, i64, vp, i64, vp]),
    "kvq_topk_retain_workspace": (i64, [i64, i64]),
    "kvq_topk_retain_ws": (i32, [vp, i64, i64, i64, i64, vp, i64, vp, i64, vp]),
    "kvq_kivi_gather_dequant": (i32, [vp, vp, vp, vp, vp, i64, i64, i32, i32, i64, i64, vp, i64, i64, vp,
                                      vp, i32, i64, vp]),
    "kvq_pack_planar": (i32, [vp, i64, i64, i32, vp, vp]),
    "kvq_unpack_planar": (i32, [vp, i64, i64, i32, vp, vp]),
    "kvq_strata_center_rotate": (i32, [vp, i32, i64, i64, i64, i64, vp, vp, vp, vp]),
    "kvq_strata_quantize": (i32, [vp, i64, i64, i64, vp, i64, i32, f32, vp, vp, vp]),
    "kvq_strata_v_tile": (i32, [vp, i64, i64, i64, i32, i64, vp, vp, i64, vp, vp]),
    "kvq_strata_decode_workspace": (i64, [i64, i64, i64, i64, i64, i64, i32, vp, vp]),
    "kvq_strata_decode": (i32, [vp, i32, i64, i64, i64, i64, i64, i64, i64, i64, f32, vp, vp, vp, i32, vp, vp, vp,
                                vp, vp, vp, vp, vp, vp, i64, i64, vp, vp, vp, vp, i64, vp]),
    "kvq_strata_tier_partials": (i32, [vp, vp, i64, i64, i64, i32, i64, vp, vp, vp, vp, i64, i64, vp, vp, vp, vp, vp]),
    "kvq_dct_encode": (i32, [vp, i32, i64, i64, i64, i64, vp, i32, vp, vp, vp]),
    "kvq_dct_decode_workspace": (i64, [i64, i64, i64, i64, i64, i64, i64]),
    "kvq_dct_decode": (i32, [vp, i32, i64, i64, i64, i64, i64, i64, i64, i64, f32, vp, i64, vp, vp, vp, vp,
                             vp, vp, i64, i64, vp, vp, vp, vp, i64, i32, vp]),
    "kvq_mixed_encode": (i32, [vp, vp, i32, i64, i64, i64, i64, vp, vp, vp, vp, vp]),
    "kvq_mixed_decode_workspace": (i64, [i64, i64, i64, i64, i64, i64, i64]),
    "kvq_mixed_decode": (i32, [vp, i32, i64, i64, i64, i64, i64, i64, i64, i64, f32, vp, vp, i64, vp, vp, i64, i64,
                               vp, vp, vp, vp, i64, i32, vp]),
    "kvq_kivi_append": (i32, [vp, vp, i32, i64, i64, i64, i64, i64, i64, i64, i64, vp, vp, i64,
                              vp, vp, vp, vp, vp, i64, i32, i32, vp]),
    "kvq_selftest_mfma_layout": (i32, [vp, vp, vp, vp]),
    "kvq_kivi_retained_workspace": (i64, [i64, i64, i64, i64, i64, i64, i64]),
    "kvq_kivi_decode_retained": (i32, [vp, i32, i64, i64, i64, i64, i64, i64, i64, i64, f32, vp, vp, vp, vp, vp,
                                       i64, i64, i32, i32, vp, i64, i64, vp, vp, i32, i64, i64, vp, vp, vp, i32,
                                       vp, i64, vp]),
    "kvq_gather_rows": (i32, [vp, vp, i64, i64, i64, i64, vp, i64, i64, vp, vp, i64, vp]),
    "kvq_chunk_share_workspace": (i64, [i64, i64, i64]),
    "kvq_chunk_share": (i32, [vp, vp, i64, i64, i64, i64, vp, vp, i64, vp]),
    "kvq_absmax_fake_quant": (i32, [vp, i64, i64, i32, vp, vp]),
    "kvq_quasar_scores": (i32, [vp, i64, i64, i64, vp, i64, vp, i32, vp, i64, i64, vp, vp]),
    "kvq_quasar_values_workspace": (i64, [i64, i64, i64, i64]),
    "kvq_quasar_values": (i32, [vp, i64, i64, i64, vp, i64, vp, i32, vp, i64, i64, vp, vp, i64, vp]),
    "kvq_kivi_payload_bytes": (i64, [i64, i64, i64, i32, i32, i64, i32]),
    "kvq_kivi_export": (i32, [vp, vp, vp, vp, vp, i64, i64, i64, i64, i32, i32, vp, vp, i32, i64, i64, i64, vp, i64, vp]),
    "kvq_quasar_plan": (i32, [vp, i32, vp, i32, i64, i64, i32, vp, vp, vp, vp]),
    "kvq_strata_distortion_workspace": (i64, [i64, i64, i32]),
    "kvq_strata_distortion": (i32, [vp, vp, i64, i64, i64, vp, vp, vp, vp, vp, vp, i32, vp, vp, vp, vp, i64, vp]),
    "kvq_strata_allocate_workspace": (i64, [i64, i64, i32]),
    "kvq_strata_allocate": (i32, [vp, i64, i64, i32, vp, vp, C.c_double, i32, vp, vp, vp, vp, vp, vp, vp, i64, vp]),
    "kvq_quasar_decode_workspace": (i64, [i64, i64, i64, i64, i64, i64, i32]),
    "kvq_quasar_decode": (i32, [vp, i32, i64, i64, i64, i64, i64, i64, f32, vp, vp, i64, i64, vp, vp,
                                vp, i64, vp, i64, vp, i32, i32, vp, i32, vp, vp, i64, vp, vp, i64, i64, vp, vp,
                                vp, i32, vp, vp, i64, i32, vp]),
}


class KVQError(RuntimeError):
    """A libkvq call was rejected or failed, or the library is not available."""


_lock = threading.Lock()
_lib = None


def load() -> C.CDLL:
    """Load libkvq.so (once) and attach the ctypes signatures."""
    global _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise KVQError(f"{LIB_PATH} is not built: run `python kv-project_amd/kvq/build.py` "
                               "(or __graft_entry__.build()) first")
            lib = C.CDLL(str(LIB_PATH))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype, fn.argtypes = res, args
            _lib = lib
    return _lib


_fns: dict = {}


def call(name: str, *args) -> int:
    """Call an int-status entry point; raise KVQError with the library's message on failure.
    (The bound entry points are looked up once: a decode step pays no lock or attribute lookup.)"""
    fn = _fns.get(name)
    if fn is None:
        fn = _fns[name] = getattr(load(), name)
    rc = fn(*args)
    if rc != 0:
        msg = load().kvq_last_error().decode(errors="replace")
        raise KVQError(f"{name} failed ({rc}): {msg}")
    return rc


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of(t: torch.Tensor) -> int:
    """The current stream of t's device as a raw hipStream_t (one call, no Stream object)."""
    if _raw_stream is not None:
        return _raw_stream(t.device.index)
    return torch.cuda.current_stream(t.device).cuda_stream


def require_gpu(*tensors: torch.Tensor) -> None:
    """The product path runs only on the GPU: CPU tensors are rejected, never computed on."""
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise KVQError("kvq kernels take GPU tensors only (got a CPU tensor); there is no CPU path")


def check_q_cache(q: torch.Tensor, B: int, Hkv: int, d: int, what: str) -> None:
    """q (B, Hq, Tq, d) must match the cache it attends over: the same batch and head_dim, and a
    query head count that is a multiple of the cache's KV heads.  The kernels index the cache by
    q's batch and heads, so a mismatch is refused here rather than read past the cache."""
    if q.dim() != 4:
        raise ValueError(f"{what}: q must be (B, Hq, Tq, d), got {tuple(q.shape)}")
    qb, hq, _, qd = q.shape
    if qb != B or qd != d or Hkv <= 0 or hq % Hkv != 0:
        raise ValueError(f"{what}: q {tuple(q.shape)} does not match the cache (batch {B}, {Hkv} KV heads, "
                         f"head_dim {d})")


def out_or_new(out, shape, dtype, device, what: str) -> torch.Tensor:
    """The caller's output tensor after checking that the kernels can write ``shape`` into it
    (contiguous, that dtype, that device), or a new one.  The kernels write a dense (B, Tq, Hq, d)
    block at out's address, so any other tensor is refused."""
    if out is None:
        return torch.empty(shape, dtype=dtype, device=device)
    if tuple(out.shape) != tuple(shape) or out.dtype != dtype or not out.is_contiguous() or out.device != device:
        raise ValueError(f"{what}: out must be a contiguous {tuple(shape)} tensor of {dtype} on {device}")
    return out
