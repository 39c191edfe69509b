"""kvq — MI355X-native (gfx950) packed-KV decode hot path of TahirSher/KV-Project.

Host-side mirror of the reference's Python entry points for this path, calling hand-written HIP
kernels in ``libkvq.so`` through the C ABI of ``include/kvq.h``.  No CPU fallback exists: every
op requires GPU tensors and raises ``KVQError`` when the library is missing.
"""
from ._lib import KVQError, load as load_library
from .kivi import (kivi_quant, kivi_quant_stored, pack_codes, pack_rows, unpack_codes, unpack_rows, v_tile,
                   v_untile, vmeta_tile)
from .decode import PackedKIVICache, exact_rows_cache, kivi_decode, score_workspace_floats, workspace_floats
from .state import DecodeCtl, KIVIState, PackedState, Router, payload_bytes, register, routed, router_attention
from .evict import (chunk_share, fake_quant_tokens, finalize_chunk, gather_dequant, gather_rows, retained_cache,
                    retained_decode, retained_workspace_floats, snapkv_scores, topk_retain, topk_workspace_words)
from .evict_state import EvictedState, MTLPState, mtlp_budget, mtlp_select, snapkv_keep, streaming_keep
from .strata import (StrataCache, StrataTier, pack_planar, rotation_signs, strata_center_rotate, strata_decode,
                     strata_quantize, strata_quantize_planar, strata_v_tile, strata_workspace_floats, uniform_step,
                     unpack_planar, unpack_planar_u8)
from .dct import DctCache, dct_decode, dct_encode, dct_table, dct_workspace_floats
from .mixed import MixedKIVICache, c3_widths, mixed_decode, mixed_workspace_floats, offset_table
from .strata_state import StrataState, strata_pack, strata_tier_kernel
from .quasar import QuasarState, quasar_scores, quasar_values, stage_codebooks
from .alloc import AllocWorkspace, allocate_layer, layer_costs, strata_allocate, strata_distortion
from .coverage import coverage_groups, coverage_plan, coverage_stats
from .strata_compress import StrataCompressor, rotation_matrix

__all__ = [
    "KVQError", "load_library", "kivi_quant", "kivi_quant_stored", "pack_codes", "unpack_codes", "pack_rows", "unpack_rows",
    "v_tile", "v_untile", "vmeta_tile", "PackedKIVICache", "kivi_decode", "workspace_floats", "score_workspace_floats",
    "DecodeCtl", "KIVIState", "Router", "register", "routed", "router_attention",
    "gather_dequant", "retained_cache", "snapkv_scores", "topk_retain", "topk_workspace_words", "pack_planar", "unpack_planar", "rotation_signs",
    "uniform_step", "strata_center_rotate", "strata_quantize", "strata_quantize_planar", "unpack_planar_u8",
    "strata_v_tile", "StrataCache", "StrataTier",
    "strata_decode", "strata_workspace_floats", "DctCache", "dct_decode", "dct_encode", "dct_table",
    "dct_workspace_floats", "MixedKIVICache", "c3_widths", "mixed_decode", "mixed_workspace_floats", "offset_table",
    "StrataState", "strata_pack", "strata_tier_kernel", "QuasarState", "stage_codebooks", "payload_bytes", "AllocWorkspace", "allocate_layer", "layer_costs",
    "strata_allocate", "strata_distortion", "coverage_groups", "coverage_plan", "coverage_stats",
    "StrataCompressor", "rotation_matrix", "chunk_share", "fake_quant_tokens", "finalize_chunk", "gather_rows",
    "EvictedState", "MTLPState", "mtlp_budget", "mtlp_select", "snapkv_keep", "streaming_keep", "PackedState",
    "exact_rows_cache", "quasar_scores", "quasar_values", "retained_decode",
    "retained_workspace_floats",
]
