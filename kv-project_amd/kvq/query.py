"""Query chunking for the decode entry points.

One decode launch holds at most ``MAX_ROWS`` query rows per KV head (rows = rep * Tq: the GQA
query heads of the KV head times the step's query tokens), the register tile of the split
kernels.  A step with more query tokens -- the reference feeds a whole question in one step
(``run_tokens``, STRATA_KV.py:3238-3248) and its ``chunked_attention`` takes any Tq in chunks of
``ATTN_CHUNK`` query tokens (STRATA_KV.py:641-675, 660) -- runs as consecutive launches over
query-token pieces of at most ``MAX_ROWS // rep`` tokens (and at most ``chunk`` when the caller
gives one).  Each piece is an ordinary decode of its own tokens at their own positions, so the
result is the same attention, token by token.
"""
from __future__ import annotations

from typing import Callable, List, Optional, Tuple

import torch

from ._lib import KVQError

MAX_ROWS = 8


def query_pieces(rep: int, Tq: int, chunk: Optional[int] = None) -> List[Tuple[int, int]]:
    """[start, end) ranges of query tokens, in order, each holding at most max(1, MAX_ROWS // rep)
    tokens and at most ``chunk`` tokens.  Raises KVQError when one token already exceeds the tile
    (rep > MAX_ROWS)."""
    if rep > MAX_ROWS:
        raise KVQError(f"the decode kernels hold at most {MAX_ROWS} query heads per KV head (got {rep})")
    if chunk is not None and int(chunk) < 1:
        raise ValueError("chunk must be a positive number of query tokens")
    per = MAX_ROWS // rep
    if chunk is not None:
        per = min(per, int(chunk))
    return [(s, min(Tq, s + per)) for s in range(0, Tq, per)]


def decode_in_pieces(fn: Callable[[torch.Tensor, Optional[torch.Tensor], Optional[torch.Tensor]], torch.Tensor],
                     q: torch.Tensor, q_pos: Optional[torch.Tensor], out: Optional[torch.Tensor],
                     pieces: List[Tuple[int, int]]) -> torch.Tensor:
    """Run ``fn(q_piece, q_pos_piece, out_piece) -> (B, t, Hq, d)`` over the pieces of q (B, Hq, Tq, d)
    into ``out`` (B, Tq, Hq, d), allocated when None.  With batch 1 a piece's rows of ``out`` are one
    dense block, so each piece is decoded straight into them and the step allocates nothing beyond
    what ``fn`` does; with a larger batch they are strided, so the pieces go through one staging
    tensor of the largest piece's shape (allocated once per call) and are copied over.  Launches
    stay on the current stream in piece order."""
    B, Hq, Tq, d = q.shape
    if out is None:
        out = torch.empty((B, Tq, Hq, d), dtype=q.dtype, device=q.device)
    elif tuple(out.shape) != (B, Tq, Hq, d) or not out.is_contiguous() or out.dtype != q.dtype:
        raise ValueError("out must be a contiguous (B, Tq, Hq, d) tensor of q's dtype")
    staging = None
    if B > 1:
        staging = torch.empty((B * max(e - s for s, e in pieces) * Hq * d,), dtype=q.dtype, device=q.device)
    for s, e in pieces:
        qp = None if q_pos is None else q_pos[s:e]
        if staging is None:
            fn(q[:, :, s:e], qp, out[:, s:e])
        else:
            part = staging[:B * (e - s) * Hq * d].view(B, e - s, Hq, d)
            out[:, s:e].copy_(fn(q[:, :, s:e], qp, part))
    return out
