"""Query chunking rule of the decode entry points (host logic, no GPU): pieces of at most
8 // rep query tokens, and at most ``chunk``; one query token may not exceed the 8-row tile."""
import pytest


def test_query_pieces_rule():
    from kvq.query import query_pieces
    from kvq import KVQError
    assert query_pieces(4, 5) == [(0, 2), (2, 4), (4, 5)]
    assert query_pieces(4, 40) == [(s, s + 2) for s in range(0, 40, 2)]
    assert query_pieces(1, 8) == [(0, 8)]
    assert query_pieces(1, 9) == [(0, 8), (8, 9)]
    assert query_pieces(3, 7, chunk=1) == [(i, i + 1) for i in range(7)]
    assert query_pieces(2, 7, chunk=256) == [(0, 4), (4, 7)]
    assert query_pieces(8, 2) == [(0, 1), (1, 2)]
    with pytest.raises(KVQError):
        query_pieces(16, 1)
    with pytest.raises(ValueError):
        query_pieces(4, 3, chunk=0)


@pytest.mark.parametrize("B", [1, 3])
def test_decode_in_pieces_writes_every_piece(B):
    """Every piece's rows land in out (batch 1: decoded straight into out's own rows, no copy)."""
    import torch
    from kvq.query import decode_in_pieces, query_pieces
    Hq, Tq, d = 8, 7, 4
    q = torch.randn(B, Hq, Tq, d)
    pieces = query_pieces(4, Tq)
    out = torch.full((B, Tq, Hq, d), float("nan"))
    seen = []

    def fn(qs, qp, o):
        assert o is not None and o.is_contiguous() and tuple(o.shape) == (B, qs.shape[2], Hq, d)
        seen.append(o.data_ptr())
        o.copy_(qs.transpose(1, 2) * 2.0 + qp[:, None, None].float())
        return o

    res = decode_in_pieces(fn, q, torch.arange(Tq) * 10, out, pieces)
    assert res is out
    want = q.transpose(1, 2) * 2.0 + (torch.arange(Tq) * 10).float()[None, :, None, None]
    assert torch.equal(out, want)
    if B == 1:                                            # each piece written in place
        assert seen == [out[:, s:e].data_ptr() for s, e in pieces]
    with pytest.raises(ValueError):
        decode_in_pieces(fn, q, None, torch.empty(B, Tq, Hq, d + 1), pieces)


def test_shape_checks_of_the_decode_boundary():
    """q must match the cache (batch, head_dim, heads a multiple of the KV heads) and a caller's
    out must be the dense block the kernels write; both are refused on the host."""
    import torch
    from kvq import _lib
    q = torch.empty(2, 8, 1, 128)
    _lib.check_q_cache(q, 2, 4, 128, "t")
    for B, Hkv, d in ((4096, 4, 128), (2, 3, 128), (2, 4, 64)):
        with pytest.raises(ValueError):
            _lib.check_q_cache(q, B, Hkv, d, "t")
    o = torch.empty(2, 1, 8, 128)
    assert _lib.out_or_new(o, (2, 1, 8, 128), torch.float32, o.device, "t") is o
    for bad in (torch.empty(2, 1, 8, 64), torch.empty(2, 1, 8, 128, dtype=torch.float16),
                torch.empty(2, 1, 8, 256)[..., :128]):
        with pytest.raises(ValueError):
            _lib.out_or_new(bad, (2, 1, 8, 128), torch.float32, o.device, "t")
