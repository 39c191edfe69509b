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
