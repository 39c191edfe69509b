"""The QUASAR split plan (kvq_quasar_plan, host code: runs without a GPU).

Chunk costs follow the plan's model (coefficients the 64-token chunk's tokens own over both sides,
plus a fixed part); a split's time is the makespan of its four wavefronts claiming its chunks in
order.  The plan must cover every chunk once, in order, within one resident round of workgroups,
and its longest split must be no longer than that of cutting the chunks into splits of equal cost.
"""
import ctypes as C

import numpy as np

N_C, HKV, MAX_SPLITS, FIXED = 45056, 8, 1024, 6144.0


def _tables(n_c):
    """Bands 16/16/32/64 over stages of 2/2/4 bits (12 steps a side, 128 code bytes per token),
    step l owning the first n_c * (1 - 0.9 l / 11) tokens, offsets as the flat buffer packs them."""
    rows, off = [], 0
    bands = [(0, 16), (16, 16), (32, 32), (64, 64)]
    l = 0
    for stage, bits in enumerate((2, 2, 4)):
        for a, w in bands:
            n_s = int(n_c * (1.0 - 0.9 * l / 11))
            nb = w * bits // 8
            rows.append([off, n_s, nb, a, w, bits, 16 * stage])
            off += HKV * n_s * nb
            l += 1
    return np.asarray(rows, dtype=np.int32)


def _costs(tab_k, tab_v, n_c):
    n_ch = (n_c + 63) // 64
    cost = np.full(n_ch, FIXED)
    for tab in (tab_k, tab_v):
        for n_s, w in zip(tab[:, 1], tab[:, 4]):
            for c in range(n_ch):
                if c * 64 >= n_s:
                    break
                cost[c] += min(64, n_s - c * 64) * w
    return cost


def _span(costs):
    fin = np.zeros(4)
    for x in costs:
        fin[np.argmin(fin)] += x
    return fin.max()


def _plan(tab_k, tab_v, n_c):
    from kvq import _lib
    lib = _lib.load()
    bounds = np.zeros(MAX_SPLITS + 1, dtype=np.int32)
    slots = np.zeros((2, 32, 8), dtype=np.int32)
    n_slots = np.zeros(2, dtype=np.int32)
    n_splits = C.c_int32(0)
    rc = lib.kvq_quasar_plan(tab_k.ctypes.data, tab_k.shape[0], tab_v.ctypes.data, tab_v.shape[0], n_c, HKV,
                             MAX_SPLITS, bounds.ctypes.data, C.addressof(n_splits), slots.ctypes.data,
                             n_slots.ctypes.data)
    assert rc == 0
    return bounds[:n_splits.value + 1].copy(), n_slots


def test_plan_covers_every_chunk_in_one_round_and_bounds_the_makespan():
    tab_k = _tables(N_C)
    tab_v = tab_k.copy()
    b, n_slots = _plan(tab_k, tab_v, N_C)
    n_ch = (N_C + 63) // 64
    S = len(b) - 1
    assert list(n_slots) == [32, 32]
    assert b[0] == 0 and b[-1] == n_ch and np.all(np.diff(b) >= 1)
    assert S <= 768 // HKV
    cost = _costs(tab_k, tab_v, N_C)
    span = max(_span(cost[b[i]:b[i + 1]]) for i in range(S))
    # splits of equal cost over the same split count
    cum = np.cumsum(cost)
    eq = [0] + [int(np.searchsorted(cum, cum[-1] * (i + 1) / S) + 1) for i in range(S - 1)] + [n_ch]
    eq_span = max(_span(cost[eq[i]:eq[i + 1]]) for i in range(S) if eq[i + 1] > eq[i])
    assert span <= eq_span
    # no split can be shorter than its heaviest chunk, nor the longest shorter than the average share
    assert span >= cost.max() and span >= cost.sum() / (4 * S)


def test_plan_small_context_and_empty():
    tab = _tables(300)
    b, _ = _plan(tab, tab.copy(), 300)
    assert b[0] == 0 and b[-1] == 5 and np.all(np.diff(b) >= 1) and len(b) - 1 <= 2   # at least 4 chunks a split on average
    b, _ = _plan(tab[:0], tab[:0], 0)
    assert list(b) == [0, 0]
