"""Offset table of the mixed-width cache (host logic, CPU)."""
import numpy as np
import torch

from kvq.mixed import UNIT, c3_widths, offset_table
from oracle.mixed import c3_widths as c3_widths_oracle


def test_offset_table_layout():
    g = torch.Generator().manual_seed(0)
    w = torch.tensor([2, 4, 8])[torch.randint(0, 3, (2, 3, 11), generator=g)]
    bits, off, base, seg, units = offset_table(w)
    wn = w.numpy()
    assert units == int((wn + 1).sum())
    start = 0
    for bh in range(6):
        b, h = divmod(bh, 3)
        assert int(base[bh]) == start
        ws = wn[b, h]
        assert seg[bh].tolist() == [start, (ws == 8).sum(), (ws == 4).sum(), (ws == 2).sum()]
        # storage order: width 8, 4, 2, token order within a width; contiguous, no overlap
        expect, u = {}, 0
        for width in (8, 4, 2):
            for i in np.nonzero(ws == width)[0]:
                expect[i] = u
                u += width + 1
        assert [int(off[b, h, i]) for i in range(11)] == [expect[i] for i in range(11)]
        assert bits[b, h].tolist() == ws.tolist()
        start += u
    assert UNIT == 2048


def test_c3_widths_matches_oracle_rule():
    imp = torch.distributions.LogNormal(0.0, 1.0).sample((2, 8, 256))
    got = c3_widths(imp).numpy()
    np.testing.assert_array_equal(got, c3_widths_oracle(imp.numpy().astype(np.float64)))
    assert ((got == 8).sum(-1) == 25).all() and ((got == 4).sum(-1) == 77).all()
