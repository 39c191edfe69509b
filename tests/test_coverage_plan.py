"""Host side of the device coverage statistics (kvq/coverage.py), no GPU needed.

* kvq.coverage.coverage_groups equals the reference's own draws (tests/golden/coverage_groups.npz,
  STRATA_KV.py:1206-1222) for the reference's default Config and its test Config.
* The row plan: every kept group reaches [rs, re) and every other does not (STRATA_KV.py:1259-1261),
  rows are laid out [group][query head][query padded to 16], each real row names its group's
  position and every 64-row block of every group is one work item.
"""
from pathlib import Path
from types import SimpleNamespace

import numpy as np

from kvq.coverage import coverage_groups, coverage_plan

GOLD = Path(__file__).resolve().parent / "golden" / "coverage_groups.npz"


def test_groups_match_reference_draws():
    z = np.load(GOLD)
    for name in ("default", "test"):
        N_SINK, LOCAL, W_OBS, SEG, QUER = (int(x) for x in z[f"{name}_params"])
        cfg = SimpleNamespace(N_SINK=N_SINK, STRATA_LOCAL=LOCAL, W_OBS=W_OBS, STRATA_SEGMENT=SEG,
                              STRATA_QUERIES=QUER, STRATA_FLOOR=1e-3)
        for H in (200, 700, 1500, 4100):
            gs = coverage_groups(H, cfg)
            np.testing.assert_array_equal([len(g) for g in gs], z[f"{name}_{H}_lengths"])
            np.testing.assert_array_equal(np.concatenate(gs), z[f"{name}_{H}_positions"])


def test_plan_layout():
    H, rs, re, rep = 1500, 600, 1400, 3
    plan = coverage_plan(H, rs, re, rep, device="cpu")
    groups = coverage_groups(H)
    assert [len(g) for g in plan.groups] == [len(g) for g in groups]
    reach = [gi for gi, P in enumerate(groups) if min(re, int(P.max()) + 1) > rs]
    assert plan.kept == reach and len(reach) < len(groups)            # the first segment is skipped
    gtab, rowpos, rowgrp = plan.gtab.numpy(), plan.rowpos.numpy(), plan.rowgrp.numpy()
    rlist, items = plan.rlist.numpy(), plan.items.numpy()
    assert plan.NR % 16 == 0 and plan.NR == len(rowpos) and rlist.shape == (rep, plan.NR // rep)
    n_items = 0
    for gk, gi in enumerate(plan.kept):
        P = groups[gi]
        base, nq, nq_pad, mmax, te, local = gtab[gk, :6]
        assert nq == len(P) and nq_pad % 16 == 0 and nq_pad - nq < 16
        assert mmax == P.max() + 1 and te == min(re, mmax)
        assert local == (1 if gi == len(groups) - 1 else 64)
        for r in range(rep):
            rows = base + r * nq_pad + np.arange(nq_pad)
            np.testing.assert_array_equal(rowpos[rows[:nq]], P)
            assert (rowpos[rows[nq:]] == -1).all() and (rowgrp[rows] == gk).all()
            assert set(rlist[r][rlist[r] >= 0]) >= set(rows[:nq])
        blocks = items[items[:, 0] == gk, 1]
        np.testing.assert_array_equal(blocks, np.arange(-(-(rep * nq_pad) // 64)))
        n_items += len(blocks)
    assert n_items == len(items)
    # the gathered rows: row_p indexes positions, so positions[row_p] == rowpos on real rows
    real = rowpos >= 0
    np.testing.assert_array_equal(plan.positions.numpy()[plan.row_p.numpy()[real]], rowpos[real])
    np.testing.assert_array_equal(plan.row_r.numpy(), (np.arange(plan.NR) - gtab[rowgrp, 0]) // gtab[rowgrp, 2])
