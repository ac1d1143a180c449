"""CPU checks of the launch orders (tca_plan_launch_orders).  Workgroup b of a
launch runs on XCD b % 8; the panel kernel's workgroups and the row kernel's
wavefront slots are ordered so that work on one XCD covers one column range.
Checked: every unit / task runs exactly once, idle entries pad only the ends
of the XCD queues, the wide rows' quarter groups keep their 4-aligned
workgroups, and the long rows' segments reach each XCD in column order."""
import numpy as np
import pytest

import spmm_amd as S

XCDS, SLOTS = 8, 4


def _zipf():
    return S.gen_zipf_rows(20000, 20000, 600000, seed=5, dtype=S.TCA_F16)[0]


def test_row_order_segments_by_column_per_xcd():
    a = _zipf()
    lo = S.plan_launch_orders(a, 64, S.TCA_PLAN_NO_PANELS)
    tasks, order = lo["tasks"], lo["row_order"]
    kind = tasks[:, 3] & 3
    nw, ns = int((kind == 3).sum()), int((kind == 2).sum())
    assert ns >= XCDS * SLOTS and len(order) % SLOTS == 0
    # every task once
    assert sorted(order[order >= 0].tolist()) == list(range(len(tasks)))
    # wide quarters in place (each group of 4 one workgroup), then segments, then the rest in task order
    assert np.array_equal(order[:nw], np.arange(nw))
    rest = order[order >= nw + ns]
    assert np.array_equal(rest, np.arange(nw + ns, len(tasks)))
    first_rest = int(np.nonzero(order >= nw + ns)[0][0]) if len(rest) else len(order)
    seg_slots = order[nw:first_rest]
    assert np.all((seg_slots == -1) | ((seg_slots >= nw) & (seg_slots < nw + ns)))
    # per XCD: the segments in ascending middle column, queues of equal count (+-1)
    mid = {t: a.colidx[tasks[t, 1] + (tasks[t, 2] - tasks[t, 1]) // 2] for t in range(nw, nw + ns)}
    counts = []
    for x in range(XCDS):
        q = [int(t) for b in range(nw // SLOTS, first_rest // SLOTS) if b % XCDS == x
             for t in order[SLOTS * b:SLOTS * (b + 1)] if t >= 0]
        cols = [mid[t] for t in q]
        assert cols == sorted(cols), x
        counts.append(len(q))
    assert max(counts) - min(counts) <= 1
    # and the queues cover increasing column ranges
    firsts = []
    for x in range(XCDS):
        q = [int(t) for b in range(nw // SLOTS, first_rest // SLOTS) if b % XCDS == x
             for t in order[SLOTS * b:SLOTS * (b + 1)] if t >= 0]
        firsts.append((mid[q[0]], mid[q[-1]]))
    assert all(firsts[x][1] <= firsts[x + 1][0] for x in range(XCDS - 1))


def test_row_order_off_without_enough_segments(monkeypatch):
    a, _ = S.gen_bernoulli(3000, 2000, 0.01, seed=1, dtype=S.TCA_F16)  # short rows only
    assert len(S.plan_launch_orders(a, 256, S.TCA_PLAN_NO_MFMA)["row_order"]) == 0
    monkeypatch.setenv("TCA_ROW_ORDER", "0")
    assert len(S.plan_launch_orders(_zipf(), 64, S.TCA_PLAN_NO_PANELS)["row_order"]) == 0


def test_panel_order_units_once_xcd_queues(monkeypatch):
    monkeypatch.setenv("TCA_PANEL_MIN_NNZ", "1000")
    monkeypatch.setenv("TCA_PANEL_UNIT", "3000")  # split panels: many local units
    a, _ = S.gen_rmat(13, 8000, 300000, seed=3, dtype=S.TCA_F32)
    pp = S.plan_panels(a, 128)
    lo = S.plan_launch_orders(a, 128)
    order = lo["panel_order"]
    n_units = len(pp["units"])
    assert n_units > XCDS and len(order) % XCDS == 0
    assert sorted(order[order >= 0].tolist()) == list(range(n_units))
    # idle workgroups only at the end of each XCD's queue
    for x in range(XCDS):
        q = order[x::XCDS]
        idle = np.nonzero(q < 0)[0]
        assert len(idle) == 0 or np.all(q[idle[0]:] < 0), x
    # local units (column span <= K / 4) reach each XCD in column order, queue x below queue x + 1
    P, K = pp["P"], a.ncol
    def span(u):
        t0, nt = pp["units"][u, 1], pp["units"][u, 2]
        return int(pp["cols"][t0 * P]), int(pp["cols"][(t0 + nt) * P - 1])
    mids = []
    for x in range(XCDS):
        loc = [span(u) for u in order[x::XCDS] if u >= 0 and (span(u)[1] - span(u)[0]) * (XCDS // 2) <= K]
        m = [lo_ + hi for lo_, hi in loc]
        assert m == sorted(m), x
        mids.append(m)
    assert sum(len(m) for m in mids) > 0
    for x in range(XCDS - 1):
        if mids[x] and mids[x + 1]:
            assert mids[x][-1] <= mids[x + 1][0]
    monkeypatch.setenv("TCA_PANEL_ORDER", "0")
    assert np.array_equal(S.plan_launch_orders(a, 128)["panel_order"], np.arange(n_units))
