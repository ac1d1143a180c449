"""CPU checks of the panel plan (tca_plan_panels): an emulation of the panel
kernel's traversal over the plan arrays reproduces the oracle's SpMM bit for
bit on exact-arithmetic inputs, touches every nonzero of the panel rows
exactly once, and maps every staged position back to the nonzero's column."""
import numpy as np
import pytest

from conftest import exact_dense, exact_values
from oracle import oracle

import spmm_amd as S


def emulate(a: S.CSR, b: np.ndarray, pp: dict, n: int):
    """The panel kernel's traversal (units -> slots -> tiles -> CSR runs) in
    numpy; returns {row: C row} for the rows in panels and the visit mask."""
    R, P, rpg, stride = pp["R"], pp["P"], pp["rpg"], pp["cnt_stride"]
    crow, mxd = pp["cnt_rows"], pp["max_dword"]
    vals = a.values_f32()
    bf = S.from_storage(b, a.dtype).astype(np.float32)
    seen = np.zeros(a.nnz, np.int32)
    out = {}
    partials = np.zeros((max(pp["segments"], 1), n), np.float32)
    for u, (panel, t0, nt, segbase) in enumerate(pp["units"]):
        nu = pp["panel_units"][panel]
        for s in range(R):
            row = pp["rows"][panel * R + s]
            wave, i, g = s // (4 * rpg), (s // 4) % rpg, s % 4
            cur = pp["ustart"][u * R + s]
            acc = np.zeros(n, np.float32)
            for t in range(t0, t0 + nt):
                c = int(pp["cnt"][t * stride + (wave * crow + i) * 4 + g])
                if row < 0:
                    assert c == 0
                    continue
                # the longest run of the entry's four groups: the steps the wave takes
                c4 = pp["cnt"][t * stride + (wave * crow + i) * 4:][:4]
                assert int(pp["cnt"][t * stride + (wave * crow + mxd + i // 4) * 4 + i % 4]) == int(c4.max())
                for k in range(cur, cur + c):
                    # positions are 1-based (0 is the kernel's zero row)
                    assert 1 <= int(pp["pos"][k]) <= int(pp["width"][t]) <= P
                    col = pp["cols"][t * P + int(pp["pos"][k]) - 1]
                    assert col == a.colidx[k], (u, s, t, k)
                    seen[k] += 1
                    acc = acc + np.float32(vals[k]) * bf[col]
                cur += c
            if row < 0:
                continue
            if segbase < 0:
                out[row] = acc
            else:
                partials[segbase + s * nu] = acc
    for row, first, nseg, _ in pp["longrows"]:
        acc = np.zeros(n, np.float32)
        for k in range(nseg):
            acc = acc + partials[first + k]
        out[row] = acc
    return out, seen


def check_plan(a, n, flags=S.TCA_PLAN_FORCE_PANELS):
    rng = np.random.default_rng(a.nnz + n)
    b = S.to_storage(exact_dense(rng, (a.ncol, n)), a.dtype)
    pp = S.plan_panels(a, n, flags)
    assert pp["panels"] > 0, pp
    # a row holds at most 16 nonzeros of a tile (one 16-lane batch), a tile at most P columns
    assert int(pp["cnt"].max()) <= 16
    assert int(pp["pos"].max()) <= pp["P"]
    got, seen = emulate(a, b, pp, n)
    panel_rows = np.array(sorted(got), np.int64)
    # every nonzero of a panel row visited once, nothing else
    rl = np.diff(a.rowptr)
    want_seen = np.zeros(a.nnz, np.int32)
    for r in panel_rows:
        want_seen[a.rowptr[r]:a.rowptr[r + 1]] = 1
    assert np.array_equal(seen, want_seen)
    assert pp["n_rows"] == len(panel_rows) and pp["nnz"] == int(rl[panel_rows].sum())
    ref = oracle.csr_spmm(a.rowptr, a.colidx, a.values_f32(), S.from_storage(b, a.dtype))
    for r in panel_rows:
        assert np.array_equal(got[r], ref[r]), r
    return pp


def exact_csr(a: S.CSR, dtype):
    rng = np.random.default_rng(7)
    v = exact_values(rng, a.nnz)
    return S.CSR(a.nrow, a.ncol, a.rowptr, a.colidx, S.to_storage(v, dtype), dtype)


@pytest.mark.parametrize("dtype,n", [(S.TCA_F32, 128), (S.TCA_F32, 64), (S.TCA_F16, 64), (S.TCA_F32, 256),
                                     (S.TCA_BF16, 128)])
def test_panel_plan_rmat(dtype, n):
    a, _ = S.gen_rmat(12, 3000, 40000, seed=3)
    pp = check_plan(exact_csr(a, dtype), n)
    assert pp["elems"] * 16 * pp["chunks"] == n


def test_panel_plan_split_panels(monkeypatch):
    """Small units force panels into several units with partial rows."""
    monkeypatch.setenv("TCA_PANEL_UNIT", "2000")
    a, _ = S.gen_zipf_rows(3000, 5000, 150000, s=1.5, cap=4000, seed=5)
    pp = check_plan(exact_csr(a, S.TCA_F32), 128)
    assert pp["segments"] > 0 and len(pp["longrows"]) > 0
    assert (pp["panel_units"] > 1).any()


def test_panel_plan_routing_by_reuse(monkeypatch):
    """Default routing keeps a panel only when its nonzeros reuse its column
    union at least 1.02 times; uniform short rows over a wide K do not.  (The
    minimum of nonzeros in panels is lowered for these small matrices.)"""
    monkeypatch.setenv("TCA_PANEL_MIN_NNZ", "1000")
    rng = np.random.default_rng(11)
    a, _ = S.gen_bernoulli(2000, 200000, 0.00005, seed=2, dtype=S.TCA_F32)
    assert S.plan_panels(a, 128)["panels"] == 0
    dense_cols, _ = S.gen_bernoulli(800, 300, 0.3, seed=2, dtype=S.TCA_F32)
    pp = S.plan_panels(dense_cols, 128)
    assert pp["panels"] > 0
    assert S.plan_panels(dense_cols, 128, S.TCA_PLAN_NO_PANELS)["panels"] == 0
    # widths the lane geometry cannot cover
    assert S.plan_panels(dense_cols, 100)["panels"] == 0
    assert S.plan_panels(dense_cols, 24)["panels"] == 0


def test_panel_plan_edge_rows():
    """Empty rows, one-element rows, a full row, a partial last panel."""
    rng = np.random.default_rng(13)
    k = 700
    lens = [0, 1, k, 3, 0, 350] + list(rng.integers(0, 60, 1200))
    rowptr = np.zeros(len(lens) + 1, np.int32)
    np.cumsum(lens, out=rowptr[1:])
    colidx = np.concatenate([np.sort(rng.choice(k, size=int(l), replace=False)) for l in lens]).astype(np.int32)
    v = exact_values(rng, int(rowptr[-1]))
    a = S.CSR(len(lens), k, rowptr, colidx, S.to_storage(v, S.TCA_F32), S.TCA_F32)
    pp = check_plan(a, 128)
    assert (pp["rows"] == -1).any()  # the last panel is partial
    assert 0 not in set(np.flatnonzero(np.diff(rowptr) == 0)) & set(pp["rows"].tolist())


def test_panel_plan_small_matrices_stay_on_rows():
    """Below 2^21 nonzeros in panels the default plan keeps every row on the
    row kernel (too few workgroups to fill the GPU); forcing still plans them."""
    a, _ = S.gen_bernoulli(2048, 512, 0.1, seed=1, dtype=S.TCA_F32)
    assert S.plan_panels(a, 128)["panels"] == 0
    assert S.plan_panels(a, 128, S.TCA_PLAN_FORCE_PANELS)["panels"] > 0
