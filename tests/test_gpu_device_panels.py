"""Row panels planned on the GPU (tca_spmm_plan_create_device,
device_panel_planner.hpp): every array the panel kernel reads -- panel rows,
staged B rows, counts, positions, units, their cursors, launch order and the
split panels' long rows -- equals the host planner's (plan_panels) entry for
entry, the row kernel's plan of the other rows too, and both plans give
bit-identical products equal to the oracle on exact inputs.  Cases: default
routing on an R-MAT graph large enough for panels, forced panels on lognormal
rows (fp32 and fp16, one and two column chunks, 152- and 255-column tiles),
units forced small (split panels, partial rows), a column range past 2^19
(several bitmap chunks per panel), panels beside MFMA windows, and a matrix
with no panel rows."""
import os

import numpy as np
import pytest

from conftest import exact_dense, exact_values
from oracle import oracle
from test_gpu_parity import _dev

import spmm_amd as S

pytestmark = pytest.mark.gpu

PANEL_KEYS = ("rows", "boff", "cnt", "pos", "units", "order", "panel_units", "ustart", "longrows", "window")


def _exact(a, seed):
    rng = np.random.default_rng(seed)
    return S.CSR(a.nrow, a.ncol, a.rowptr, a.colidx, S.to_storage(exact_values(rng, a.nnz), a.dtype), a.dtype)


def _mixed_f16(seed):
    """Dense 128-row windows (rows 0..383) routed to the matrix cores, the
    other rows long enough for forced panels."""
    rng = np.random.default_rng(seed)
    m, k = 1500, 3000
    lens = np.where(np.arange(m) < 384, rng.integers(80, 140, m), rng.integers(0, 60, m))
    rowptr = np.zeros(m + 1, np.int32)
    np.cumsum(lens, out=rowptr[1:])
    cols = [np.sort(rng.choice(900 if r < 384 else k, lens[r], replace=False)).astype(np.int32) for r in range(m)]
    colidx = np.concatenate(cols).astype(np.int32)
    return S.CSR(m, k, rowptr, colidx, S.to_storage(np.ones(len(colidx), np.float32), S.TCA_F16), S.TCA_F16)


def _cases():
    # name, matrix, N, flags, environment
    yield "rmat-default", S.gen_rmat(16, 65536, 1500000, seed=3, dtype=S.TCA_F32)[0], 128, S.TCA_PLAN_DEFAULT, {}
    yield "lognormal-f32", S.gen_lognormal_rows(2000, 3000, 60, seed=2, dtype=S.TCA_F32)[0], 128, \
        S.TCA_PLAN_FORCE_PANELS, {}
    yield "lognormal-f32-n64", S.gen_lognormal_rows(1500, 2500, 40, seed=5, dtype=S.TCA_F32)[0], 64, \
        S.TCA_PLAN_FORCE_PANELS, {}
    yield "lognormal-f16-2chunks", S.gen_lognormal_rows(1800, 2200, 50, seed=6, dtype=S.TCA_F16)[0], 256, \
        S.TCA_PLAN_NO_MFMA | S.TCA_PLAN_FORCE_PANELS, {}
    yield "split-units", S.gen_rmat(13, 8192, 200000, seed=7, dtype=S.TCA_F32)[0], 128, \
        S.TCA_PLAN_FORCE_PANELS, {"TCA_PANEL_UNIT": "3000"}
    yield "wide-k", S.gen_lognormal_rows(1200, 1500000, 80, seed=8, dtype=S.TCA_F32)[0], 128, \
        S.TCA_PLAN_FORCE_PANELS, {}
    yield "beside-mfma", _mixed_f16(9), 128, S.TCA_PLAN_FORCE_PANELS | S.TCA_PLAN_MFMA_DENSE, {}
    yield "no-panel-rows", S.gen_bernoulli(700, 900, 0.002, seed=10, dtype=S.TCA_F32)[0], 128, \
        S.TCA_PLAN_DEFAULT, {}
    # B of 512 MB, past the MALL: by default every row with nonzeros in panels
    yield "past-mall", S.gen_rmat(20, 1 << 20, 1500000, seed=11, dtype=S.TCA_F32)[0], 128, S.TCA_PLAN_DEFAULT, {}


CASES = list(_cases())


@pytest.mark.parametrize("name,a,n,flags,env", CASES, ids=[c[0] for c in CASES])
def test_device_panels_equal_host_panels(torch_cuda, name, a, n, flags, env):
    torch = torch_cuda
    print(f"device panels {name}: M={a.nrow} K={a.ncol} nnz={a.nnz} N={n} flags={flags} env={env}", flush=True)
    a = _exact(a, 11)
    old = {k: os.environ.get(k) for k in env}
    os.environ.update(env)
    try:
        hp = S.Plan(a, n, flags)
        drp, dci = _dev(torch, a.rowptr), _dev(torch, a.colidx)
        dp = S.Plan.from_device(drp, dci, a.nrow, a.ncol, a.nnz, n, a.dtype, flags)
    finally:
        for k, v in old.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v
    try:
        hx, dx = hp.export_panels(), dp.export_panels()
        for k in ("panels", "tiles", "n_units", "R", "P"):
            assert hx[k] == dx[k], (name, k, hx[k], dx[k])
        for k in PANEL_KEYS:
            assert np.array_equal(hx[k], dx[k]), (name, k)
        hi, di = hp.info(), dp.info()
        for key in ("n_panels", "n_panel_units", "rows_panels", "nnz_panels", "staged_panels", "panel_blocks",
                    "panel_window", "rows_beside_panels", "n_row_tasks", "n_multi_tasks", "n_seg_tasks", "n_long_rows", "scratch_bytes", "row_blocks"):
            assert hi[key] == di[key], (name, key, hi[key], di[key])
        if name == "no-panel-rows":
            assert hx["panels"] == 0
        else:
            assert hx["panels"] > 0, name
        if name == "split-units":
            assert len(hx["longrows"]) > 0 and hx["n_units"] > hx["panels"], name
        if name == "wide-k":
            assert a.ncol > 2 * (1 << 19)
        if name == "past-mall":
            assert hi["rows_panels"] == int((np.diff(a.rowptr) > 0).sum()), hi
            assert hi["rows_beside_panels"] == int(hi["n_row_tasks"] > 0), hi
        # the other rows: the same row-kernel plan
        ht, hperm, hl = hp.export_rows()
        dt, dperm, dl = dp.export_rows()
        assert np.array_equal(ht, dt) and np.array_equal(hperm, dperm) and np.array_equal(hl, dl), name
        assert np.array_equal(hp.export_order(), dp.export_order()), name
        rng = np.random.default_rng(12)
        b = S.to_storage(exact_dense(rng, (a.ncol, n)), a.dtype)
        val, bd = _dev(torch, a.values), _dev(torch, b)
        outs = []
        for pl in (hp, dp):
            c = torch.full((a.nrow, n), float("nan"), dtype=torch.float32, device="cuda:0")
            pl.run(val, bd, c)
            torch.cuda.synchronize()
            outs.append(c.cpu().numpy())
        assert np.array_equal(outs[0], outs[1]), name
        gold = oracle.csr_spmm(a.rowptr, a.colidx, a.values_f32(), S.from_storage(b, a.dtype), 0)
        assert np.array_equal(outs[1], gold), name
    finally:
        hp.close()
        dp.close()
