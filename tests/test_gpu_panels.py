"""GPU parity of the panel kernel (row panels with B rows staged in LDS):
bit-exact against the oracle on exact-arithmetic inputs for every lane
geometry (fp32 E = 8/4/2, fp16 and bf16 E = 8/4, several column chunks),
split panels (partial rows summed in a fixed order), panels beside MFMA windows
and the row kernel, determinism, and exactness of the masked steps with
non-finite B rows; each with the run data loaded where it lies and through
per-row windows."""
import numpy as np
import pytest

from conftest import exact_dense, exact_values
from oracle import oracle

import spmm_amd as S
from test_gpu_parity import _dev, assert_parity, make_csr, oracle_c, run_gpu

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True, params=["0", "1"], ids=["direct", "window"])
def window_mode(request, monkeypatch):
    """Every test with the run data loaded where it lies and through per-row windows."""
    monkeypatch.setenv("TCA_PANEL_WINDOW", request.param)
    return int(request.param)


def exact(a: S.CSR, dtype, seed=7):
    rng = np.random.default_rng(seed)
    v = exact_values(rng, a.nnz)
    v[v == 0] = 0.5
    return S.CSR(a.nrow, a.ncol, a.rowptr, a.colidx, S.to_storage(v, dtype), dtype)


@pytest.mark.parametrize("dtype,widths", [(S.TCA_F32, (32, 64, 128, 256)), (S.TCA_F16, (64, 128, 256)),
                                          (S.TCA_BF16, (64, 128))])
def test_panels_exact_all_geometries(torch_cuda, window_mode, dtype, widths):
    rng = np.random.default_rng(3 + dtype)
    base, _ = S.gen_rmat(12, 3000, 60000, seed=4)
    a = exact(base, dtype)
    for n in widths:
        b = S.to_storage(exact_dense(rng, (a.ncol, n)), dtype)
        with S.Plan(a, n, S.TCA_PLAN_NO_MFMA | S.TCA_PLAN_FORCE_PANELS) as pl:
            info = pl.info()
            got = run_gpu(torch_cuda, a, b, plan=pl)
        print(f"dtype {dtype} N={n}: {info['n_panels']} panels, {info['n_panel_units']} units, "
              f"{info['rows_panels']} rows", flush=True)
        assert info["n_panels"] > 0 and info["rows_panels"] == int((np.diff(a.rowptr) > 0).sum())
        assert info["panel_window"] == (info["n_panels"] if window_mode else 0)
        want = oracle_c(a, b)
        assert np.array_equal(got, want), (dtype, n, np.abs(got - want).max())


@pytest.mark.parametrize("unit", ["1500", "40000"])
@pytest.mark.parametrize("order", ["0", "1"])
def test_panels_split_into_units(torch_cuda, monkeypatch, unit, order):
    """Small units split panels by tiles; the partial rows are summed in a fixed order.  The
    launch order (natural, or XCD queues padded with idle workgroups) changes no result."""
    monkeypatch.setenv("TCA_PANEL_UNIT", unit)
    monkeypatch.setenv("TCA_PANEL_ORDER", order)
    rng = np.random.default_rng(17)
    base, _ = S.gen_zipf_rows(3000, 6000, 200000, s=1.5, cap=5000, seed=5)
    a = exact(base, S.TCA_F32)
    b = S.to_storage(exact_dense(rng, (a.ncol, 128)), S.TCA_F32)
    with S.Plan(a, 128, S.TCA_PLAN_FORCE_PANELS) as pl:
        info = pl.info()
        got = run_gpu(torch_cuda, a, b, plan=pl)
    assert info["n_panel_units"] > info["n_panels"] and info["n_long_rows"] > 0, info
    if order == "0":
        assert info["panel_blocks"] == info["n_panel_units"], info
    else:
        assert info["panel_blocks"] % 8 == 0 and info["panel_blocks"] >= info["n_panel_units"], info
    assert np.array_equal(got, oracle_c(a, b))


def test_panels_edge_rows(torch_cuda):
    """Empty rows (row kernel, zeros), one-element rows, full rows, a partial last panel."""
    rng = np.random.default_rng(19)
    k = 700
    lens = [0, 1, k, 3, 0, 350] + list(rng.integers(0, 60, 1200))
    a = make_csr(rng, lens, k, S.TCA_F32)
    for n in (64, 128):
        b = S.to_storage(exact_dense(rng, (k, n)), S.TCA_F32)
        with S.Plan(a, n, S.TCA_PLAN_FORCE_PANELS) as pl:
            assert pl.info()["n_panels"] > 0
            got = run_gpu(torch_cuda, a, b, plan=pl)
        assert np.array_equal(got, oracle_c(a, b)), n
        assert np.all(got[np.diff(a.rowptr) == 0] == 0.0)


def test_panels_beside_mfma_windows_and_rows(torch_cuda):
    """fp16: windows of the first 256 rows on the matrix cores, the other rows
    (which all hold columns 0..4, so their windows have steps with more
    nonzeros than the tile kernel takes) split between panels and, for the
    empty ones, the row kernel; all three kernels in one run."""
    rng = np.random.default_rng(23)
    k = 2048
    rows = [np.sort(rng.choice(k, size=int(l), replace=False)) for l in rng.binomial(k, 0.1, 256)]
    for i, l in enumerate(rng.integers(0, 150, 2000)):
        extra = rng.choice(np.arange(5, k), size=int(l), replace=False)
        rows.append(np.zeros(0, np.int64) if i % 20 == 7 else np.sort(np.concatenate([np.arange(5), extra])))
    lens = np.array([len(r) for r in rows])
    rowptr = np.zeros(len(rows) + 1, np.int32)
    np.cumsum(lens, out=rowptr[1:])
    v = exact_values(rng, int(rowptr[-1]))
    v[v == 0] = 0.5
    a = S.CSR(len(rows), k, rowptr, np.concatenate(rows).astype(np.int32), S.to_storage(v, S.TCA_F16), S.TCA_F16)
    b = S.to_storage(exact_dense(rng, (k, 128)), S.TCA_F16)
    with S.Plan(a, 128, S.TCA_PLAN_FORCE_MFMA | S.TCA_PLAN_FORCE_PANELS) as pl:
        info = pl.info()
        got = run_gpu(torch_cuda, a, b, plan=pl)
    assert info["n_windows_mfma"] > 0 and info["n_panels"] > 0 and info["n_row_tasks"] > 0, info
    assert np.array_equal(got, oracle_c(a, b))


def test_panels_deterministic_and_within_tolerance(torch_cuda, monkeypatch):
    """Ordinary values (fp32 rounding in the kernel's order): the reference
    verdict against the fp64 oracle, identical bits on repeated runs (default
    routing, its nonzero minimum lowered for this small graph)."""
    monkeypatch.setenv("TCA_PANEL_MIN_NNZ", "1000")
    rng = np.random.default_rng(29)
    a, _ = S.gen_rmat(13, 6000, 150000, norm=1, seed=6)
    b = S.gen_dense(a.ncol, 128, 1, seed=9, dtype=S.TCA_F32)
    with S.Plan(a, 128) as pl:
        info = pl.info()
        r1 = run_gpu(torch_cuda, a, b, plan=pl)
        r2 = run_gpu(torch_cuda, a, b, plan=pl)
    assert info["n_panels"] > 0, info
    assert np.array_equal(r1, r2)
    assert_parity(a, b, r1, "panels, R-MAT")


def test_panels_nonfinite_b_stays_in_its_rows(torch_cuda):
    """Steps past a run use the zero row, never another staged B row: an inf
    in one B row reaches exactly the C rows that reference its column."""
    rng = np.random.default_rng(31)
    base, _ = S.gen_rmat(11, 2000, 30000, seed=8)
    a = exact(base, S.TCA_F32)
    bf = exact_dense(rng, (a.ncol, 128))
    col = int(np.bincount(a.colidx, minlength=a.ncol).argmax())
    bf[col, 5] = np.inf
    b = S.to_storage(bf, S.TCA_F32)
    with S.Plan(a, 128, S.TCA_PLAN_FORCE_PANELS) as pl:
        got = run_gpu(torch_cuda, a, b, plan=pl)
    refs = np.zeros(a.nrow, bool)
    for r in range(a.nrow):
        refs[r] = col in set(a.colidx[a.rowptr[r]:a.rowptr[r + 1]].tolist())
    assert np.all(~np.isfinite(got[refs, 5])) and np.all(np.isfinite(got[~refs]))
    want = oracle_c(a, b)
    fin = np.isfinite(want)
    assert np.array_equal(got[fin], want[fin])


def test_rows_beside_panels_follow_the_run_stream(torch_cuda, monkeypatch):
    """A row phase that only clears empty rows (every row with nonzeros in panels)
    runs on the plan's second stream beside the panel kernel.  Its clears start
    after the work queued before the run on the run's stream (a NaN fill behind a
    sleep: clearing early would leave NaN rows), the segment sums and the work
    queued after the run wait for them, and the product equals the oracle and the
    one-stream run (TCA_ROWS_BESIDE=0) bit for bit."""
    torch = torch_cuda
    monkeypatch.setenv("TCA_PANEL_MIN_REUSE", "0")
    monkeypatch.setenv("TCA_PANEL_MIN_NNZ", "0")
    base, _ = S.gen_rmat(16, 65536, 100000, norm=1, seed=21)
    a = exact(base, S.TCA_F32, seed=22)
    n = 128
    nonempty = int((np.diff(a.rowptr) > 0).sum())
    b = S.to_storage(exact_dense(np.random.default_rng(23), (a.ncol, n)), S.TCA_F32)
    want = oracle_c(a, b)
    val, bd = _dev(torch, a.values), _dev(torch, b)
    outs = {}
    for beside in ("1", "0"):
        monkeypatch.setenv("TCA_ROWS_BESIDE", beside)
        with S.Plan(a, n) as pl:
            info = pl.info()
            print(f"rows beside panels={beside}: {info['rows_panels']} panel rows of {a.nrow}, "
                  f"{info['n_row_tasks']} row tasks, {info['n_long_rows']} long rows", flush=True)
            assert info["rows_panels"] == nonempty and info["n_row_tasks"] > 0 and info["n_long_rows"] > 0
            assert info["rows_beside_panels"] == int(beside)
            s = torch.cuda.Stream()
            c = torch.zeros((a.nrow, n), dtype=torch.float32, device="cuda:0")
            torch.cuda.synchronize()
            with torch.cuda.stream(s):
                torch.cuda._sleep(50_000_000)
                c.fill_(float("nan"))
                pl.run(val, bd, c, stream=s.cuda_stream)
                copy = c.clone()
            s.synchronize()
            outs[beside] = copy.cpu().numpy()
            # the timing entry points on the same plan: phase subsets with and
            # without the fork, the per-phase spans (one stream), whole runs
            for phases in (("rows",), ("panels", "rows", "segments"), pl.phases()):
                assert pl.time_subset(val, bd, c, phases, warmup=1, iters=2) > 0.0, phases
            pl.time_phases(val, bd, c, warmup=1, iters=2)
            assert pl.time(val, bd, c, warmup=1, iters=2) > 0.0
            torch.cuda.synchronize()
            assert np.array_equal(c.cpu().numpy(), want), beside
        assert np.array_equal(outs[beside], want), (beside, int(np.isnan(outs[beside]).any(axis=1).sum()))
    assert np.array_equal(outs["1"], outs["0"])


def test_rows_beside_panels_under_graph_capture(torch_cuda, monkeypatch):
    """The second stream's fork and join are captured into a HIP graph with the
    run (torch.cuda.graph on the plan's allocation-free run): every replay,
    with eager work and synchronisations between replays, gives the eager
    product bit for bit."""
    torch = torch_cuda
    monkeypatch.setenv("TCA_PANEL_MIN_REUSE", "0")
    monkeypatch.setenv("TCA_PANEL_MIN_NNZ", "0")
    base, _ = S.gen_rmat(15, 32768, 60000, norm=1, seed=31)
    a = exact(base, S.TCA_F32, seed=32)
    n = 64
    b = S.to_storage(exact_dense(np.random.default_rng(33), (a.ncol, n)), S.TCA_F32)
    want = oracle_c(a, b)
    val, bd = _dev(torch, a.values), _dev(torch, b)
    with S.Plan(a, n, S.TCA_PLAN_NO_SCRATCH) as pl:
        info = pl.info()
        print(f"graph capture: {info['rows_panels']} panel rows of {a.nrow}, {info['n_row_tasks']} row tasks, "
              f"rows beside panels {info['rows_beside_panels']}", flush=True)
        assert info["rows_beside_panels"] == 1
        c = torch.zeros((a.nrow, n), dtype=torch.float32, device="cuda:0")
        pl.run_static(val, bd, c)
        torch.cuda.synchronize()
        assert np.array_equal(c.cpu().numpy(), want)
        g = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            with torch.cuda.graph(g, stream=s):
                pl.run_static(val, bd, c, stream=s.cuda_stream)
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        for rep in range(3):
            c.fill_(float("nan"))
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            assert np.array_equal(c.cpu().numpy(), want), rep
        del g
