"""GPU parity: the gfx950 kernels (through the C ABI) against the CPU oracle
and the committed golden fixtures.

Bars:
* bit-exact where the arithmetic is exact (values in {+-1,+-1/2,+-2}, B in
  {k/256}, rows short enough that every partial sum is exact in fp32 in any
  order): GPU == fp32 oracle bit for bit;
* elsewhere (fp32 accumulation in another order than the oracle's), against
  the fp64-accumulated oracle G: the reference verdict compare_mat(G, C,
  1e-3) must pass, and the relative error |C - G| / max(|G|, 1e-3 * S) must
  be <= 1e-3 for every element, where S = sum_j |a_j * b_j| of that element
  (the floor makes outputs that cancel to ~0 compare on the scale of their
  terms; any wrong or missing term of ordinary size still fails it)."""
import ctypes
import os

import numpy as np
import pytest

from conftest import GOLDEN, exact_dense, exact_values
from oracle import oracle

import spmm_amd as S

pytestmark = pytest.mark.gpu

TOL = 1e-3       # target: max relative error <= 1e-3 (the reference verdict tolerance)
FLOOR = 1e-2     # |gold| floor of the relative-error report (outputs are O(0.1..10))


def _dev(torch, arr):
    a = np.ascontiguousarray(arr)
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    return torch.from_numpy(a).to("cuda:0")


def run_gpu(torch, a: S.CSR, b: np.ndarray, flags=S.TCA_PLAN_DEFAULT, plan=None, out=None):
    n = b.shape[1]
    own = plan is None
    if own:
        plan = S.Plan(a, n, flags)
    val = _dev(torch, a.values) if a.nnz else torch.zeros(1, device="cuda:0")
    bd = _dev(torch, b)
    c = out if out is not None else torch.full((a.nrow, n), float("nan"), dtype=torch.float32, device="cuda:0")
    plan.run(val, bd, c)
    torch.cuda.synchronize()
    res = c.cpu().numpy()
    if own:
        plan.close()
    return res


def oracle_c(a: S.CSR, b: np.ndarray):
    return oracle.csr_spmm(a.rowptr, a.colidx, a.values_f32(), S.from_storage(b, a.dtype))


def assert_close(gold, got, what=""):
    """Small-row cases: reference verdict and relative error with an absolute floor."""
    v = S.compare_mat(gold, got, TOL, FLOOR)
    assert v["success"], (what, v)
    assert v["max_rel_floor"] <= TOL, (what, v)
    assert np.all(np.isfinite(got)), what


def assert_parity(a: S.CSR, b: np.ndarray, got: np.ndarray, what=""):
    """GPU result against the fp64-accumulated oracle (see module docstring)."""
    vals = a.values_f32().astype(np.float64)
    bf = S.from_storage(b, a.dtype).astype(np.float64)
    g64 = oracle.csr_spmm_f64(a.rowptr, a.colidx, vals, bf)
    s64 = oracle.csr_spmm_f64(a.rowptr, a.colidx, np.abs(vals), np.abs(bf))
    assert np.all(np.isfinite(got)), what
    v = S.compare_mat(g64.astype(np.float32), got, TOL)
    assert v["success"], (what, v)
    zero = s64 == 0
    assert np.all(got[zero] == 0.0), what
    rel = np.abs(got.astype(np.float64) - g64)[~zero] / np.maximum(np.abs(g64), 1e-3 * s64)[~zero]
    worst = float(rel.max()) if rel.size else 0.0
    print(f"{what}: max rel err {worst:.3e} (bar {TOL})", flush=True)
    assert worst <= TOL, (what, worst)
    return worst


def make_csr(rng, lens, k, dtype, values="exact"):
    lens = np.asarray(lens, np.int64)
    rowptr = np.zeros(len(lens) + 1, np.int32)
    np.cumsum(lens, out=rowptr[1:])
    colidx = np.concatenate([np.sort(rng.choice(k, size=int(l), replace=False)) for l in lens]
                            + [np.zeros(0, np.int64)]).astype(np.int32)
    nnz = int(rowptr[-1])
    v = exact_values(rng, nnz) if values == "exact" else (rng.standard_normal(nnz) * 0.02).astype(np.float32)
    v[v == 0] = 0.5
    return S.CSR(len(lens), k, rowptr, colidx, S.to_storage(v, dtype), dtype)


# ------------------------------------------------------------ golden
def test_golden_scipy_fixtures(torch_cuda):
    data = np.load(os.path.join(GOLDEN, "scipy_spmm.npz"))
    names = sorted({k.split("__")[0] for k in data.files})
    for nm in names:
        rp, ci, v, b, c = (data[f"{nm}__{x}"] for x in ("rowptr", "colidx", "values", "b", "c"))
        dtype = S.TCA_F32 if v.dtype == np.float32 else S.TCA_F16
        a = S.CSR(len(rp) - 1, b.shape[0], rp, ci, v, dtype)
        got = run_gpu(torch_cuda, a, b)
        print(nm, a.nrow, b.shape, flush=True)
        assert_close(c.astype(np.float32), got, nm)
        assert_parity(a, b, got, nm)


def test_fixture_smtx_reference_flow(torch_cuda):
    """The reference harness flow: .smtx -> CSR (1.0 values), N = 256, seeded B."""
    a = S.read_smtx(os.path.join(GOLDEN, "body_decoder_layer_2_ffn_conv1.smtx"))
    for n in (64, 128, 256, 512):
        b = S.gen_dense(a.ncol, n, 3, seed=n, dtype=S.TCA_F16, sparsity=0.1)
        got = run_gpu(torch_cuda, a, b)
        assert_parity(a, b, got, f"fixture N={n}")
        empty = np.diff(a.rowptr) == 0
        assert np.all(got[empty] == 0.0)


# ------------------------------------------------------- exact vectors
SHAPES_N = [1, 2, 3, 8, 12, 16, 24, 64, 96, 100, 128, 200, 256, 512, 520, 1000, 1024]


@pytest.mark.parametrize("dtype", [S.TCA_F16, S.TCA_BF16, S.TCA_F32])
def test_exact_bit_equal_all_widths(torch_cuda, dtype):
    rng = np.random.default_rng(11 + dtype)
    k = 3000
    # empty rows, 1..8 (multi), medium, and long rows (split into segments)
    lens = np.concatenate([np.zeros(9, np.int64), rng.integers(1, 9, 60), rng.integers(9, 300, 40),
                           [600, 1500, 2999, 2500]])
    rng.shuffle(lens)
    a = make_csr(rng, lens, k, dtype)
    for n in SHAPES_N:
        b = S.to_storage(exact_dense(rng, (k, n)), dtype)
        got = run_gpu(torch_cuda, a, b)
        want = oracle_c(a, b)
        assert np.array_equal(got, want), (dtype, n, np.abs(got - want).max())


@pytest.mark.parametrize("variant", [S.TCA_PLAN_MFMA_PAIR, 0, S.TCA_PLAN_MFMA_DENSE, S.TCA_PLAN_MFMA_COMPACT],
                         ids=["pair", "default", "dense", "compact"])
@pytest.mark.parametrize("dtype", [S.TCA_F16, S.TCA_BF16])
def test_mfma_exact_bit_equal(torch_cuda, dtype, variant):
    """Condensed-tile MFMA path (forced on every eligible window) is bit-equal
    to the oracle on exact-arithmetic inputs, for partial windows, partial
    column blocks and empty rows.  The cases cover steps of up to 256, 512
    and more than 512 nonzeros and windows whose steps span several pipeline
    blocks, for the paired kernel (MFMA and staging wavefronts) and the dense
    tiles (plain, natural column order, compacted).  The paired kernel takes
    at most 512 nonzeros per step: the cases marked dense stay on the row
    kernel under it (still checked against the oracle)."""
    rng = np.random.default_rng(71 + dtype)
    dense = {(200, 64, 0.45), (128, 2048, 0.2), (64, 1500, 0.4)}
    for m, k, p in [(64, 256, 0.1), (130, 700, 0.05), (200, 64, 0.45), (17, 40, 0.3), (96, 5000, 0.004),
                    (128, 2048, 0.2), (64, 1500, 0.4), (128, 2048, 0.1), (100, 1000, 0.12), (150, 30, 0.1)]:
        lens = rng.binomial(k, p, m)
        lens[rng.random(m) < 0.1] = 0
        a = make_csr(rng, lens, k, dtype)
        for n in (8, 16, 64, 128, 136, 256, 512):
            b = S.to_storage(exact_dense(rng, (k, n)), dtype)
            with S.Plan(a, n, S.TCA_PLAN_FORCE_MFMA | variant) as pl:
                info = pl.info()
                got = run_gpu(torch_cuda, a, b, plan=pl)
            assert info["n_windows_mfma"] > 0 or (m, k, p) in dense, (m, k, n)
            want_kernel = {S.TCA_PLAN_MFMA_PAIR: {3}, 0: {3, 5, 7, 8}, S.TCA_PLAN_MFMA_DENSE: {4, 5},
                           S.TCA_PLAN_MFMA_COMPACT: {7, 4, 5}}[variant]
            assert info["tile_kernel"] in want_kernel or info["n_windows_mfma"] == 0, (variant, info["tile_kernel"])
            want = oracle_c(a, b)
            assert np.array_equal(got, want), (m, k, p, n, np.abs(got - want).max())


@pytest.mark.parametrize("dtype", [S.TCA_F16, S.TCA_BF16])
def test_short_k_kernel_bit_exact(torch_cuda, dtype):
    """The short-K kernel (every row; 32-row windows built in LDS from the
    CSR each run) is bit-equal to the oracle on exact-arithmetic inputs:
    partial windows and column blocks, K not a multiple of 32, K = 1 and
    640, empty rows and rows holding all of K.  Routing: the flag forces it
    at any row length; by default it takes K <= 640 at >= max(8, 0.08 K)
    nonzeros per row; K = 641, fp32, TCA_PLAN_NO_MFMA and sparser rows stay
    off it."""
    rng = np.random.default_rng(131 + dtype)
    for m, k, p in [(2048, 512, 0.1), (37, 40, 0.5), (64, 640, 0.05), (100, 1, 1.0), (33, 100, 1.0),
                    (5, 600, 0.02), (300, 33, 0.3), (1, 64, 0.0), (200, 97, 0.2)]:
        lens = rng.binomial(k, p, m)
        lens[rng.random(m) < 0.1] = 0
        if m > 3:
            lens[3] = k  # a row holding all of K
        a = make_csr(rng, lens, k, dtype)
        for n in (8, 16, 64, 136, 256):
            b = S.to_storage(exact_dense(rng, (k, n)), dtype)
            with S.Plan(a, n, S.TCA_PLAN_MFMA_SHORT) as pl:
                info = pl.info()
                got = run_gpu(torch_cuda, a, b, plan=pl)
            assert info["tile_kernel"] == S.TCA_TILES_SHORT and info["n_row_tasks"] == 0, (m, k, n, info)
            want = oracle_c(a, b)
            assert np.array_equal(got, want), (m, k, p, n, np.abs(got - want).max())
    a0, n0, _ = S.gen_config(0, seed=1)
    with S.Plan(a0, n0) as pl:
        assert pl.info()["tile_kernel"] == S.TCA_TILES_SHORT
    sparse, _ = S.gen_bernoulli(256, 512, 0.05, seed=2, dtype=S.TCA_F16)       # ~26 per row, 5 %
    wide, _ = S.gen_bernoulli(256, 641, 0.1, seed=3, dtype=S.TCA_F16)
    for mat, flags in ((sparse, 0), (wide, S.TCA_PLAN_MFMA_SHORT), (a0, S.TCA_PLAN_NO_MFMA),
                       (a0.astype(S.TCA_F32), S.TCA_PLAN_MFMA_SHORT), (a0, S.TCA_PLAN_MFMA_PAIR)):
        with S.Plan(mat, 64, flags) as pl:
            assert pl.info()["tile_kernel"] != S.TCA_TILES_SHORT, flags


def test_mfma_and_row_paths_agree(torch_cuda):
    rng = np.random.default_rng(81)
    a, _ = S.gen_bernoulli(300, 900, 0.05, seed=5, dtype=S.TCA_F16)
    a = S.CSR(a.nrow, a.ncol, a.rowptr, a.colidx, S.to_storage(exact_values(rng, a.nnz), S.TCA_F16), S.TCA_F16)
    b = S.to_storage(exact_dense(rng, (900, 256)), S.TCA_F16)
    outs = {}
    for flags in (S.TCA_PLAN_NO_MFMA, S.TCA_PLAN_FORCE_MFMA, S.TCA_PLAN_DEFAULT):
        with S.Plan(a, 256, flags) as pl:
            nwin = pl.info()["n_windows_mfma"]
            outs[flags] = run_gpu(torch_cuda, a, b, plan=pl)
        if flags != S.TCA_PLAN_DEFAULT:
            assert (nwin > 0) == (flags == S.TCA_PLAN_FORCE_MFMA)
    assert np.array_equal(outs[S.TCA_PLAN_NO_MFMA], outs[S.TCA_PLAN_FORCE_MFMA])
    assert np.array_equal(outs[S.TCA_PLAN_DEFAULT], oracle_c(a, b))


@pytest.mark.parametrize("lookahead", ["3", "4"])
def test_compact_tiles_equal_dense_tiles(torch_cuda, lookahead, monkeypatch):
    """Compacted steps (only the non-empty 16-byte fragment cells) give the
    dense-tile kernel's products bit for bit (same fragments, same MFMA and
    partial-sum order) on a config-1-like matrix, natural and condensed
    column order, both lookaheads; a step with more than 255 non-empty
    cells keeps the plain dense tiles."""
    monkeypatch.setenv("TCA_COMPACT_LB", lookahead)
    rng = np.random.default_rng(91)
    for m, k, mean, n in [(1024, 2048, 100, 512), (640, 4096, 60, 136), (300, 8000, 20, 64)]:
        print(f"compact vs dense LB={lookahead}: M={m} K={k} mean={mean} N={n}", flush=True)
        a, _ = S.gen_lognormal_rows(m, k, mean, seed=7, dtype=S.TCA_F16)
        a = S.CSR(a.nrow, a.ncol, a.rowptr, a.colidx, S.to_storage(exact_values(rng, a.nnz), S.TCA_F16), S.TCA_F16)
        b = S.to_storage(exact_dense(rng, (k, n)), S.TCA_F16)
        outs = {}
        for flags in (S.TCA_PLAN_FORCE_MFMA | S.TCA_PLAN_MFMA_DENSE, S.TCA_PLAN_FORCE_MFMA | S.TCA_PLAN_MFMA_COMPACT):
            with S.Plan(a, n, flags) as pl:
                info = pl.info()
                outs[flags] = run_gpu(torch_cuda, a, b, plan=pl)
            assert info["n_windows_mfma"] > 0, (m, k)
            if flags & S.TCA_PLAN_MFMA_COMPACT:
                assert info["tile_kernel"] == S.TCA_TILES_COMPACT, info["tile_kernel"]
        vals = list(outs.values())
        assert np.array_equal(vals[0], vals[1]), (m, k, n, np.abs(vals[0] - vals[1]).max())
        assert np.array_equal(vals[1], oracle_c(a, b)), (m, k, n)
    # every cell of a step non-empty: no compaction
    a, _ = S.gen_bernoulli(256, 512, 0.6, seed=9, dtype=S.TCA_F16)
    a = S.CSR(a.nrow, a.ncol, a.rowptr, a.colidx, S.to_storage(exact_values(rng, a.nnz), S.TCA_F16), S.TCA_F16)
    b = S.to_storage(exact_dense(rng, (512, 64)), S.TCA_F16)
    with S.Plan(a, 64, S.TCA_PLAN_FORCE_MFMA | S.TCA_PLAN_MFMA_COMPACT) as pl:
        assert pl.info()["tile_kernel"] in (S.TCA_TILES_DENSE, S.TCA_TILES_DENSE_K), pl.info()["tile_kernel"]
        got = run_gpu(torch_cuda, a, b, plan=pl)
    assert np.array_equal(got, oracle_c(a, b))


@pytest.mark.parametrize("order", ["0", "1"])
def test_exact_long_rows_many_segments(torch_cuda, monkeypatch, order):
    """Rows far above the segment length; every output element exact, with the
    segments launched in task order or by column range per XCD."""
    monkeypatch.setenv("TCA_ROW_ORDER", order)
    rng = np.random.default_rng(21)
    k = 16000
    lens = [15000, 9000, 12000, 0, 3, 16000 - 1]
    a = make_csr(rng, lens, k, S.TCA_F16)
    info = None
    for n in (64, 256, 512):
        b = S.to_storage(exact_dense(rng, (k, n)), S.TCA_F16)
        with S.Plan(a, n, S.TCA_PLAN_NO_MFMA | S.TCA_PLAN_NO_PANELS) as p:  # the segment path of the row kernel
            info = p.info()
            got = run_gpu(torch_cuda, a, b, plan=p)
        assert info["n_long_rows"] >= 4
        slots = (info["n_row_tasks"] + 3) // 4 * info["col_chunks"]
        if order == "1" and info["col_chunks"] == 1:  # segments reordered (idle slots pad the XCD queues)
            assert info["row_blocks"] >= slots, info
        else:
            assert info["row_blocks"] == slots, info
        assert np.array_equal(got, oracle_c(a, b)), n


@pytest.mark.parametrize("n", [3, 13, 1023])
def test_exact_segments_ragged_widths(torch_cuda, n):
    """Segmented long rows at widths that are not a multiple of 4: the segment
    sums take the scalar path, each thread its own (up to) 4 columns."""
    rng = np.random.default_rng(23 + n)
    k = 12000
    a = make_csr(rng, [11000, 7, 9000, 0, 11999], k, S.TCA_F32)
    b = S.to_storage(exact_dense(rng, (k, n)), S.TCA_F32)
    with S.Plan(a, n, S.TCA_PLAN_NO_MFMA | S.TCA_PLAN_NO_PANELS) as p:
        info = p.info()
        got = run_gpu(torch_cuda, a, b, plan=p)
    assert info["n_long_rows"] >= 3, info
    assert np.array_equal(got, oracle_c(a, b)), n


def test_plan_reuse_and_determinism(torch_cuda):
    """One plan, several B: tickets reset between launches; identical bits on repeat."""
    rng = np.random.default_rng(31)
    a, _ = S.gen_zipf_rows(4000, 20000, 300000, s=1.5, cap=50000, seed=3)
    n = 64
    with S.Plan(a, n) as p:
        assert p.info()["n_long_rows"] > 0
        outs = []
        for seed in (1, 2, 1):
            b = S.gen_dense(a.ncol, n, 0, seed=seed, dtype=S.TCA_F16)
            got = run_gpu(torch_cuda, a, b, plan=p)
            assert_parity(a, b, got, f"seed {seed}")
            outs.append(got)
        assert np.array_equal(outs[0], outs[2])
        assert not np.array_equal(outs[0], outs[1])


def test_empty_and_degenerate(torch_cuda):
    rng = np.random.default_rng(41)
    # no nonzeros at all: C must be all zeros
    a = S.CSR(5, 7, np.zeros(6, np.int32), np.zeros(0, np.int32), np.zeros(0, np.float16), S.TCA_F16)
    got = run_gpu(torch_cuda, a, S.to_storage(np.ones((7, 16)), S.TCA_F16))
    assert np.array_equal(got, np.zeros((5, 16), np.float32))
    # a single dense row
    a = make_csr(rng, [300], 300, S.TCA_F32)
    b = S.to_storage(exact_dense(rng, (300, 33)), S.TCA_F32)
    assert np.array_equal(run_gpu(torch_cuda, a, b), oracle_c(a, b))
    # one column matrix
    a = make_csr(rng, [1, 0, 1], 1, S.TCA_F16)
    b = S.to_storage(np.array([[0.75]]), S.TCA_F16)
    assert np.array_equal(run_gpu(torch_cuda, a, b), oracle_c(a, b))


@pytest.mark.parametrize("dtype,n", [(S.TCA_F16, 64), (S.TCA_F32, 128), (S.TCA_F32, 7), (S.TCA_BF16, 1000)],
                         ids=["f16-n64", "f32-n128", "f32-n7", "bf16-n1000-chunks"])
def test_runs_of_empty_rows(torch_cuda, dtype, n):
    """Empty rows in long consecutive runs (zero tasks whose rows are one
    contiguous range of C, cleared as one range) and scattered ones (the
    row-by-row clear), between rows with nonzeros; N not a multiple of 4 and
    several column chunks keep the row-by-row clear.  C starts as NaN, so
    every row must be written."""
    rng = np.random.default_rng(61 + n)
    lens = np.zeros(6000, np.int64)
    lens[::97] = rng.integers(1, 40, len(lens[::97]))   # long runs of empty rows between them
    lens[3000:3300:2] = rng.integers(1, 5, 150)          # a stretch of alternating rows
    lens[5999] = 3
    k = 500
    a = make_csr(rng, lens, k, dtype)
    b = S.to_storage(exact_dense(rng, (k, n)), dtype)
    got = run_gpu(torch_cuda, a, b, S.TCA_PLAN_NO_MFMA | S.TCA_PLAN_NO_PANELS)
    assert np.array_equal(got, oracle_c(a, b))


def test_misaligned_b_is_rejected(torch_cuda):
    torch = torch_cuda
    rng = np.random.default_rng(51)
    a = make_csr(rng, [3, 4], 10, S.TCA_F16)
    with S.Plan(a, 64) as p:
        buf = torch.zeros(10 * 64 + 1, dtype=torch.float16, device="cuda:0")
        c = torch.zeros((2, 64), dtype=torch.float32, device="cuda:0")
        val = _dev(torch, a.values)
        with pytest.raises(S.TcaError):
            p.run(val, buf.data_ptr() + 2, c)


def test_nondefault_stream(torch_cuda):
    torch = torch_cuda
    rng = np.random.default_rng(61)
    a = make_csr(rng, rng.integers(0, 50, 500), 800, S.TCA_F16)
    b = S.to_storage(exact_dense(rng, (800, 128)), S.TCA_F16)
    s = torch.cuda.Stream()
    with S.Plan(a, 128) as p:
        val, bd = _dev(torch, a.values), _dev(torch, b)
        c = torch.empty((a.nrow, 128), dtype=torch.float32, device="cuda:0")
        torch.cuda.synchronize()
        p.run(val, bd, c, stream=s.cuda_stream)
        s.synchronize()
        assert np.array_equal(c.cpu().numpy(), oracle_c(a, b))


def test_host_driver_our_spmm_balanced(torch_cuda):
    a = S.read_smtx(os.path.join(GOLDEN, "body_decoder_layer_2_ffn_conv1.smtx"))
    b = S.gen_dense(a.ncol, 256, 3, seed=7, dtype=S.TCA_F16, sparsity=0.1)
    c, ms = S.our_spmm_balanced(a, b, n_iter=10)
    assert ms > 0
    assert_parity(a, b, c, "host driver")


# ------------------------------------------------------------- configs
@pytest.mark.parametrize("cfg", [0, 1])
def test_config_full_size_small(torch_cuda, cfg):
    a, n, st = S.gen_config(cfg, seed=1)
    dist = 0
    b = S.gen_dense(a.ncol, n, dist, seed=100 + cfg, dtype=a.dtype)
    print(f"config {cfg}: M={a.nrow} K={a.ncol} N={n} nnz={a.nnz}", flush=True)
    got = run_gpu(torch_cuda, a, b)
    assert_close(oracle_c(a, b), got, f"config {cfg} vs fp32 oracle")
    assert_parity(a, b, got, f"config {cfg}")
    # both kernels on the whole matrix
    for flags, what in ((S.TCA_PLAN_NO_MFMA | S.TCA_PLAN_NO_PANELS, "row kernel only"),
                        (S.TCA_PLAN_FORCE_MFMA, "MFMA tiles only")):
        with S.Plan(a, n, flags) as pl:
            info = pl.info()
            got_k = run_gpu(torch_cuda, a, b, plan=pl)
        assert (info["rows_mfma"] == a.nrow) == (flags == S.TCA_PLAN_FORCE_MFMA)
        assert_parity(a, b, got_k, f"config {cfg} {what}")


@pytest.mark.parametrize("cfg", [2, 3, 4])
def test_config_full_size_large(torch_cuda, cfg):
    a, n, st = S.gen_config(cfg, seed=1)
    dist = 1 if cfg in (2, 3) else 0
    b = S.gen_dense(a.ncol, n, dist, seed=100 + cfg, dtype=a.dtype)
    print(f"config {cfg}: M={a.nrow} K={a.ncol} N={n} nnz={a.nnz}", flush=True)
    got = run_gpu(torch_cuda, a, b)
    assert_parity(a, b, got, f"config {cfg}")
    # size-independent check: row sums of C equal A times the row sums of B
    row_sum_gold = oracle.csr_spmm_f64(a.rowptr, a.colidx, a.values_f32().astype(np.float64),
                                       S.from_storage(b, a.dtype).astype(np.float64).sum(1, keepdims=True))
    s_abs = oracle.csr_spmm_f64(a.rowptr, a.colidx, np.abs(a.values_f32().astype(np.float64)),
                                np.abs(S.from_storage(b, a.dtype).astype(np.float64)).sum(1, keepdims=True))
    err = np.abs(got.astype(np.float64).sum(1) - row_sum_gold[:, 0])
    assert np.all(err <= 1e-3 * np.maximum(np.abs(row_sum_gold[:, 0]), 1e-3 * s_abs[:, 0]) + 1e-30)


def test_phase_timing_reports_the_kernels_a_plan_uses(torch_cuda):
    """tca_spmm_time_phases: a phase the plan does not use reads 0, the used
    ones are positive, and C holds the exact product afterwards (short-K
    plan: one launch, no pack; dense-tile and paired-kernel plans; row-kernel
    and panel plans)."""
    torch = torch_cuda
    rng = np.random.default_rng(97)
    a, _ = S.gen_bernoulli(256, 512, 0.08, seed=9, dtype=S.TCA_F16)
    a = S.CSR(a.nrow, a.ncol, a.rowptr, a.colidx, S.to_storage(exact_values(rng, a.nnz), S.TCA_F16), S.TCA_F16)
    b = S.to_storage(exact_dense(rng, (512, 256)), S.TCA_F16)
    dev = torch.device("cuda:0")
    val = torch.from_numpy(a.values.view(np.int16)).to(dev)
    bd = torch.from_numpy(b.view(np.int16)).to(dev)
    for flags, used in ((S.TCA_PLAN_FORCE_MFMA, {"tiles"}),
                        (S.TCA_PLAN_FORCE_MFMA | S.TCA_PLAN_MFMA_DENSE, {"pack", "tiles"}),
                        (S.TCA_PLAN_FORCE_MFMA | S.TCA_PLAN_MFMA_PAIR, {"pack", "tiles"}),
                        (S.TCA_PLAN_NO_MFMA | S.TCA_PLAN_NO_PANELS, {"rows"}),
                        (S.TCA_PLAN_NO_MFMA | S.TCA_PLAN_FORCE_PANELS, {"panels"})):
        c = torch.zeros((a.nrow, 256), dtype=torch.float32, device=dev)
        with S.Plan(a, 256, flags) as pl:
            ph = pl.time_phases(val, bd, c, warmup=1, iters=3)
            if pl.info()["n_long_rows"] > 0:  # rows split over several units or segments
                used = used | {"segments"}
            named = pl.phases()
        torch.cuda.synchronize()
        assert {k for k, v in ph.items() if v > 0} == used, (flags, ph)
        assert set(named) == used and list(named) == [k for k in ("pack", "tiles", "panels", "rows", "segments")
                                                      if k in used], (flags, named)
        assert np.array_equal(c.cpu().numpy(), oracle_c(a, b))


def test_subset_timing_runs_only_the_named_phases(torch_cuda):
    """tca_spmm_time_subset: with every phase of the plan C holds the exact
    product; with all but the first phase the rows of that phase stay as they
    were (NaN here) while the other rows are exact; an empty subset launches
    nothing; a mask bit beyond the phases is rejected."""
    torch = torch_cuda
    rng = np.random.default_rng(98)
    a, _ = S.gen_bernoulli(256, 512, 0.08, seed=10, dtype=S.TCA_F16)
    a = S.CSR(a.nrow, a.ncol, a.rowptr, a.colidx, S.to_storage(exact_values(rng, a.nnz), S.TCA_F16), S.TCA_F16)
    b = S.to_storage(exact_dense(rng, (512, 256)), S.TCA_F16)
    dev = torch.device("cuda:0")
    val = torch.from_numpy(a.values.view(np.int16)).to(dev)
    bd = torch.from_numpy(b.view(np.int16)).to(dev)
    want = oracle_c(a, b)
    # MFMA windows on the leading rows, the row kernel on the rest
    flags = S.TCA_PLAN_FORCE_MFMA | S.TCA_PLAN_MFMA_DENSE
    with S.Plan(a, 256, flags) as pl:
        phases = pl.phases()
        assert phases[:2] == ("pack", "tiles"), phases
        c = torch.full((a.nrow, 256), float("nan"), dtype=torch.float32, device=dev)
        assert pl.time_subset(val, bd, c, phases, warmup=1, iters=3) > 0
        torch.cuda.synchronize()
        assert np.array_equal(c.cpu().numpy(), want)
        c.fill_(float("nan"))
        assert pl.time_subset(val, bd, c, (), warmup=1, iters=2) >= 0
        torch.cuda.synchronize()
        assert torch.isnan(c).all().item()
        if "rows" in phases:
            pl.time_subset(val, bd, c, ("rows",) + (("segments",) if "segments" in phases else ()), warmup=0, iters=1)
            torch.cuda.synchronize()
            got = c.cpu().numpy()
            done = ~np.isnan(got).any(axis=1)
            assert done.any() and not done.all()
            assert np.array_equal(got[done], want[done])
        with pytest.raises(S.TcaError) as ei:
            S._lib.call("tca_spmm_time_subset", pl._p, val.data_ptr(), bd.data_ptr(), c.data_ptr(), None,
                        1 << len(S.Plan.PHASES), 0, 1, ctypes.byref(ctypes.c_float()))
        assert ei.value.status == 1
