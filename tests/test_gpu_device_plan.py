"""Planning on the GPU (tca_spmm_plan_create_device): the task list built by
device kernels from a device-resident CSR equals the host planner's
(TCA_PLAN_NO_MFMA | TCA_PLAN_NO_PANELS; panels: test_gpu_device_panels.py)
entry for entry, the matrix-core windows and their dense
tiles (natural and condensed) equal the host planner's for the same flags,
and the plans give bit-identical products; invalid structures are rejected
on the device."""
import numpy as np
import pytest

from conftest import exact_dense
from oracle import oracle
from test_gpu_parity import _dev

import spmm_amd as S

pytestmark = pytest.mark.gpu


def _cases():
    yield "bernoulli", S.gen_bernoulli(3000, 2000, 0.01, seed=1, dtype=S.TCA_F16)[0], 256
    yield "lognormal", S.gen_lognormal_rows(4096, 4096, 205, seed=1, dtype=S.TCA_F16)[0], 512
    yield "lognormal-f32", S.gen_lognormal_rows(2000, 3000, 50, seed=2, dtype=S.TCA_F32)[0], 128
    yield "rmat", S.gen_rmat(14, 12000, 400000, seed=3, dtype=S.TCA_F32)[0], 128
    yield "zipf", S.gen_zipf_rows(60000, 60000, 2000000, seed=4, dtype=S.TCA_F16)[0], 64
    yield "narrow", S.gen_bernoulli(500, 700, 0.05, seed=5, dtype=S.TCA_F16)[0], 8
    yield "wide-n", S.gen_bernoulli(300, 400, 0.05, seed=6, dtype=S.TCA_F32)[0], 1000


@pytest.mark.parametrize("name,a,n", list(_cases()), ids=[c[0] for c in _cases()])
def test_device_plan_equals_host_plan(torch_cuda, name, a, n):
    torch = torch_cuda
    print(f"device plan {name}: M={a.nrow} K={a.ncol} nnz={a.nnz} N={n}", flush=True)
    drp, dci = _dev(torch, a.rowptr), _dev(torch, a.colidx)
    with S.Plan(a, n, S.TCA_PLAN_NO_MFMA | S.TCA_PLAN_NO_PANELS) as hp:
        dp = S.Plan.from_device(drp, dci, a.nrow, a.ncol, a.nnz, n, a.dtype, S.TCA_PLAN_NO_MFMA | S.TCA_PLAN_NO_PANELS)
        try:
            ht, hperm, hl = hp.export_rows()
            dt, dperm, dl = dp.export_rows()
            assert np.array_equal(ht, dt) and np.array_equal(hperm, dperm) and np.array_equal(hl, dl), name
            ho, do = hp.export_order(), dp.export_order()
            assert np.array_equal(ho, do), name  # the same launch order (segments by column range per XCD)
            if len(ho):
                assert sorted(ho[ho >= 0].tolist()) == list(range(len(ht))), name  # every task once
            if name == "zipf":
                assert len(ho) > 0, name  # long rows in segments, one column chunk: ordered
            hi, di = hp.info(), dp.info()
            for key in ("n_row_tasks", "n_multi_tasks", "n_seg_tasks", "n_long_rows", "n_wide_tasks", "scratch_bytes",
                        "row_blocks"):  # row_blocks: the same launch order length (segments by column range)
                assert hi[key] == di[key], (name, key)
            rng = np.random.default_rng(7)
            b = S.to_storage(exact_dense(rng, (a.ncol, n)), a.dtype)
            val, bd = _dev(torch, a.values), _dev(torch, b)
            outs = []
            for pl in (hp, dp):
                c = torch.full((a.nrow, n), float("nan"), dtype=torch.float32, device="cuda:0")
                pl.run(val, bd, c)
                torch.cuda.synchronize()
                outs.append(c.cpu().numpy())
            assert np.array_equal(outs[0], outs[1]), name
            assert np.all(np.isfinite(outs[1]))
        finally:
            dp.close()


def _mixed(seed):
    """Dense windows (rows 0..383, ~40 % of K) over sparse ones: some windows
    are routed, the rest stay on the row kernel, the routed ones condense."""
    rng = np.random.default_rng(seed)
    m, k = 900, 2000
    lens = np.where(np.arange(m) < 384, rng.integers(60, 120, m), rng.integers(0, 6, m))
    rowptr = np.zeros(m + 1, np.int32)
    np.cumsum(lens, out=rowptr[1:])
    cols = []
    for r in range(m):
        pool = 800 if r < 384 else k
        cols.append(np.sort(rng.choice(pool, lens[r], replace=False)).astype(np.int32))
    colidx = np.concatenate(cols).astype(np.int32)
    return S.CSR(m, k, rowptr, colidx, S.to_storage(np.ones(len(colidx), np.float32), S.TCA_F16), S.TCA_F16)


def _mfma_cases():
    yield "lognormal-natural", S.gen_lognormal_rows(4096, 4096, 205, seed=1, dtype=S.TCA_F16)[0], 512
    yield "ragged-natural", S.gen_lognormal_rows(1000, 1500, 80, seed=9, dtype=S.TCA_BF16)[0], 136
    yield "mixed-condensed", _mixed(3), 256
    yield "bernoulli", S.gen_bernoulli(3000, 2000, 0.01, seed=1, dtype=S.TCA_F16)[0], 256


@pytest.mark.parametrize("flags", [S.TCA_PLAN_DEFAULT, S.TCA_PLAN_MFMA_DENSE,
                                   S.TCA_PLAN_FORCE_MFMA | S.TCA_PLAN_MFMA_DENSE, S.TCA_PLAN_MFMA_COMPACT],
                         ids=["default", "dense", "force-dense", "compact"])
@pytest.mark.parametrize("name,a,n", list(_mfma_cases()), ids=[c[0] for c in _mfma_cases()])
def test_device_mfma_plan_equals_host_plan(torch_cuda, name, a, n, flags):
    """Windows, dense-tile positions (compacted or not), B row offsets and
    row tasks equal the host planner's; products bit-identical and equal to
    the oracle on exact inputs.  (By default, windows that do not cover most
    of K run on the paired kernel when planned on the host and on condensed
    dense tiles when planned on the GPU: there only the products are
    compared.)"""
    torch = torch_cuda
    print(f"device mfma plan {name} flags={flags}: M={a.nrow} K={a.ncol} nnz={a.nnz} N={n}", flush=True)
    rng = np.random.default_rng(11)
    v = rng.choice(np.array([-2.0, -1.0, -0.5, 0.5, 1.0, 2.0], np.float32), size=a.nnz)
    a = S.CSR(a.nrow, a.ncol, a.rowptr, a.colidx, S.to_storage(v, a.dtype), a.dtype)
    b = S.to_storage(exact_dense(rng, (a.ncol, n)), a.dtype)
    with S.Plan(a, n, flags | S.TCA_PLAN_NO_PANELS) as hp:
        dp = S.Plan.from_device(_dev(torch, a.rowptr), _dev(torch, a.colidx), a.nrow, a.ncol, a.nnz, n, a.dtype, flags)
        try:
            hi, di = hp.info(), dp.info()
            # host default tiles the device planner does not build: paired (3);
            # the device plans condensed dense tiles there
            same = not (flags == S.TCA_PLAN_DEFAULT and hi["tile_kernel"] == 3)
            for key in ("n_windows_mfma", "rows_mfma", "nnz_mfma"):
                assert hi[key] == di[key], (name, key, hi[key], di[key])
            if same:
                for key in ("cond_cols_mfma", "tile_kernel", "mfma_blocks", "n_row_tasks", "n_multi_tasks",
                            "n_seg_tasks", "n_long_rows", "n_wide_tasks"):
                    assert hi[key] == di[key], (name, key, hi[key], di[key])
                for x, y in zip(hp.export_rows(), dp.export_rows()):
                    assert np.array_equal(x, y), name
                for x, y in zip(hp.export_tiles(), dp.export_tiles()):
                    assert np.array_equal(x, y), name
            else:
                assert di["tile_kernel"] == 4, (hi["tile_kernel"], di["tile_kernel"])
            if flags == S.TCA_PLAN_DEFAULT and name.endswith("-natural") and hi["n_windows_mfma"] > 0:
                assert hi["tile_kernel"] == di["tile_kernel"] == S.TCA_TILES_COMPACT, (hi, di)
            val, bd = _dev(torch, a.values), _dev(torch, b)
            outs = []
            for pl in (hp, dp):
                c = torch.full((a.nrow, n), float("nan"), dtype=torch.float32, device="cuda:0")
                pl.run(val, bd, c)
                torch.cuda.synchronize()
                outs.append(c.cpu().numpy())
            want = oracle.csr_spmm(a.rowptr, a.colidx, a.values_f32(), S.from_storage(b, a.dtype))
            assert np.array_equal(outs[1], want), name
            assert np.array_equal(outs[0], outs[1]), name
        finally:
            dp.close()


def test_device_plan_result_matches_oracle(torch_cuda):
    torch = torch_cuda
    a = S.gen_lognormal_rows(1000, 1500, 80, seed=9, dtype=S.TCA_F16)[0]
    rng = np.random.default_rng(9)
    v = rng.choice(np.array([-2.0, -1.0, -0.5, 0.5, 1.0, 2.0], np.float32), size=a.nnz)
    a = S.CSR(a.nrow, a.ncol, a.rowptr, a.colidx, S.to_storage(v, S.TCA_F16), S.TCA_F16)
    b = S.to_storage(exact_dense(rng, (a.ncol, 128)), S.TCA_F16)
    dp = S.Plan.from_device(_dev(torch, a.rowptr), _dev(torch, a.colidx), a.nrow, a.ncol, a.nnz, 128, a.dtype)
    c = torch.empty((a.nrow, 128), dtype=torch.float32, device="cuda:0")
    dp.run(_dev(torch, a.values), _dev(torch, b), c)
    torch.cuda.synchronize()
    dp.close()
    want = oracle.csr_spmm(a.rowptr, a.colidx, a.values_f32(), S.from_storage(b, S.TCA_F16))
    assert np.array_equal(c.cpu().numpy(), want)


@pytest.mark.parametrize("bad", ["rowptr-decreasing", "rowptr-end", "col-range", "col-order"])
def test_device_plan_rejects_invalid_structure(torch_cuda, bad):
    torch = torch_cuda
    rowptr = np.array([0, 2, 3, 5], np.int32)
    colidx = np.array([0, 3, 1, 2, 4], np.int32)
    if bad == "rowptr-decreasing":
        rowptr[2] = 1
    elif bad == "rowptr-end":
        rowptr[3] = 4
    elif bad == "col-range":
        colidx[4] = 5
    else:
        colidx[1] = 0
    with pytest.raises(S.TcaError) as ei:
        S.Plan.from_device(_dev(torch, rowptr), _dev(torch, colidx), 3, 5, 5, 64, S.TCA_F32)
    assert ei.value.status == 1


@pytest.mark.parametrize("m,k,p,n", [(2048, 512, 0.1, 256), (1000, 97, 0.3, 136), (70, 640, 0.2, 8)])
def test_device_short_k_plan_equals_host_plan(torch_cuda, m, k, p, n):
    """Short K: host and device planners both route every row to the short-K
    kernel (the same windows and launch), and the products are bit-identical
    and equal to the oracle on exact inputs."""
    torch = torch_cuda
    print(f"device short-K plan: M={m} K={k} p={p} N={n}", flush=True)
    rng = np.random.default_rng(m + k)
    a = S.gen_bernoulli(m, k, p, seed=m, dtype=S.TCA_F16)[0]
    v = rng.choice(np.array([-2.0, -1.0, -0.5, 0.5, 1.0, 2.0], np.float32), size=a.nnz)
    a = S.CSR(a.nrow, a.ncol, a.rowptr, a.colidx, S.to_storage(v, a.dtype), a.dtype)
    b = S.to_storage(exact_dense(rng, (k, n)), a.dtype)
    with S.Plan(a, n) as hp:
        dp = S.Plan.from_device(_dev(torch, a.rowptr), _dev(torch, a.colidx), m, k, a.nnz, n, a.dtype)
        try:
            hi, di = hp.info(), dp.info()
            for key in ("tile_kernel", "n_windows_mfma", "rows_mfma", "nnz_mfma", "mfma_blocks", "n_row_tasks"):
                assert hi[key] == di[key], (key, hi[key], di[key])
            assert hi["tile_kernel"] == S.TCA_TILES_SHORT
            val, bd = _dev(torch, a.values), _dev(torch, b)
            outs = []
            for pl in (hp, dp):
                c = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda:0")
                pl.run(val, bd, c)
                torch.cuda.synchronize()
                outs.append(c.cpu().numpy())
            want = oracle.csr_spmm(a.rowptr, a.colidx, a.values_f32(), S.from_storage(b, a.dtype))
            assert np.array_equal(outs[0], want) and np.array_equal(outs[1], want)
        finally:
            dp.close()
