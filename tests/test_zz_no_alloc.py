"""The allocation-free entry point tca_spmm_run_static (through the C ABI)
against tca_spmm_run: the same kernels with the partial rows of split rows in
the library's static scratch instead of plan-owned memory, so the products
must be bit-identical -- on two calls in a row, the second on a smaller
input, with plans that have partial rows from both the row kernel's
segments and split panels."""
import numpy as np
import pytest

from conftest import exact_dense, exact_values

import spmm_amd as S
from test_gpu_parity import _dev, oracle_c

pytestmark = pytest.mark.gpu

STATIC_BYTES = 64 << 20


def _case(rows, k, total, cap, seed, dtype):
    a, _ = S.gen_zipf_rows(rows, k, total, s=1.5, cap=cap, seed=seed)
    rng = np.random.default_rng(seed)
    v = exact_values(rng, a.nnz)
    v[v == 0] = 0.5
    return S.CSR(a.nrow, a.ncol, a.rowptr, a.colidx, S.to_storage(v, dtype), dtype)


def _run_both(torch, a, n, flags):
    rng = np.random.default_rng(a.nnz)
    b = S.to_storage(exact_dense(rng, (a.ncol, n)), a.dtype)
    val, bd = _dev(torch, a.values), _dev(torch, b)
    c_ref = torch.full((a.nrow, n), float("nan"), dtype=torch.float32, device="cuda:0")
    c_st = torch.full((a.nrow, n), float("nan"), dtype=torch.float32, device="cuda:0")
    with S.Plan(a, n, flags) as pr, S.Plan(a, n, flags | S.TCA_PLAN_NO_SCRATCH) as ps:
        info = ps.info()
        assert info["scratch_bytes"] > 0, info  # the plan has partial rows
        assert info["scratch_bytes"] <= STATIC_BYTES
        pr.run(val, bd, c_ref)
        ps.run_static(val, bd, c_st)
        with pytest.raises(S.TcaError):  # a plan without scratch needs the static entry point
            ps.run(val, bd, c_st)
    torch.cuda.synchronize()
    got, want = c_st.cpu().numpy(), c_ref.cpu().numpy()
    assert np.array_equal(got, want)
    assert np.array_equal(got, oracle_c(a, b))  # exact-arithmetic inputs: the oracle's bits
    return info


def test_run_static_equals_run_two_calls(torch_cuda, monkeypatch):
    monkeypatch.setenv("TCA_PANEL_UNIT", "4000")  # split panels into units (partial rows)
    # first call: row-kernel segments (long rows) and split panels, fp32 N = 128
    big = _case(6000, 20000, 400000, 30000, 3, S.TCA_F32)
    i1 = _run_both(torch_cuda, big, 128, S.TCA_PLAN_FORCE_PANELS)
    assert i1["n_panels"] > 0 and i1["n_long_rows"] > 0
    # second call, smaller: the row kernel's segments only, fp16 N = 64
    small = _case(1500, 8000, 60000, 12000, 5, S.TCA_F16)
    i2 = _run_both(torch_cuda, small, 64, S.TCA_PLAN_NO_PANELS | S.TCA_PLAN_NO_MFMA)
    assert i2["n_long_rows"] > 0 and i2["scratch_bytes"] < i1["scratch_bytes"]


def test_run_static_rejects_plans_past_the_scratch(torch_cuda, monkeypatch):
    """A plan whose partial rows exceed the 64 MiB static array is refused
    before any launch, with the sizes in the message."""
    monkeypatch.setenv("TCA_PANEL_UNIT", "600")
    a = _case(4000, 3000, 150000, 3000, 7, S.TCA_F32)
    n = 1024
    with S.Plan(a, n, S.TCA_PLAN_FORCE_PANELS | S.TCA_PLAN_NO_SCRATCH) as ps:
        assert ps.info()["scratch_bytes"] > STATIC_BYTES
        val = _dev(torch_cuda, a.values)
        bd = torch_cuda.zeros((a.ncol, n), dtype=torch_cuda.float32, device="cuda:0")
        c = torch_cuda.zeros((a.nrow, n), dtype=torch_cuda.float32, device="cuda:0")
        with pytest.raises(S.TcaError, match="static scratch holds"):
            ps.run_static(val, bd, c)
