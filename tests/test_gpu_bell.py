"""GPU parity of the Blocked-ELL MFMA kernel (tca_bell_spmm) against the CPU
oracle: bit-exact on exact-arithmetic inputs, within the reference verdict
and a 1e-3 relative bar elsewhere, for block sizes 32 and 64, fp16 / bf16,
ragged M, K and N, block rows without blocks and long block lists."""
import numpy as np
import pytest

from conftest import exact_dense, exact_values
from oracle import oracle
from test_gpu_parity import _dev, assert_parity

import spmm_amd as S

pytestmark = pytest.mark.gpu


def _csr(rng, m, k, p, dtype, exact=True, empty_rows=()):
    mask = rng.random((m, k)) < p
    for r in empty_rows:
        mask[r] = False
    lens = mask.sum(axis=1)
    rowptr = np.zeros(m + 1, np.int32)
    np.cumsum(lens, out=rowptr[1:])
    colidx = np.nonzero(mask)[1].astype(np.int32)
    nnz = int(rowptr[-1])
    v = exact_values(rng, nnz) if exact else (rng.standard_normal(nnz) * 0.02).astype(np.float32)
    v[v == 0] = 0.5
    return S.CSR(m, k, rowptr, colidx, S.to_storage(v, dtype), dtype)


def _run(torch, a, b, bs):
    colind, vals = S.csr_to_bell(a, bs)
    n = b.shape[1]
    dc = _dev(torch, colind)
    dv = _dev(torch, vals)
    db = _dev(torch, b)
    c = torch.full((a.nrow, n), float("nan"), dtype=torch.float32, device="cuda:0")
    print(f"bell M={a.nrow} K={a.ncol} N={n} bs={bs} ell_blocks={colind.shape[1]} nnz={a.nnz}", flush=True)
    S.bell_spmm(dc, dv, a.nrow, a.ncol, n, bs, a.dtype, db, c)
    torch.cuda.synchronize()
    return c.cpu().numpy()


@pytest.mark.parametrize("bs", [32, 64])
@pytest.mark.parametrize("dtype", [S.TCA_F16, S.TCA_BF16])
def test_bell_exact_bit_equal(torch_cuda, dtype, bs):
    rng = np.random.default_rng(5 + dtype + bs)
    for m, k, p in [(128, 256, 0.02), (100, 70, 0.1), (257, 1000, 0.005), (64, 64, 0.6), (33, 5, 0.3)]:
        a = _csr(rng, m, k, p, dtype, empty_rows=range(0, m, 7))
        for n in (8, 64, 256, 264, 512):
            b = S.to_storage(exact_dense(rng, (k, n)), dtype)
            got = _run(torch_cuda, a, b, bs)
            want = oracle.csr_spmm(a.rowptr, a.colidx, a.values_f32(), S.from_storage(b, dtype))
            assert np.array_equal(got, want), (m, k, p, n, bs, np.abs(got - want).max())


@pytest.mark.parametrize("bs", [32, 64])
def test_bell_random_values_within_tolerance(torch_cuda, bs):
    rng = np.random.default_rng(17 + bs)
    a = _csr(rng, 2048, 2048, 0.01, S.TCA_F16, exact=False)
    b = S.to_storage(rng.uniform(-1, 1, (2048, 256)).astype(np.float32), S.TCA_F16)
    got = _run(torch_cuda, a, b, bs)
    assert_parity(a, b, got, f"bell bs={bs}")


def test_bell_block_row_without_blocks_is_zero(torch_cuda):
    rng = np.random.default_rng(3)
    a = _csr(rng, 96, 128, 0.1, S.TCA_F16, empty_rows=range(32, 64))
    b = S.to_storage(exact_dense(rng, (128, 64)), S.TCA_F16)
    got = _run(torch_cuda, a, b, 32)
    assert np.all(got[32:64] == 0.0)
    assert np.array_equal(got, oracle.csr_spmm(a.rowptr, a.colidx, a.values_f32(), S.from_storage(b, S.TCA_F16)))
