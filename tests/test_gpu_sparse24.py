"""GPU parity of the 2:4 sparse-MFMA kernel (tca_spmm_24) against the CPU
oracle on the pruned matrix: bit-exact on exact-arithmetic inputs, within
the reference verdict and a 1e-3 relative bar elsewhere; fp16 / bf16, K not
a multiple of 64, ragged M and N, rows without entries."""
import numpy as np
import pytest

from conftest import exact_dense, exact_values
from oracle import oracle
from test_gpu_parity import _dev, assert_parity

import spmm_amd as S

pytestmark = pytest.mark.gpu


def _pruned(rng, m, k, p, dtype, exact=True):
    a, _ = S.gen_bernoulli(m, k, p, seed=int(rng.integers(1 << 30)), dtype=dtype)
    v = exact_values(rng, a.nnz) if exact else (rng.standard_normal(a.nnz) * 0.02).astype(np.float32)
    v[v == 0] = 0.5
    a = S.CSR(a.nrow, a.ncol, a.rowptr, a.colidx, S.to_storage(v, dtype), dtype)
    return S.prune_24(a)


def _run(torch, a, b):
    vals, meta = S.csr_to_24(a)
    n = b.shape[1]
    c = torch.full((a.nrow, n), float("nan"), dtype=torch.float32, device="cuda:0")
    print(f"2:4 M={a.nrow} K={a.ncol} N={n} nnz={a.nnz}", flush=True)
    S.spmm_24(_dev(torch, vals), _dev(torch, meta), a.nrow, a.ncol, n, a.dtype, _dev(torch, b), c)
    torch.cuda.synchronize()
    return c.cpu().numpy()


@pytest.mark.parametrize("dtype", [S.TCA_F16, S.TCA_BF16])
def test_spmm_24_exact_bit_equal(torch_cuda, dtype):
    rng = np.random.default_rng(31 + dtype)
    for m, k, p in [(64, 64, 0.5), (100, 200, 0.3), (17, 1000, 0.05), (256, 130, 0.9), (1, 64, 1.0)]:
        a = _pruned(rng, m, k, p, dtype)
        for n in (8, 64, 256, 264):
            b = S.to_storage(exact_dense(rng, (k, n)), dtype)
            got = _run(torch_cuda, a, b)
            want = oracle.csr_spmm(a.rowptr, a.colidx, a.values_f32(), S.from_storage(b, dtype))
            assert np.array_equal(got, want), (m, k, p, n, np.abs(got - want).max())


def test_spmm_24_random_values_within_tolerance(torch_cuda):
    rng = np.random.default_rng(47)
    a = _pruned(rng, 2048, 2048, 0.4, S.TCA_F16, exact=False)
    b = S.to_storage(rng.uniform(-1, 1, (2048, 512)).astype(np.float32), S.TCA_F16)
    got = _run(torch_cuda, a, b)
    assert_parity(a, b, got, "2:4 2048x2048")
