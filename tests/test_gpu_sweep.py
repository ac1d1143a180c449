"""A seeded sweep over the routing choices a plan can make: structure
generators (uniform, lognormal rows, R-MAT, Zipf rows, dense-column blocks),
value types, widths N (including ones no vector path covers) and plan flags
(default, no matrix cores, no panels, forced panels, forced matrix-core
tiles of each kind, short-K, no scratch).  Every case is bit-exact against
the oracle on exact-arithmetic inputs and identical on a second run; plans
that keep no scratch run through the allocation-free entry point.  Each
case's parameters and plan are printed before it runs."""
import numpy as np
import pytest

from conftest import exact_dense, exact_values
from oracle import oracle

import spmm_amd as S
from test_gpu_parity import _dev

pytestmark = pytest.mark.gpu

FLAGS_ANY = [S.TCA_PLAN_DEFAULT, S.TCA_PLAN_NO_MFMA, S.TCA_PLAN_NO_PANELS, S.TCA_PLAN_FORCE_PANELS,
             S.TCA_PLAN_FORCE_PANELS | S.TCA_PLAN_NO_MFMA, S.TCA_PLAN_NO_SCRATCH,
             S.TCA_PLAN_FORCE_PANELS | S.TCA_PLAN_NO_SCRATCH]
FLAGS_HALF = [S.TCA_PLAN_FORCE_MFMA, S.TCA_PLAN_MFMA_DENSE, S.TCA_PLAN_MFMA_COMPACT, S.TCA_PLAN_MFMA_PAIR,
              S.TCA_PLAN_MFMA_SHORT, S.TCA_PLAN_FORCE_MFMA | S.TCA_PLAN_FORCE_PANELS]
# widths the panel and matrix-core geometries take (multiples of 64) drawn
# more often than those only the row kernel covers
WIDTHS = [64, 128, 256, 64, 128, 256, 1, 3, 8, 16, 24, 32, 96, 200]


def _structure(rng, kind):
    seed = int(rng.integers(1, 1 << 30))
    if kind == "bernoulli":
        m, k = int(rng.integers(1, 2500)), int(rng.integers(1, 4000))
        return S.gen_bernoulli(m, k, float(rng.choice([0.001, 0.01, 0.05])), seed=seed, dtype=S.TCA_F32)[0]
    if kind == "lognormal":
        m, k = int(rng.integers(50, 2500)), int(rng.integers(200, 5000))
        return S.gen_lognormal_rows(m, k, float(rng.choice([5, 30, 120])), seed=seed, dtype=S.TCA_F32)[0]
    if kind == "rmat":
        n = int(rng.integers(500, 8000))
        return S.gen_rmat(13, n, int(rng.integers(5000, 120000)), norm=int(rng.integers(0, 3)), seed=seed)[0]
    if kind == "zipf":
        m = int(rng.integers(200, 4000))
        return S.gen_zipf_rows(m, int(rng.integers(500, 6000)), int(rng.integers(2000, 150000)), cap=5000, seed=seed,
                               dtype=S.TCA_F32)[0]
    # dense-column block: rows sharing few columns (panel tiles, matrix-core windows)
    m, k = int(rng.integers(100, 1200)), int(rng.integers(40, 700))
    return S.gen_bernoulli(m, k, float(rng.choice([0.2, 0.4])), seed=seed, dtype=S.TCA_F32)[0]


def _cases(n_cases=48, seed=2026):
    rng = np.random.default_rng(seed)
    kinds = ["bernoulli", "lognormal", "rmat", "zipf", "dense-cols"]
    for c in range(n_cases):
        kind = kinds[c % len(kinds)]
        dtype = [S.TCA_F32, S.TCA_F16, S.TCA_BF16][int(rng.integers(0, 3))]
        flags = FLAGS_ANY + (FLAGS_HALF if dtype != S.TCA_F32 else [])
        yield c, kind, dtype, int(rng.choice(WIDTHS)), int(flags[int(rng.integers(0, len(flags)))]), int(rng.integers(1, 1 << 30))


CASES = list(_cases())


@pytest.mark.parametrize("case,kind,dtype,n,flags,seed", CASES, ids=[f"case{c[0]}-{c[1]}" for c in CASES])
def test_routing_sweep_bit_exact(torch_cuda, case, kind, dtype, n, flags, seed):
    torch = torch_cuda
    rng = np.random.default_rng(seed)
    base = _structure(rng, kind)
    vals = exact_values(rng, base.nnz)
    a = S.CSR(base.nrow, base.ncol, base.rowptr, base.colidx, S.to_storage(vals, dtype), dtype)
    b = S.to_storage(exact_dense(rng, (a.ncol, n)), dtype)
    print(f"sweep case {case}: {kind} M={a.nrow} K={a.ncol} nnz={a.nnz} N={n} dtype={dtype} flags={flags}",
          flush=True)
    want = oracle.csr_spmm(a.rowptr, a.colidx, a.values_f32(), S.from_storage(b, dtype))
    val, bd = _dev(torch, a.values if a.nnz else np.zeros(1, a.values.dtype)), _dev(torch, b)
    with S.Plan(a, n, flags) as pl:
        info = pl.info()
        print(f"  plan: tile kernel {info['tile_kernel']}, {info['n_windows_mfma']} windows, "
              f"{info['n_panels']} panels, {info['n_row_tasks']} row tasks, {info['n_long_rows']} long rows",
              flush=True)
        outs = []
        for _ in range(2):
            c = torch.full((a.nrow, n), float("nan"), dtype=torch.float32, device="cuda:0")
            if flags & S.TCA_PLAN_NO_SCRATCH:
                pl.run_static(val, bd, c)
            else:
                pl.run(val, bd, c)
            torch.cuda.synchronize()
            outs.append(c.cpu().numpy())
    assert np.array_equal(outs[0], want), (case, np.nanmax(np.abs(outs[0] - want)) if outs[0].size else 0)
    assert np.array_equal(outs[0], outs[1]), case
