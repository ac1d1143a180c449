"""Blocked-ELL: the oracle's restatement of the reference conversion
(src/spmm_cusparse.cu:201-342) pinned by brute force and round trips, the
library's conversion (tca_csr_to_bell) against it, and the argument checks
of tca_bell_spmm that run before any device work.  GPU parity of the
Blocked-ELL kernel is in test_gpu_bell.py."""
import numpy as np
import pytest

from oracle import oracle

import spmm_amd as S


def _dense(rng, m, k, p, zero_block_rows=()):
    d = np.where(rng.random((m, k)) < p, rng.standard_normal((m, k)), 0.0).astype(np.float16)
    for i in zero_block_rows:
        d[i] = 0
    return d


@pytest.mark.parametrize("m,k,bs", [(64, 64, 32), (100, 70, 32), (33, 200, 32), (130, 129, 64), (5, 3, 32)])
def test_oracle_bell_round_trip_and_brute_force(m, k, bs):
    rng = np.random.default_rng(m * 1000 + k)
    d = _dense(rng, m, k, 0.03)
    colind, vals = oracle.dense_to_bell(d, bs)
    brows, bcols = -(-m // bs), -(-k // bs)
    assert colind.shape[0] == brows and vals.shape == (brows * bs, colind.shape[1] * bs)
    # brute force: block (i, j) is listed iff it holds a nonzero value
    pad = np.zeros((brows * bs, bcols * bs), np.float16)
    pad[:m, :k] = d
    for i in range(brows):
        want = [j for j in range(bcols) if np.any(pad[i * bs:(i + 1) * bs, j * bs:(j + 1) * bs] != 0)]
        got = [int(x) for x in colind[i] if x >= 0]
        assert got == want
        assert np.all(colind[i, len(want):] == -1)  # padding only after the list
    assert colind.shape[1] == max([int(np.sum(colind[i] >= 0)) for i in range(brows)] + [0])
    back = oracle.bell_to_dense(colind, vals, bs, k)
    assert np.array_equal(back[:m], d) and not np.any(back[m:])


def test_oracle_bell_hand_built():
    # 4 x 4 with bsize 2: blocks (0,1) and (1,0) hold values; block row 1's
    # (1,1) block holds only a zero; a third block row of zeros.
    d = np.zeros((6, 4), np.float16)
    d[0, 3] = 1.0
    d[3, 0] = 2.0
    d[2, 1] = -0.5
    colind, vals = oracle.dense_to_bell(d, 2)
    assert colind.tolist() == [[1], [0], [-1]]
    assert vals.shape == (6, 2)
    assert vals[0, 1] == 1.0 and vals[3, 0] == 2.0 and vals[2, 1] == -0.5
    assert np.count_nonzero(vals) == 3


@pytest.mark.parametrize("dtype", [S.TCA_F16, S.TCA_BF16, S.TCA_F32])
@pytest.mark.parametrize("m,k,p,bs", [(256, 300, 0.02, 32), (97, 1000, 0.01, 64), (64, 64, 0.5, 32),
                                      (300, 40, 0.05, 64), (1, 1, 1.0, 32)])
def test_library_conversion_matches_oracle(dtype, m, k, p, bs):
    a, _ = S.gen_bernoulli(m, k, p, seed=m + k, dtype=dtype)
    colind, vals = S.csr_to_bell(a, bs)
    dense = S.csr_to_dense(a)
    ocol, ovals = oracle.dense_to_bell(dense, bs)
    assert np.array_equal(colind, ocol)
    assert vals.dtype == ovals.dtype and np.array_equal(vals.view(np.uint8), ovals.view(np.uint8))


def test_library_conversion_drops_zero_valued_entries():
    """An explicit zero in the CSR is not a nonzero value (the reference
    counts values != 0): a block holding only zeros is not listed."""
    rowptr = np.array([0, 2, 2, 3], np.int32)
    colidx = np.array([0, 40, 5], np.int32)
    vals = S.to_storage(np.array([1.0, 0.0, -0.0], np.float32), S.TCA_F16)
    a = S.CSR(3, 64, rowptr, colidx, vals, S.TCA_F16)
    colind, ev = S.csr_to_bell(a, 32)
    assert colind.tolist() == [[0]]
    assert ev.shape == (32, 32)


def test_library_conversion_rejects_bad_input():
    a, _ = S.gen_bernoulli(10, 10, 0.3, seed=1, dtype=S.TCA_F16)
    with pytest.raises(S.TcaError):
        S.csr_to_bell(a, 0)
    bad = S.CSR(a.nrow, a.ncol, a.rowptr, a.colidx.copy(), a.values, a.dtype)
    bad.colidx[0] = a.ncol  # out of range
    with pytest.raises(S.TcaError):
        S.csr_to_bell(bad, 32)


@pytest.mark.parametrize("kw,status", [(dict(bsize=16), 4), (dict(bsize=48), 4), (dict(n=12), 4),
                                       (dict(dtype=S.TCA_F32), 4), (dict(n=0), 1), (dict(k=0), 1),
                                       (dict(ell_blocks=-1), 1)])
def test_bell_spmm_argument_checks(kw, status):
    """These checks precede any device call, so they run without a GPU."""
    args = dict(m=64, k=64, n=64, bsize=32, ell_blocks=1, dtype=S.TCA_F16)
    args.update(kw)
    with pytest.raises(S.TcaError) as ei:
        S._lib.call("tca_bell_spmm", None, None, args["m"], args["k"], args["n"], args["bsize"],
                    args["ell_blocks"], args["dtype"], None, None, None)
    assert ei.value.status == status
