"""2:4 structured sparsity: the oracle's restatement of the STRIP pruning
rule (src/spmm_cusparse.cu:83-84) pinned by brute force, the library's
pruning and compression (tca_prune_24, tca_csr_to_24) against it, the index
word layout on hand-built rows, and the argument checks of tca_spmm_24 that
run before any device work.  GPU parity is in test_gpu_sparse24.py."""
import itertools

import numpy as np
import pytest

from oracle import oracle

import spmm_amd as S


def _brute_prune(dense):
    out = np.zeros_like(dense)
    for r in range(dense.shape[0]):
        for g0 in range(0, dense.shape[1], 4):
            grp = np.abs(dense[r, g0:g0 + 4].astype(np.float64))
            best = None
            for pair in itertools.combinations(range(len(grp)), min(2, len(grp))):
                score = sum(grp[i] for i in pair)
                if best is None or score > best[0]:
                    best = (score, pair)  # combinations come lexicographically: first max = lowest columns
            for i in best[1]:
                if grp[i] != 0:
                    out[r, g0 + i] = dense[r, g0 + i]
    return out


@pytest.mark.parametrize("m,k,p", [(16, 16, 0.9), (40, 37, 0.5), (7, 130, 0.3)])
def test_oracle_prune_matches_brute_force(m, k, p):
    rng = np.random.default_rng(m + k)
    d = np.where(rng.random((m, k)) < p, rng.integers(-3, 4, (m, k)), 0).astype(np.float16)  # many ties
    got = oracle.prune_24(d)
    assert np.array_equal(got, _brute_prune(d))
    for r in range(m):
        for g0 in range(0, k, 4):
            assert np.count_nonzero(got[r, g0:g0 + 4]) <= 2


@pytest.mark.parametrize("dtype", [S.TCA_F16, S.TCA_BF16])
@pytest.mark.parametrize("m,k,p", [(64, 64, 0.5), (100, 200, 0.9), (33, 70, 0.1), (5, 1000, 0.02)])
def test_library_prune_and_compress_match_oracle(dtype, m, k, p):
    a, _ = S.gen_bernoulli(m, k, p, seed=m * k, dtype=dtype)
    pa = S.prune_24(a)
    dense = S.from_storage(S.csr_to_dense(a), dtype)  # exact fp32 values
    want = oracle.prune_24(dense)
    assert np.array_equal(S.from_storage(S.csr_to_dense(pa), dtype), want)
    vals, meta = S.csr_to_24(pa)
    assert vals.shape == (m, (k + 63) // 64 * 32) and meta.shape == (m, (k + 63) // 64 * 4)
    back = oracle.decompress_24(S.from_storage(vals, dtype), meta, k)
    assert np.array_equal(back, want)
    # positions inside each group are ascending and distinct
    for w in np.unique(meta):
        for g in range(4):
            assert ((int(w) >> (4 * g)) & 3) < ((int(w) >> (4 * g + 2)) & 3)


def test_compress_index_words_hand_built():
    # row 0: cols 1, 3 (group 0), col 4 (group 1), col 19 (word 1, group 0);
    # row 1: col 63 (word 3, group 3) alone at position 3
    rowptr = np.array([0, 4, 5], np.int32)
    colidx = np.array([1, 3, 4, 19, 63], np.int32)
    v = S.to_storage(np.array([1.0, 2.0, 3.0, 4.0, 5.0], np.float32), S.TCA_F16)
    a = S.CSR(2, 64, rowptr, colidx, v, S.TCA_F16)
    vals, meta = S.csr_to_24(a)
    f = vals.view(np.float16).astype(np.float32)
    # group 0: positions (1, 3); group 1: position 0 with a zero at 1; others (0, 1) zeros
    assert meta[0, 0] == (1 | 3 << 2) | (0 | 1 << 2) << 4 | 0x4 << 8 | 0x4 << 12
    assert f[0, :4].tolist() == [1.0, 2.0, 3.0, 0.0]
    # word 1 covers columns 16..31: col 19 is group 0, position 3 -> pair (2, 3), value second
    assert meta[0, 1] & 0xf == (2 | 3 << 2) and f[0, 8:10].tolist() == [0.0, 4.0]
    # row 1: col 63 = word 3, group 3, position 3 -> pair (2, 3)
    assert (meta[1, 3] >> 12) & 0xf == (2 | 3 << 2) and f[1, 8 * 3 + 6:8 * 3 + 8].tolist() == [0.0, 5.0]


def test_compress_rejects_three_in_a_group():
    a = S.CSR(1, 8, np.array([0, 3], np.int32), np.array([0, 1, 2], np.int32),
              S.to_storage(np.ones(3, np.float32), S.TCA_F16), S.TCA_F16)
    with pytest.raises(S.TcaError):
        S.csr_to_24(a)
    assert S.prune_24(a).nnz == 2


@pytest.mark.parametrize("kw,status", [(dict(n=12), 4), (dict(dtype=S.TCA_F32), 4), (dict(k=0), 1), (dict(n=0), 1)])
def test_spmm_24_argument_checks(kw, status):
    args = dict(m=64, k=64, n=64, dtype=S.TCA_F16)
    args.update(kw)
    with pytest.raises(S.TcaError) as ei:
        S._lib.call("tca_spmm_24", None, None, args["m"], args["k"], args["n"], args["dtype"], None, None, None)
    assert ei.value.status == status
