"""Pins the CPU oracle (oracle/) against what fixes it independently of its
own code: the reference fixture's known answers, exact-arithmetic closed
forms, scipy fixtures, brute force, and deliberately planted mistakes that
the pins must catch."""
import json
import os
import re

import numpy as np
import pytest

from conftest import FIXTURE_SMTX, GOLDEN, exact_dense, exact_values
from oracle import oracle


# ------------------------------------------------------------ fixture parse
def test_fixture_known_answers(fixture_text):
    nrow, ncol, nnz, rowptr, colidx = oracle.parse_smtx(fixture_text)
    # Header line of data/body_decoder_layer_2_ffn_conv1.smtx
    assert (nrow, ncol, nnz) == (2048, 512, 1005)
    assert len(rowptr) == 2049 and rowptr[0] == 0 and rowptr[-1] == 1005
    assert len(colidx) == 1005
    assert colidx.min() == 2 and colidx.max() == 511
    lens = np.diff(rowptr)
    assert (lens == 0).sum() == 2020
    assert lens.max() == 65
    # row-length buckets of the reference's warp split (src/our_spmm.cu:372-391)
    assert ((lens > 0) & (lens <= 8)).sum() == 0
    assert ((lens > 8) & (lens <= 16)).sum() == 1
    assert ((lens > 16) & (lens <= 32)).sum() == 9
    assert ((lens > 32) & (lens <= 64)).sum() == 17
    assert (lens > 64).sum() == 1
    for r in range(nrow):  # columns strictly ascending inside each row
        seg = colidx[rowptr[r]:rowptr[r + 1]]
        assert np.all(np.diff(seg) > 0)


def test_fixture_parse_independent_tokeniser(fixture_text):
    """A regex tokeniser (no split logic shared with parse_smtx) agrees."""
    nrow, ncol, nnz, rowptr, colidx = oracle.parse_smtx(fixture_text)
    lines = fixture_text.splitlines()
    head = [int(x) for x in re.findall(r"-?\d+", lines[0])]
    assert head == [nrow, ncol, nnz]
    assert [int(x) for x in re.findall(r"-?\d+", lines[1])] == rowptr.tolist()
    assert [int(x) for x in re.findall(r"-?\d+", " ".join(lines[2:]))] == colidx.tolist()


def test_fixture_dense_round_trip(fixture_text):
    """.smtx -> dense -> CSR reproduces the file's arrays (sorted, unique)."""
    nrow, ncol, nnz, rowptr, colidx = oracle.parse_smtx(fixture_text)
    d = oracle.smtx_to_dense(nrow, ncol, rowptr, colidx)
    assert d.dtype == np.float16 and d.sum(dtype=np.float64) == nnz
    rp, ci, v = oracle.dense_to_csr(d)
    assert np.array_equal(rp, rowptr) and np.array_equal(ci, colidx)
    assert np.all(v == 1.0)
    assert np.array_equal(oracle.csr_to_dense(rp, ci, v, ncol), d)


# ------------------------------------------------------- dense <-> CSR
def test_dense_to_csr_drops_signed_zeros_and_orders():
    d = np.array([[0.0, -0.0, 1.5, 0.0], [2.0, 0.0, 0.0, -3.0], [0.0, 0.0, 0.0, 0.0]], np.float16)
    rp, ci, v = oracle.dense_to_csr(d)
    assert rp.tolist() == [0, 1, 3, 3]
    assert ci.tolist() == [2, 0, 3]
    assert v.tolist() == [1.5, 2.0, -3.0]


def test_dense_csr_identity_random():
    rng = np.random.default_rng(7)
    d = rng.standard_normal((37, 53)).astype(np.float32)
    d[rng.random(d.shape) < 0.8] = 0.0
    d[0, 0] = -0.0
    rp, ci, v = oracle.dense_to_csr(d)
    assert np.array_equal(oracle.csr_to_dense(rp, ci, v, 53), np.where(d == 0, 0, d))
    # brute-force count of nonzeros per row
    assert np.array_equal(np.diff(rp), (d != 0).sum(1))


# --------------------------------------------------------------- SpMM
def _rand_csr(rng, m, k, p, values):
    mask = rng.random((m, k)) < p
    rows, cols = np.nonzero(mask)
    rp = np.zeros(m + 1, np.int32)
    np.cumsum(np.bincount(rows, minlength=m), out=rp[1:])
    return rp, cols.astype(np.int32), values(len(rows))


def test_spmm_exact_vectors_bit_equal():
    """A in {+-1,+-1/2,+-2}, B in {k/256}: every partial sum is exact in fp32,
    so the result is bit-equal to the fp64 product whatever the order."""
    rng = np.random.default_rng(1)
    for m, k, n, p in [(64, 48, 32, 0.3), (200, 300, 17, 0.05), (5, 1000, 8, 0.9)]:
        rp, ci, v = _rand_csr(rng, m, k, p, lambda c: exact_values(rng, c))
        b = exact_dense(rng, (k, n))
        dense = oracle.csr_to_dense(rp, ci, v.astype(np.float64), k)
        want = dense @ b.astype(np.float64)
        got = oracle.csr_spmm(rp, ci, v, b)
        assert np.array_equal(got, want.astype(np.float32))
        assert np.array_equal(got.astype(np.float64), want)


def test_spmm_closed_forms():
    rng = np.random.default_rng(2)
    k, n = 50, 12
    b = rng.standard_normal((k, n)).astype(np.float32)
    # identity: C = B
    rp = np.arange(k + 1, dtype=np.int32)
    ci = np.arange(k, dtype=np.int32)
    assert np.array_equal(oracle.csr_spmm(rp, ci, np.ones(k, np.float32), b), b)
    # permutation: C = B[perm]
    perm = rng.permutation(k).astype(np.int32)
    assert np.array_equal(oracle.csr_spmm(rp, perm, np.ones(k, np.float32), b), b[perm])
    # one all-ones row: C = column sums (exact inputs keep the sum exact)
    be = exact_dense(rng, (k, n))
    c = oracle.csr_spmm(np.array([0, k], np.int32), np.arange(k, dtype=np.int32), np.ones(k, np.float32), be)
    assert np.array_equal(c[0], be.astype(np.float64).sum(0).astype(np.float32))
    # empty rows produce zeros (beta = 0)
    c = oracle.csr_spmm(np.array([0, 0, 0], np.int32), np.zeros(0, np.int32), np.zeros(0, np.float32), b)
    assert np.array_equal(c, np.zeros((2, n), np.float32))


def test_spmm_matches_dense_naive_gemm():
    """CSR oracle == literal naive_gemm restatement (skipped terms are +-0)."""
    rng = np.random.default_rng(3)
    rp, ci, v = _rand_csr(rng, 40, 70, 0.2, lambda c: rng.standard_normal(c).astype(np.float32))
    b = rng.standard_normal((70, 24)).astype(np.float32)
    dense = oracle.csr_to_dense(rp, ci, v, 70)
    assert np.array_equal(oracle.csr_spmm(rp, ci, v, b), oracle.dense_spmm(dense, b))


def test_spmm_scipy_fixtures():
    """scipy.sparse csr @ B results committed under tests/golden/."""
    data = np.load(os.path.join(GOLDEN, "scipy_spmm.npz"))
    names = sorted({k.split("__")[0] for k in data.files})
    assert names
    for nm in names:
        rp, ci, v, b, c = (data[f"{nm}__{x}"] for x in ("rowptr", "colidx", "values", "b", "c"))
        got = oracle.csr_spmm(rp, ci, v.astype(np.float32), b.astype(np.float32))
        np.testing.assert_allclose(got, c, rtol=1e-5, atol=1e-5)


def test_spmm_tiny_brute_force():
    rng = np.random.default_rng(4)
    for _ in range(20):
        m, k, n = rng.integers(1, 6, 3)
        rp, ci, v = _rand_csr(rng, m, k, 0.5, lambda c: rng.standard_normal(c).astype(np.float32))
        b = rng.standard_normal((k, n)).astype(np.float32)
        want = np.zeros((m, n))
        for r in range(m):
            for j in range(rp[r], rp[r + 1]):
                for col in range(n):
                    want[r, col] += float(v[j]) * float(b[ci[j], col])
        np.testing.assert_allclose(oracle.csr_spmm_f64(rp, ci, v, b), want, rtol=1e-12, atol=1e-12)
        np.testing.assert_allclose(oracle.csr_spmm(rp, ci, v, b), want, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("mistake", ["dropped_term", "wrong_index", "transposed", "sign"])
def test_pins_catch_planted_mistakes(mistake):
    """Each plausible mistake, planted in a copy of the oracle's formula,
    fails the exact-vector pin above."""
    rng = np.random.default_rng(5)
    m = k = 24
    n = 24
    rp, ci, v = _rand_csr(rng, m, k, 0.3, lambda c: exact_values(rng, c))
    b = exact_dense(rng, (k, n))
    want = (oracle.csr_to_dense(rp, ci, v.astype(np.float64), k) @ b.astype(np.float64)).astype(np.float32)

    def wrong():
        c = np.zeros((m, n), np.float32)
        for r in range(m):
            js = list(range(rp[r], rp[r + 1]))
            if mistake == "dropped_term" and js:
                js = js[:-1]
            for j in js:
                col = ci[j] + 1 if mistake == "wrong_index" else ci[j]
                col %= k
                row_b = b[:, col] if mistake == "transposed" else b[col]
                a = -v[j] if (mistake == "sign" and j == rp[r]) else v[j]
                c[r] += np.float32(a) * row_b
        return c

    assert np.array_equal(oracle.csr_spmm(rp, ci, v, b), want)
    assert not np.array_equal(wrong(), want)


# ------------------------------------------------------------ verdict
def test_compare_mat_branches():
    tol = 1e-3
    g = np.array([1.0, 1.0, 0.0, 1e-4, 100.0, 0.0], np.float32)
    # 0: equal; 1: rel 2e-3 & abs 2e-3 -> fail; 2: g = 0, c = 0 -> pass (rel nan);
    # 3: abs tiny -> pass; 4: rel 5e-6 -> pass; 5: g = 0, c = 0.01 -> rel inf, abs 1e-2 -> fail
    c = np.array([1.0, 1.002, 0.0, 5e-4, 100.0005, 0.01], np.float32)
    ok, fc, ff, mr = oracle.compare_mat(g, c, tol)
    assert not ok and fc == 2 and ff == 1
    ok, fc, ff, mr = oracle.compare_mat(g[[0, 2, 3, 4]], c[[0, 2, 3, 4]], tol)
    assert ok and fc == 0 and ff == -1
    # the scan stops at the 10th failure
    ok, fc, ff, _ = oracle.compare_mat(np.ones(50, np.float32), np.full(50, 2.0, np.float32), tol)
    assert not ok and fc == 10 and ff == 0


# ---------------------------------------------------- condensed windows
def test_condense_windows_reconstruct_and_brute_force():
    rng = np.random.default_rng(6)
    for m, k, p, win in [(64, 100, 0.1, 16), (37, 20, 0.5, 16), (10, 1000, 0.01, 4), (33, 33, 0.0, 16)]:
        rp, ci, v = _rand_csr(rng, m, k, p, lambda c: rng.standard_normal(c).astype(np.float32))
        uoff, ucols, cpos = oracle.condense_windows(rp, ci, m, win)
        nw = (m + win - 1) // win
        assert len(uoff) == nw + 1
        dense = oracle.csr_to_dense(rp, ci, v, k)
        for w in range(nw):
            r0, r1 = w * win, min(m, (w + 1) * win)
            u = ucols[uoff[w]:uoff[w + 1]]
            # brute force: the union is the set of columns with any nonzero
            assert u.tolist() == [c for c in range(k) if np.any(dense[r0:r1, c] != 0)]
            # scatter the condensed tile back through the union: the dense window
            tile = np.zeros((r1 - r0, len(u)), np.float32)
            for r in range(r0, r1):
                for j in range(rp[r], rp[r + 1]):
                    tile[r - r0, cpos[j]] = v[j]
            back = np.zeros((r1 - r0, k), np.float32)
            back[:, u] = tile
            assert np.array_equal(back, dense[r0:r1])


def test_golden_manifest_lists_fixtures():
    with open(os.path.join(GOLDEN, "MANIFEST.json")) as f:
        man = json.load(f)
    for name in man["files"]:
        assert os.path.exists(os.path.join(GOLDEN, name)), name
    assert os.path.basename(FIXTURE_SMTX) in man["files"]


# ------------------------------------------------ MatrixMarket readers
def _mm_text(rng, m, k, n, one_based=True, banner=True, dup=0, values=True):
    r = rng.integers(0, m, n)
    c = rng.integers(0, k, n)
    if dup:
        r = np.concatenate([r, r[:dup]])
        c = np.concatenate([c, c[:dup]])
    v = np.round(rng.uniform(-4, 4, len(r)), 3)
    lines = ["%%MatrixMarket matrix coordinate real general"] if banner else []
    lines += ["% comment", f"{m} {k} {len(r)}"]
    off = 1 if one_based else 0
    for i in range(len(r)):
        lines.append(f"{r[i] + off} {c[i] + off} {v[i]:g}" if values else f"{r[i] + off} {c[i] + off}")
    return "\n".join(lines) + "\n", r, c, v


def test_parse_mtx_entries_match_scipy_mmread():
    """The oracle's entries, in file order, equal scipy.io.mmread's (an
    independent MatrixMarket parser that keeps file order), duplicates included."""
    import io
    import scipy.io
    rng = np.random.default_rng(3)
    for m, k, n, dup in [(20, 30, 50, 0), (5, 5, 20, 6), (1, 40, 10, 2)]:
        text, _, _, _ = _mm_text(rng, m, k, n, dup=dup)
        rows, cols, ents = oracle.parse_mtx(text, zero_based=False, read_value=True, missing=0.0)
        mm = scipy.io.mmread(io.BytesIO(text.encode()))
        assert (rows, cols) == mm.shape
        assert [e[0] for e in ents] == mm.row.tolist() and [e[1] for e in ents] == mm.col.tolist()
        assert np.array_equal(np.array([e[2] for e in ents], np.float32), mm.data.astype(np.float32))


def test_mtx_oracle_csr_and_dense_match_scipy_on_unique_entries():
    """Unique entries: the file-order CSR, scattered to dense, and the dense
    reader both equal scipy's dense form of the file."""
    import io
    import scipy.io
    rng = np.random.default_rng(4)
    text, r, c, v = _mm_text(rng, 40, 25, 400)
    keep = {}
    for i in range(len(r)):
        keep.setdefault((r[i], c[i]), i)
    lines = text.splitlines()
    body = [lines[3 + i] for i in sorted(keep.values())]
    text = "\n".join(lines[:2] + [f"40 25 {len(body)}"] + body) + "\n"
    want = scipy.io.mmread(io.BytesIO(text.encode())).toarray().astype(np.float32)
    m, k, rp, ci, vals = oracle.mtx_to_csr_file_order(text, pattern_only=False, zero_based=False)
    assert np.array_equal(oracle.csr_to_dense(rp, ci, vals, k), want)
    assert np.array_equal(oracle.mtx_to_dense(text, zero_based=False), want)


def test_mtx_oracle_known_answers():
    """What scipy does not fix: each row's entries in file order, duplicates
    kept by the CSR reader and the last one winning in the dense reader, a
    missing value read as 0 (CSR) or 1 (dense, pattern), zero-based indices."""
    text = "%c\n3 4 6\n2 3 1.5\n1 4 2\n2 1 -1\n3 2 0.25\n1 1 7\n2 3 5\n"
    m, k, rp, ci, v = oracle.mtx_to_csr_file_order(text, pattern_only=False, zero_based=False)
    assert (m, k) == (3, 4)
    assert rp.tolist() == [0, 2, 5, 6]
    assert ci.tolist() == [3, 0, 2, 0, 2, 1]
    assert v.tolist() == [2.0, 7.0, 1.5, -1.0, 5.0, 0.25]
    d = oracle.mtx_to_dense(text, zero_based=False)
    assert d[1, 2] == 5.0 and d[0, 0] == 7.0 and d[2, 1] == 0.25 and np.count_nonzero(d) == 5
    pat = "2 2 2\n0 1\n1 0 3.5\n"
    _, _, rp, ci, v = oracle.mtx_to_csr_file_order(pat, pattern_only=True, zero_based=True)
    assert rp.tolist() == [0, 1, 2] and ci.tolist() == [1, 0] and v.tolist() == [1.0, 1.0]
    _, _, _, _, v = oracle.mtx_to_csr_file_order(pat, pattern_only=False, zero_based=True)
    assert v.tolist() == [0.0, 3.5]
    assert oracle.mtx_to_dense(pat, zero_based=True).tolist() == [[0.0, 1.0], [3.5, 0.0]]
