"""CPU tests of the product's host library (readers, conversion, verdict,
generators, planner) against the oracle and the reference fixture."""
import os
import subprocess
import sys

import numpy as np
import pytest

from conftest import FIXTURE_SMTX, ROOT
from oracle import oracle

import spmm_amd as S


# ------------------------------------------------------------- readers
def test_smtx_reader_matches_oracle(fixture_text):
    nrow, ncol, nnz, rowptr, colidx = oracle.parse_smtx(fixture_text)
    a = S.read_smtx(FIXTURE_SMTX)
    assert (a.nrow, a.ncol, a.nnz) == (nrow, ncol, nnz)
    assert np.array_equal(a.rowptr, rowptr) and np.array_equal(a.colidx, colidx)
    assert a.values.dtype == np.float16 and np.all(a.values == 1.0)
    a.validate()


def test_smtx_dense_reader_matches_reference_semantics(fixture_text):
    nrow, ncol, nnz, rowptr, colidx = oracle.parse_smtx(fixture_text)
    d = S.read_smtx_dense(FIXTURE_SMTX)
    assert np.array_equal(d, oracle.smtx_to_dense(nrow, ncol, rowptr, colidx))
    # .smtx -> dense -> CSR equals the direct reader
    a = S.dense_to_csr(d, S.TCA_F16)
    b = S.read_smtx(FIXTURE_SMTX)
    assert np.array_equal(a.rowptr, b.rowptr) and np.array_equal(a.colidx, b.colidx)


def test_smtx_write_round_trip_is_byte_identical(tmp_path):
    a = S.read_smtx(FIXTURE_SMTX)
    out = tmp_path / "w.smtx"
    S.write_smtx(str(out), a)
    with open(FIXTURE_SMTX, "rb") as f1, open(out, "rb") as f2:
        assert f1.read() == f2.read()


def test_smtx_reader_sorts_and_dedupes_like_dense_path(tmp_path):
    p = tmp_path / "u.smtx"
    p.write_text("3, 5, 6\n0 3 3 6 \n4 1 1 0 2 4\n")
    a = S.read_smtx(str(p))
    assert a.rowptr.tolist() == [0, 2, 2, 5] and a.colidx.tolist() == [1, 4, 0, 2, 4]
    d = S.read_smtx_dense(str(p))
    b = S.dense_to_csr(d, S.TCA_F16)
    assert np.array_equal(a.rowptr, b.rowptr) and np.array_equal(a.colidx, b.colidx)


@pytest.mark.parametrize("text", [
    "2, 3\n0 1 1\n0\n",                 # short header
    "2, 3, 1\n0 1\n0\n",                # too few row offsets
    "2, 3, 1\n0 1 1 1\n0\n",            # too many row offsets
    "2, 3, 1\n1 1 1\n0\n",              # rowptr[0] != 0
    "2, 3, 2\n0 2 1\n0 1\n",            # decreasing / not ending at nnz
    "2, 3, 1\n0 1 1\n3\n",              # column out of range
    "2, 3, 2\n0 1 2\n0\n",              # too few column indices
    "2, 3, 1\n0 1 1\n0 1\n",            # too many column indices
    "2, 3, 1\n0 x 1\n0\n",              # bad token
])
def test_smtx_reader_rejects_malformed(tmp_path, text):
    p = tmp_path / "bad.smtx"
    p.write_text(text)
    with pytest.raises(S.TcaError) as e:
        S.read_smtx(str(p))
    assert e.value.status == 6  # TCA_ERR_FORMAT


def test_missing_file_is_io_error():
    with pytest.raises(S.TcaError) as e:
        S.read_smtx("/nonexistent/file.smtx")
    assert e.value.status == 5


def test_mtx_reader(tmp_path):
    p = tmp_path / "m.mtx"
    p.write_text("%%MatrixMarket matrix coordinate real general\n% c\n3 4 4\n3 4 2.5\n1 2 1.0\n1 1 -1\n2 3 4\n")
    a = S.read_mtx(str(p), pattern_only=False, zero_based=False, dtype=S.TCA_F32)
    assert a.rowptr.tolist() == [0, 2, 3, 4]
    assert a.colidx.tolist() == [0, 1, 2, 3]
    assert a.values.tolist() == [-1.0, 1.0, 4.0, 2.5]
    b = S.read_mtx(str(p), pattern_only=True, zero_based=False, dtype=S.TCA_F16)
    assert np.all(b.values == 1.0)
    p.write_text("3 4 2\n0 0\n0 0\n")
    with pytest.raises(S.TcaError):
        S.read_mtx(str(p), pattern_only=True, zero_based=True)  # duplicate entry
    p.write_text("3 4 3\n1 1\n")
    with pytest.raises(S.TcaError):
        S.read_mtx(str(p), pattern_only=True)  # count mismatch (reference asserts)


# ---------------------------------------------------------- conversions
def test_f16_conversion_matches_numpy():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    f = S.from_storage(h.view(np.float16), S.TCA_F16)
    ref = h.view(np.float16).astype(np.float32)
    same = (f.view(np.uint32) == ref.view(np.uint32)) | (np.isnan(f) & np.isnan(ref))
    assert same.all()
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(200000).astype(np.float32) * 10.0 ** rng.integers(-9, 6, 200000),
        np.array([65504, 65519.99, 65520, 1e6, -1e6, 2 ** -24, 2 ** -25, 2 ** -25 * 1.0001, 6.0e-8, 0.0, -0.0,
                  np.inf, -np.inf], np.float32),
        (np.arange(-70000, 70000, 0.5, dtype=np.float32)),
    ]).astype(np.float32)
    got = S.to_storage(x, S.TCA_F16)
    assert np.array_equal(got.view(np.uint16), x.astype(np.float16).view(np.uint16))


def _bf16_ref(x):
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(x)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def test_bf16_conversion():
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(100000) * 10.0 ** rng.integers(-30, 30, 100000)).astype(np.float32)
    x = np.concatenate([x, np.array([np.nan, np.inf, -np.inf, 0.0, -0.0, 3.4e38], np.float32)])
    got = S.to_storage(x, S.TCA_BF16)
    assert np.array_equal(got, _bf16_ref(x))
    back = S.from_storage(got, S.TCA_BF16)
    assert np.array_equal(back.view(np.uint32), got.astype(np.uint32) << 16)


def test_dense_to_csr_and_back_match_oracle():
    rng = np.random.default_rng(2)
    d = rng.standard_normal((60, 45)).astype(np.float16)
    d[rng.random(d.shape) < 0.85] = 0
    d[3, 4] = -0.0
    a = S.dense_to_csr(d, S.TCA_F16)
    rp, ci, v = oracle.dense_to_csr(d)
    assert np.array_equal(a.rowptr, rp) and np.array_equal(a.colidx, ci) and np.array_equal(a.values, v)
    assert np.array_equal(S.csr_to_dense(a), np.where(d == 0, np.float16(0), d))


# -------------------------------------------------------------- verdict
def test_compare_mat_matches_oracle():
    rng = np.random.default_rng(3)
    for _ in range(50):
        g = rng.standard_normal(200).astype(np.float32)
        c = g + rng.standard_normal(200).astype(np.float32) * 10.0 ** rng.integers(-6, 0)
        c[rng.random(200) < 0.05] = 0
        g[rng.random(200) < 0.05] = 0
        ours = S.compare_mat(g, c, 1e-3)
        ok, fc, ff, mr = oracle.compare_mat(g, c, 1e-3)
        assert (ours["success"], ours["fail_count"], ours["first_fail"]) == (ok, fc, ff)
        assert ours["max_rel"] == pytest.approx(mr, nan_ok=True)


def test_naive_csr_spmm_bit_equal_to_oracle():
    rng = np.random.default_rng(4)
    a, _ = S.gen_bernoulli(100, 80, 0.2, seed=9, dtype=S.TCA_F16)
    b = S.gen_dense(80, 48, 0, seed=3, dtype=S.TCA_F16)
    got = S.naive_csr_spmm(a, b)
    want = oracle.csr_spmm(a.rowptr, a.colidx, a.values_f32(), b.astype(np.float32))
    assert np.array_equal(got, want)


# ----------------------------------------------------------- generators
def test_generators_deterministic_and_valid():
    a1, st1 = S.gen_bernoulli(256, 128, 0.1, seed=5)
    a2, _ = S.gen_bernoulli(256, 128, 0.1, seed=5)
    a3, _ = S.gen_bernoulli(256, 128, 0.1, seed=6)
    assert np.array_equal(a1.colidx, a2.colidx) and np.array_equal(a1.values, a2.values)
    assert not np.array_equal(a1.rowptr, a3.rowptr)
    a1.validate()
    p = a1.nnz / (256 * 128)
    assert abs(p - 0.1) < 0.01
    v = a1.values_f32()
    assert abs(v.std() - 0.02) < 0.002 and np.all(v != 0)


def test_generators_independent_of_thread_count():
    code = ("import sys; sys.path.insert(0, %r); import spmm_amd as S, hashlib;"
            "a,_=S.gen_lognormal_rows(512, 1024, 60, seed=3); r,_=S.gen_rmat(12, 3000, 40000, seed=3);"
            "z,_=S.gen_zipf_rows(2000, 5000, 40000, cap=3000, seed=3);"
            "print(hashlib.sha1(a.colidx.tobytes()+a.values.tobytes()+r.colidx.tobytes()+r.values.tobytes()"
            "+z.colidx.tobytes()+z.rowptr.tobytes()).hexdigest())") % ROOT
    outs = []
    for t in ("1", "3", "8"):
        env = dict(os.environ, OMP_NUM_THREADS=t)
        outs.append(subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True,
                                   check=True).stdout.strip())
    assert len(set(outs)) == 1, outs


def test_lognormal_rows_stats():
    a, st = S.gen_lognormal_rows(4096, 4096, 205.0, 1.0, seed=1)
    a.validate()
    lens = np.diff(a.rowptr)
    assert 190 < lens.mean() < 215
    # log-lengths ~ N(ln 205 - 0.5, 1)
    ll = np.log(lens[lens > 0])
    assert abs(ll.mean() - (np.log(205) - 0.5)) < 0.06 and abs(ll.std() - 1.0) < 0.06


def test_rmat_small_structure():
    a, st = S.gen_rmat(10, 1000, 20000, norm=0, seed=2)
    a.validate()
    d = S.csr_to_dense(a.astype(S.TCA_F32)).astype(np.float64)
    assert np.allclose(d, d.T)  # symmetric values D^-1/2 (A+I) D^-1/2
    assert np.all(np.diag(d) > 0)  # self-loops
    deg = np.diff(a.rowptr).astype(np.float64)
    r = 5
    cols = a.colidx[a.rowptr[r]:a.rowptr[r + 1]]
    np.testing.assert_allclose(d[r, cols], 1.0 / np.sqrt(deg[r] * deg[cols]), rtol=1e-6)
    m, _ = S.gen_rmat(10, 1000, 20000, norm=1, seed=2)
    lens = np.diff(m.rowptr)
    for r in np.nonzero(lens)[0][:20]:
        assert np.allclose(m.values[m.rowptr[r]:m.rowptr[r + 1]], 1.0 / lens[r])


def test_zipf_rows_total_and_cap():
    z, st = S.gen_zipf_rows(20000, 20000, 400000, s=1.5, cap=15000, seed=4)
    z.validate()
    lens = np.diff(z.rowptr)
    assert z.nnz == 400000 and lens.max() <= 15000 and st["max_row"] == lens.max()


# --------------------------------------------------- condensed windows
@pytest.mark.parametrize("m,k,p,win", [(130, 300, 0.05, 64), (64, 64, 0.5, 16), (37, 1000, 0.01, 4), (20, 20, 0.0, 16)])
def test_condense_windows_bit_exact_with_oracle(m, k, p, win):
    a, _ = S.gen_bernoulli(m, k, p, seed=m + k, dtype=S.TCA_F16)
    uoff, ucols, cpos = S.condense_windows(a, win)
    ou, oc, op = oracle.condense_windows(a.rowptr, a.colidx, m, win)
    assert np.array_equal(uoff, ou) and np.array_equal(ucols, oc) and np.array_equal(cpos, op)


@pytest.mark.parametrize("m,k,n,p,flags", [(200, 700, 128, 0.06, S.TCA_PLAN_FORCE_MFMA | S.TCA_PLAN_MFMA_DENSE),
                                           (130, 300, 64, 0.02, S.TCA_PLAN_FORCE_MFMA | S.TCA_PLAN_MFMA_PAIR),
                                           (64, 2048, 256, 0.3, S.TCA_PLAN_FORCE_MFMA | S.TCA_PLAN_MFMA_DENSE),
                                           (300, 700, 128, 0.06, S.TCA_PLAN_FORCE_MFMA),
                                           (129, 1500, 64, 0.1, S.TCA_PLAN_FORCE_MFMA)])
def test_mfma_window_plan_decodes_to_the_csr(m, k, n, p, flags):
    """Every MFMA window's steps, B-row lists and entries reproduce the CSR
    exactly, with the oracle's condensed positions (128-row windows; the
    dense-tile shape admits any number of entries per step, the paired one at
    most 512)."""
    a, _ = S.gen_bernoulli(m, k, p, seed=7, dtype=S.TCA_F16)
    windows, ucols, eoff, entries = S.plan_mfma_windows(a, n, flags=flags)
    assert len(windows) > 0
    win = 128
    uo, uc, cp = oracle.condense_windows(a.rowptr, a.colidx, m, win)
    for row0, steps, gstep, nz0 in windows:
        w = row0 // win
        assert row0 % win == 0 and nz0 == a.rowptr[row0]
        u = uc[uo[w]:uo[w + 1]]
        assert steps == (len(u) + 31) // 32
        cols = ucols[gstep * 32:(gstep + steps) * 32]
        assert np.array_equal(cols[:len(u)], u) and np.all(cols[len(u):] == -1)
        seen = []
        for s in range(steps):
            for e in entries[eoff[gstep + s]:eoff[gstep + s + 1]]:
                r, kk, rel = int(e) & 127, (int(e) >> 7) & 31, int(e) >> 12
                j = nz0 + rel
                assert a.rowptr[row0 + r] <= j < a.rowptr[row0 + r + 1]
                assert cp[j] == 32 * s + kk and cols[32 * s + kk] == a.colidx[j]
                seen.append(j)
        r1 = min(m, row0 + win)
        assert sorted(seen) == list(range(a.rowptr[row0], a.rowptr[r1]))
    none = S.plan_mfma_windows(a, n, flags=S.TCA_PLAN_NO_MFMA)[0]
    assert len(none) == 0
    assert len(S.plan_mfma_windows(a.astype(S.TCA_F32), n, flags=S.TCA_PLAN_FORCE_MFMA)[0]) == 0  # fp32: no MFMA
    assert len(S.plan_mfma_windows(a, 100, flags=S.TCA_PLAN_FORCE_MFMA)[0]) == 0  # N % 8 != 0


@pytest.mark.parametrize("kernel", [0, S.TCA_PLAN_MFMA_PAIR], ids=["default", "pair"])
def test_mfma_default_routing_follows_the_cost_model(kernel):
    """Default routing of 128-row windows (whatever tile kernel then takes
    them): the lognormal 4096 x 4096 layer
    (config 1) goes to the tile kernel, the small 2048 x 512 Bernoulli layer
    (config 0) stays on the row kernel (too few steps and workgroups to
    amortise the pipeline fill), and a very sparse matrix (density below
    0.04) stays on the row kernel."""
    win = 128
    a1, n1, _ = S.gen_config(1, seed=1)
    w1 = S.plan_mfma_windows(a1, n1, flags=kernel)[0]
    assert len(w1) == (a1.nrow + win - 1) // win
    a0, n0, _ = S.gen_config(0, seed=1)
    assert len(S.plan_mfma_windows(a0, n0, flags=kernel)[0]) == 0
    sparse, _ = S.gen_lognormal_rows(4096, 4096, 50, seed=5)
    assert len(S.plan_mfma_windows(sparse, 512, flags=kernel)[0]) == 0
    # the density floor is overridable for tuning, the cost model still applies
    forced = S.plan_mfma_windows(a0, n0, flags=S.TCA_PLAN_FORCE_MFMA | kernel)[0]
    assert len(forced) == (a0.nrow + win - 1) // win


@pytest.mark.parametrize("m,k,p", [(50, 70, 0.1), (1, 1, 1.0), (300, 20, 0.3), (20, 300, 0.05), (5, 5, 0.0)])
def test_csr_transpose_matches_the_dense_transpose(m, k, p):
    """tca_csr_transpose: the transpose's structure and the value permutation
    reproduce the dense transpose exactly, with ascending columns per row."""
    import ctypes
    a, _ = S.gen_bernoulli(m, k, p, seed=m * 7 + k, dtype=S.TCA_F32)
    rpt = np.zeros(k + 1, np.int32)
    cit = np.zeros(max(a.nnz, 1), np.int32)
    perm = np.zeros(max(a.nnz, 1), np.int32)
    rp = np.ascontiguousarray(a.rowptr, np.int32)
    ci = np.ascontiguousarray(a.colidx, np.int32)
    S.call("tca_csr_transpose", S.np_ptr(rp, ctypes.c_int32), S.np_ptr(ci, ctypes.c_int32), m, k, a.nnz,
           S.np_ptr(rpt, ctypes.c_int32), S.np_ptr(cit, ctypes.c_int32), S.np_ptr(perm, ctypes.c_int32))
    at = S.CSR(k, m, rpt, cit[:a.nnz], a.values[perm[:a.nnz]], S.TCA_F32)
    assert np.array_equal(S.csr_to_dense(at), S.csr_to_dense(a).T)
    for r in range(k):
        assert np.all(np.diff(at.colidx[at.rowptr[r]:at.rowptr[r + 1]]) > 0)
    assert np.array_equal(np.sort(perm[:a.nnz]), np.arange(a.nnz))


@pytest.mark.parametrize("dtype", [S.TCA_F16, S.TCA_F32, S.TCA_BF16])
def test_binary_csr_cache_and_values_sidecar_round_trip(tmp_path, dtype):
    a, _ = S.gen_lognormal_rows(300, 500, 30, seed=3, dtype=dtype)
    p = str(tmp_path / "a.tcsr")
    S.write_csr_binary(p, a)
    b = S.read_csr_binary(p)
    assert (b.nrow, b.ncol, b.dtype) == (a.nrow, a.ncol, a.dtype)
    assert np.array_equal(b.rowptr, a.rowptr) and np.array_equal(b.colidx, a.colidx)
    assert np.array_equal(b.values.view(np.uint8), a.values.view(np.uint8))
    # .smtx pattern + values sidecar reproduce the matrix; values convert to the requested dtype
    sm, sv = str(tmp_path / "a.smtx"), str(tmp_path / "a.values")
    S.write_smtx(sm, a)
    S.write_values(sv, a)
    c = S.read_smtx(sm, dtype, values_path=sv)
    assert np.array_equal(c.colidx, a.colidx) and np.array_equal(c.values.view(np.uint8), a.values.view(np.uint8))
    c32 = S.read_smtx(sm, S.TCA_F32, values_path=sv)
    assert np.array_equal(c32.values, a.values_f32())


def test_binary_files_reject_damage(tmp_path):
    a, _ = S.gen_bernoulli(40, 30, 0.2, seed=2, dtype=S.TCA_F32)
    p = tmp_path / "a.tcsr"
    S.write_csr_binary(str(p), a)
    raw = p.read_bytes()
    (tmp_path / "short.tcsr").write_bytes(raw[:-4])                       # truncated
    (tmp_path / "magic.tcsr").write_bytes(b"X" + raw[1:])                 # wrong magic
    bad = bytearray(raw)
    off = 8 + 24 + 4 * 41                                                 # first column index
    bad[off:off + 4] = (10 ** 6).to_bytes(4, "little")                    # column out of range
    (tmp_path / "col.tcsr").write_bytes(bytes(bad))
    for name in ("short", "magic", "col"):
        with pytest.raises(S.TcaError):
            S.read_csr_binary(str(tmp_path / f"{name}.tcsr"))
    sm, sv = str(tmp_path / "a.smtx"), str(tmp_path / "b.values")
    S.write_smtx(sm, a)
    other, _ = S.gen_bernoulli(40, 30, 0.5, seed=9, dtype=S.TCA_F32)
    S.write_values(sv, other)                                             # nnz mismatch
    with pytest.raises(S.TcaError):
        S.read_smtx(sm, S.TCA_F32, values_path=sv)


# -------------------------------------------------------------- planner
@pytest.mark.parametrize("n,dtype", [(256, S.TCA_F16), (512, S.TCA_F16), (64, S.TCA_F16), (128, S.TCA_F32),
                                     (7, S.TCA_F32), (100, S.TCA_BF16), (1000, S.TCA_F16)])
def test_plan_covers_every_row_once(n, dtype):
    rng = np.random.default_rng(n)
    lens = np.concatenate([rng.integers(0, 40, 3000), [0, 0, 5000, 20000, 1, 2, 3]])
    rowptr = np.zeros(len(lens) + 1, np.int32)
    np.cumsum(lens, out=rowptr[1:])
    a = S.CSR(len(lens), 1, rowptr, np.zeros(rowptr[-1], np.int32), np.zeros(rowptr[-1], np.float32), S.TCA_F32)
    tasks, perm, longrows, geo = S.plan_row_tasks(a, n, dtype)
    e, g, cl, nch = geo["elems_per_lane"], geo["lanes_per_row"], geo["chunk_lanes"], geo["col_chunks"]
    es = 4 if dtype == S.TCA_F32 else 2
    assert e * es <= 16 and n % e == 0 and g in (1, 2, 4, 8, 16, 32, 64)
    assert cl <= g < 2 * cl and nch * cl * e >= n and (nch - 1) * cl * e < n
    if nch > 1:
        assert cl * e * es >= 128 or nch * cl > 64 * (nch // 2)  # chunks span whole L2 lines
    covered = np.zeros(len(lens), np.int64)
    parts = {}
    for i, (x, y, z, w) in enumerate(tasks):
        if w == 0:
            assert (y, z) == (rowptr[x], rowptr[x + 1]) and 0 < z - y <= geo["row_len"]
            covered[x] += 1
        elif w == 1:
            rows = perm[x:x + y]
            if z == 0:  # zero task: empty rows only, ascending (the kernel clears consecutive ones as one range)
                assert 1 <= y <= 64 and np.all(lens[rows] == 0)
                assert np.all(np.diff(rows) > 0)
            else:
                assert 1 <= y <= min(64, 4 * (64 // g)) and np.all(lens[rows] > 0)  # up to 4 passes of 64 / g rows
                assert z == lens[rows].max() and z <= geo["multi_max"]
            covered[rows] += 1
        elif w & 3 == 2:
            row, first, nseg, _ = longrows[x]
            assert first <= (w >> 2) < first + nseg
            assert lens[row] > geo["wide_len"]
            parts.setdefault(("seg", row), []).append((y, z))
        else:
            assert w & 3 == 3 and i % 4 == (w >> 2)  # quarters are 4-aligned, in order
            assert geo["row_len"] < lens[x] <= geo["wide_len"]
            parts.setdefault(("wide", x), []).append((y, z))
    for (kind, row), segs in parts.items():
        segs.sort()
        assert segs[0][0] == rowptr[row] and segs[-1][1] == rowptr[row + 1]
        assert all(segs[i][1] == segs[i + 1][0] for i in range(len(segs) - 1))
        if kind == "seg":
            assert max(z - y for y, z in segs) <= geo["seg_len"]
        else:
            assert len(segs) == 4
        covered[row] += 1
    assert np.all(covered == 1)
    # wide groups first, then segments, rows and multi groups
    kinds = [w & 3 for *_, w in tasks]
    assert kinds == sorted(kinds, key=lambda k: {3: 0, 2: 1, 0: 2, 1: 3}[k])
    zero = [w == 1 and z == 0 for _, _, z, w in tasks]
    assert zero == sorted(zero)  # zero tasks last


# ------------------------------------------------------------------ COO
def _shuffled_coo(rng, m, k, density):
    d = rng.standard_normal((m, k)).astype(np.float32)
    d[rng.random((m, k)) >= density] = 0
    r, c = np.nonzero(d)
    perm = rng.permutation(len(r))
    return d, r[perm].astype(np.int32), c[perm].astype(np.int32), d[r, c][perm]


def test_oracle_coo_pinned_by_scipy_and_dense():
    import scipy.sparse as sp
    rng = np.random.default_rng(61)
    d, r, c, v = _shuffled_coo(rng, 37, 53, 0.15)
    rp, ci, vv = oracle.coo_to_csr(37, 53, r, c, v)
    ref = sp.coo_matrix((v, (r, c)), shape=(37, 53)).tocsr()
    ref.sort_indices()
    assert np.array_equal(rp, ref.indptr) and np.array_equal(ci, ref.indices) and np.array_equal(vv, ref.data)
    drp, dci, dv = oracle.dense_to_csr(d)
    assert np.array_equal(rp, drp) and np.array_equal(ci, dci) and np.array_equal(vv, dv)
    rr, cc, v2 = oracle.csr_to_coo(rp, ci, vv)
    assert np.array_equal(oracle.coo_to_csr(37, 53, rr, cc, v2)[1], ci)
    assert oracle.coo_to_csr(3, 3, [0, 1, 0], [1, 2, 1], [1.0, 2.0, 3.0]) is None   # duplicate
    assert oracle.coo_to_csr(3, 3, [0, 3], [1, 2], [1.0, 2.0]) is None             # row out of range
    # a planted mistake (columns left in entry order) fails the pin
    bad = np.argsort(r, kind="stable")
    assert not np.array_equal(c[bad], ref.indices)


@pytest.mark.parametrize("dtype", [S.TCA_F16, S.TCA_BF16, S.TCA_F32])
def test_coo_conversions_match_oracle(dtype):
    rng = np.random.default_rng(62 + dtype)
    d, r, c, v = _shuffled_coo(rng, 120, 90, 0.1)
    vs = S.to_storage(v, dtype)
    a = S.coo_to_csr(120, 90, r, c, vs, dtype)
    rp, ci, ov = oracle.coo_to_csr(120, 90, r, c, vs)
    assert np.array_equal(a.rowptr, rp) and np.array_equal(a.colidx, ci) and np.array_equal(a.values, ov)
    rows, cols, vals = S.csr_to_coo(a)
    orr, occ, ovv = oracle.csr_to_coo(rp, ci, ov)
    assert np.array_equal(rows, orr) and np.array_equal(cols, occ) and np.array_equal(vals, ovv)
    # round trip CSR -> COO -> CSR is the identity
    b = S.coo_to_csr(120, 90, rows, cols, vals, dtype)
    assert np.array_equal(b.rowptr, a.rowptr) and np.array_equal(b.colidx, a.colidx) and np.array_equal(b.values, a.values)


def test_coo_edge_cases_and_rejections():
    z = S.coo_to_csr(4, 7, [], [], np.zeros(0, np.float32), S.TCA_F32)
    assert z.nnz == 0 and np.array_equal(z.rowptr, np.zeros(5, np.int32))
    rows, cols, vals = S.csr_to_coo(z)
    assert len(rows) == len(cols) == len(vals) == 0
    # empty rows between entries, a single column
    a = S.coo_to_csr(5, 1, [4, 0, 2], [0, 0, 0], np.array([3, 1, 2], np.float32), S.TCA_F32)
    assert a.rowptr.tolist() == [0, 1, 1, 2, 2, 3] and a.values.tolist() == [1.0, 2.0, 3.0]
    for rows_, cols_ in (([0, 0], [1, 1]),      # duplicate entry
                         ([0, 5], [1, 1]),      # row out of range
                         ([0, 1], [1, -1]),     # negative column
                         ([0, 1], [1, 3])):     # column out of range
        with pytest.raises(S.TcaError):
            S.coo_to_csr(5, 3, rows_, cols_, np.ones(2, np.float32), S.TCA_F32)


def test_compat_coo_round_trip_binary():
    """The reference-named C++ wrappers (csr_to_coo / coo_to_csr in
    tca_compat.hpp), host only: round trip, unsorted input, rejections."""
    import subprocess
    exe = os.path.join(ROOT, "spmm_amd", "bin", "compat_formats")
    r = subprocess.run([exe], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0 and "compat formats ok" in r.stdout, r.stdout + r.stderr
    for mode in ("dup", "range"):
        r = subprocess.run([exe, mode], capture_output=True, text=True, timeout=60)
        assert r.returncode != 0 and "coo_to_csr" in r.stderr, (mode, r.stdout, r.stderr)


# ------------------------------------------- reference-order MatrixMarket
def _random_mtx(rng, m, k, n, dup, one_based, values):
    r = rng.integers(0, m, n)
    c = rng.integers(0, k, n)
    if dup:
        r = np.concatenate([r, r[:dup]])
        c = np.concatenate([c, c[:dup]])
    v = np.round(rng.uniform(-8, 8, len(r)), 4)
    off = 1 if one_based else 0
    lines = ["%%MatrixMarket matrix coordinate real general", f"{m} {k} {len(r)}"]
    for i in range(len(r)):
        lines.append(f"{r[i] + off} {c[i] + off} {v[i]:g}" if values else f"{r[i] + off} {c[i] + off}")
    return "\n".join(lines) + "\n"


@pytest.mark.parametrize("m,k,n,dup,one_based,pattern", [(30, 40, 200, 5, True, False), (7, 300, 60, 0, False, False),
                                                         (50, 50, 300, 20, True, True), (1, 1, 3, 2, False, False),
                                                         (10, 10, 0, 0, True, False)])
@pytest.mark.parametrize("dtype", [S.TCA_F32, S.TCA_F16])
def test_mtx_file_order_reader_matches_the_reference_oracle(tmp_path, m, k, n, dup, one_based, pattern, dtype):
    """tca_mtx_read_csr_file_order and tca_mtx_read_dense reproduce the
    reference's mtx_input_to_CSR / mtx_input_to_Dense (oracle): shuffled
    entries, duplicates, one- and zero-based files, pattern files."""
    rng = np.random.default_rng(m * 31 + n)
    text = _random_mtx(rng, m, k, n, dup, one_based, not pattern)
    p = tmp_path / "a.mtx"
    p.write_text(text)
    a = S.read_mtx(str(p), pattern_only=pattern, zero_based=not one_based, dtype=dtype, file_order=True)
    om, ok, rp, ci, vals = oracle.mtx_to_csr_file_order(text, pattern, not one_based)
    assert (a.nrow, a.ncol) == (om, ok)
    assert np.array_equal(a.rowptr, rp) and np.array_equal(a.colidx, ci)
    assert np.array_equal(S.from_storage(a.values, dtype), S.from_storage(S.to_storage(vals, dtype), dtype))
    d = S.read_mtx_dense(str(p), zero_based=not one_based, dtype=dtype)
    want = oracle.mtx_to_dense(text, not one_based)
    assert np.array_equal(S.from_storage(d, dtype), S.from_storage(S.to_storage(want, dtype), dtype))


@pytest.mark.parametrize("text", ["3 4 3\n1 1 1\n2 2 2\n",        # fewer entries than the header
                                  "3 4 1\n4 1 1\n",                # row out of range (one based)
                                  "3 4 1\n1 5 1\n",                # column out of range
                                  "3 4 1\n1 1 x\n",                # bad value
                                  "3 4\n1 1 1\n",                  # bad size line
                                  "% only a comment\n"])
def test_mtx_file_order_reader_rejects_malformed(tmp_path, text):
    p = tmp_path / "bad.mtx"
    p.write_text(text)
    for fn in (lambda: S.read_mtx(str(p), file_order=True), lambda: S.read_mtx_dense(str(p))):
        with pytest.raises(S.TcaError) as ei:
            fn()
        assert ei.value.status == 6


def test_compat_reference_signature_mtx_readers(tmp_path):
    """mtx_input_to_CSR(ifstream&, CSR**, Arguments*) and mtx_input_to_Dense
    (tca_compat.hpp, Arguments from tca_arguments.hpp) give the reference's
    CSR and dense matrix (oracle), in half precision."""
    import subprocess
    exe = os.path.join(ROOT, "spmm_amd", "bin", "compat_formats")
    rng = np.random.default_rng(12)
    text = _random_mtx(rng, 12, 9, 60, 7, True, True)
    p = tmp_path / "c.mtx"
    p.write_text(text)
    for pattern in (0, 1):
        r = subprocess.run([exe, "mtx", str(p), str(pattern), "0"], capture_output=True, text=True, timeout=60)
        assert r.returncode == 0, r.stderr
        lines = r.stdout.splitlines()
        m, k, rp, ci, vals = oracle.mtx_to_csr_file_order(text, bool(pattern), False)
        assert [int(x) for x in lines[0].split()] == [m, k, len(ci)]
        assert [int(x) for x in lines[1].split()] == rp.tolist()
        assert [int(x) for x in lines[2].split()] == ci.tolist()
        got = np.array([float(x) for x in lines[3].split()], np.float32)
        assert np.array_equal(got, vals.astype(np.float16).astype(np.float32))
    r = subprocess.run([exe, "mtxdense", str(p), "0", "12", "9"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stderr
    got = np.array([float(x) for x in r.stdout.split()], np.float32).reshape(12, 9)
    assert np.array_equal(got, oracle.mtx_to_dense(text, False).astype(np.float16).astype(np.float32))
