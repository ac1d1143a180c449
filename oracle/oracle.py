"""CPU oracle for the TCA-SpMM hot path (test infrastructure only).

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module, and only as the checker (or as the timed
CPU baseline).  The product (``spmm_amd``, the C ABI, the ``./test`` harness)
never imports or links it.

Each function names the reference lines it restates.  How each is pinned
(checked against something other than itself):

* ``parse_smtx``       -- the reference fixture's known answers (header, row
  count, nnz, per-row length buckets) and a second, independent tokeniser.
* ``dense_to_csr`` / ``csr_to_dense`` -- the fixture round trip
  (``.smtx -> dense -> CSR`` reproduces the file's arrays), CSR invariants,
  and the identity ``csr_to_dense(dense_to_csr(D)) == D``.
* ``csr_to_coo`` / ``coo_to_csr`` -- scipy's COO -> CSR conversion on
  shuffled unique entries, the dense brute force (entries placed in a dense
  matrix, then ``dense_to_csr``), and the round trip.
* ``condense_windows`` -- reconstruction: scattering every window's
  condensed tile back through its column union gives the dense window; the
  union equals the set of nonzero columns; brute force on tiny inputs.
* ``csr_spmm``         -- exact-arithmetic vectors (bit equality with an fp64
  closed form), closed forms (identity, permutation, all-ones rows), scipy
  fixtures and dense brute force.
* ``compare_mat``      -- hand-built cases for each branch of the verdict.
* ``parse_mtx`` / ``mtx_to_csr_file_order`` / ``mtx_to_dense`` -- the
  entries against scipy.io.mmread (an independent MatrixMarket parser that
  keeps file order) on shuffled files with values; the CSR and the dense
  matrix against scipy's dense form for unique entries; hand-built known
  answers for what scipy does not fix (each row's entries in file order,
  duplicates kept in the CSR, the last duplicate winning in the dense form,
  a missing value read as 0 / 1, one-based indices).
* ``dense_to_bell`` / ``bell_to_dense`` -- the round trip
  ``bell_to_dense(dense_to_bell(D)) == D`` (padded), hand-built cases (a
  block row with no blocks, zero-valued entries, ragged M and K), and the
  block lists against a brute-force scan of every block.
* ``prune_24`` / ``decompress_24`` -- the kept pair of every group against
  a brute-force search of the six pairs for the largest L1 norm (lowest
  columns on ties); ``decompress_24(compress(P)) == P`` and hand-built index
  words.  cuSPARSELt (the reference's library for this step) is not present;
  its documented STRIP rule is restated, its tie order is not pinned.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None


def build() -> None:
    """Compile oracle.c into liboracle.so (gcc, see oracle/Makefile)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        lib = ctypes.CDLL(_LIB_PATH)
        i32p = ctypes.POINTER(ctypes.c_int32)
        f32p = ctypes.POINTER(ctypes.c_float)
        f64p = ctypes.POINTER(ctypes.c_double)
        lib.oracle_csr_spmm_f32.argtypes = [i32p, i32p, f32p, ctypes.c_int32, ctypes.c_int32,
                                            f32p, f32p, ctypes.c_int]
        lib.oracle_csr_spmm_f32.restype = None
        lib.oracle_csr_spmm_f64.argtypes = [i32p, i32p, f64p, ctypes.c_int32, ctypes.c_int32,
                                            f64p, f64p, ctypes.c_int]
        lib.oracle_csr_spmm_f64.restype = None
        lib.oracle_dense_spmm_f32.argtypes = [f32p, f32p, f32p, ctypes.c_int32, ctypes.c_int32,
                                              ctypes.c_int32, ctypes.c_int]
        lib.oracle_dense_spmm_f32.restype = None
        lib.oracle_compare_mat.argtypes = [f32p, f32p, ctypes.c_int64, ctypes.c_float,
                                           ctypes.POINTER(ctypes.c_int64),
                                           ctypes.POINTER(ctypes.c_int64), f32p]
        lib.oracle_compare_mat.restype = ctypes.c_int
        _lib = lib
    return _lib


def _ptr(a: np.ndarray, ctype):
    return a.ctypes.data_as(ctypes.POINTER(ctype))


# ---------------------------------------------------------------- .smtx text
def parse_smtx(text: str):
    """Restates reference smtx_input_to_Dense's parse (src/file_input.cu:135-193).

    Line 1 is ``rows, cols, nnz`` split on ',' and read with stoi (which skips
    leading blanks).  Line 2 holds the row offsets split on ' '.  Every
    remaining line holds column indices split on ' '.  Returns
    ``(nrow, ncol, nnz, rowptr int32, colidx int32)``.
    """
    lines = text.split("\n")
    head = lines[0].split(",")
    nrow, ncol, nnz = int(head[0]), int(head[1]), int(head[2])
    rowptr = [int(t) for t in lines[1].split(" ") if t != ""]
    cols = []
    for line in lines[2:]:
        cols.extend(int(t) for t in line.split(" ") if t != "")
    return nrow, ncol, nnz, np.asarray(rowptr, np.int32), np.asarray(cols, np.int32)


def smtx_to_dense(nrow, ncol, rowptr, colidx, dtype=np.float16):
    """Dense matrix with 1.0 at every listed entry (src/file_input.cu:182-191)."""
    d = np.zeros((nrow, ncol), dtype=dtype)
    for r in range(nrow):
        for j in range(int(rowptr[r]), int(rowptr[r + 1])):
            d[r, colidx[j]] = 1.0
    return d


# ------------------------------------------------------------ dense <-> CSR
def dense_to_csr(dense: np.ndarray):
    """Restates reference convert_dense_to_csr (src/miscalleneous.cu:29-65).

    Row-major scan keeping entries whose fp32 value compares != 0.0f, so +-0
    are dropped and columns come out ascending.  Returns
    ``(rowptr int32[M+1], colidx int32[nnz], values dense.dtype[nnz])``.
    """
    m, _ = dense.shape
    keep = dense.astype(np.float32) != 0.0
    rows, cols = np.nonzero(keep)  # C order: row-major, columns ascending
    counts = np.bincount(rows, minlength=m)
    rowptr = np.zeros(m + 1, np.int32)
    np.cumsum(counts, out=rowptr[1:])
    return rowptr, cols.astype(np.int32), dense[rows, cols]


def csr_to_dense(rowptr, colidx, values, ncol):
    """Restates reference convert_csr_to_dense (src/miscalleneous.cu:66-81)."""
    m = len(rowptr) - 1
    d = np.zeros((m, ncol), dtype=values.dtype)
    for r in range(m):
        s, e = int(rowptr[r]), int(rowptr[r + 1])
        d[r, colidx[s:e]] = values[s:e]
    return d


# ------------------------------------------------------------ COO <-> CSR
def csr_to_coo(rowptr, colidx, values):
    """COO entries of a CSR matrix in CSR order.  The reference names the COO
    format only (mat_format::coo, src/mat_format.cuh:10-15); the CSR side
    follows convert_dense_to_csr's semantics (src/miscalleneous.cu:29-65)."""
    m = len(rowptr) - 1
    rows = np.repeat(np.arange(m, dtype=np.int32), np.diff(np.asarray(rowptr, np.int64)))
    return rows, np.asarray(colidx, np.int32).copy(), np.asarray(values).copy()


def coo_to_csr(nrow, ncol, rows, cols, values):
    """CSR of COO entries in any order: rows ascending, columns ascending in a
    row (the CSR indexing of src/miscalleneous.cu:29-65).  Returns None for a
    duplicate or out-of-range entry."""
    rows = np.asarray(rows, np.int64)
    cols = np.asarray(cols, np.int64)
    if len(rows) and (rows.min() < 0 or rows.max() >= nrow or cols.min() < 0 or cols.max() >= ncol):
        return None
    order = np.lexsort((cols, rows))
    r, c = rows[order], cols[order]
    if len(r) > 1 and np.any((r[1:] == r[:-1]) & (c[1:] == c[:-1])):
        return None
    rowptr = np.zeros(nrow + 1, np.int32)
    np.cumsum(np.bincount(r, minlength=nrow), out=rowptr[1:])
    return rowptr, c.astype(np.int32), np.asarray(values)[order]


# ------------------------------------------------------- condensed windows
def condense_windows(rowptr, colidx, m: int, win: int):
    """Condensed-tile indexing of the build (no reference counterpart; the
    reference kernel gathers B per nonzero, src/our_spmm.cu:44-60).

    For window w (rows [w*win, min(m, (w+1)*win))) the union U_w is the sorted
    set of its nonzero columns, and each nonzero's condensed position is its
    index in U_w.  Returns ``(uoff int64[nw+1], ucols int32, cpos int32[nnz])``.
    """
    nw = (m + win - 1) // win
    uoff = np.zeros(nw + 1, np.int64)
    ucols_parts = []
    cpos = np.zeros(len(colidx), np.int32)
    for w in range(nw):
        s = int(rowptr[w * win])
        e = int(rowptr[min(m, (w + 1) * win)])
        seg = np.asarray(colidx[s:e])
        u = np.unique(seg)
        ucols_parts.append(u.astype(np.int32))
        cpos[s:e] = np.searchsorted(u, seg).astype(np.int32)
        uoff[w + 1] = uoff[w] + len(u)
    ucols = np.concatenate(ucols_parts) if ucols_parts else np.zeros(0, np.int32)
    return uoff, ucols, cpos


# ------------------------------------------------------------------- SpMM
def csr_spmm(rowptr, colidx, values, b, threads: int = 0) -> np.ndarray:
    """fp32 CSR SpMM with reference naive_gemm arithmetic
    (src/miscalleneous.cu:114-134): per row, k ascending, fp32 multiply then
    fp32 add.  Inputs of any float dtype are first widened to fp32 exactly."""
    lib = _load()
    rowptr = np.ascontiguousarray(rowptr, np.int32)
    colidx = np.ascontiguousarray(colidx, np.int32)
    v = np.ascontiguousarray(values, np.float32)
    bb = np.ascontiguousarray(b, np.float32)
    m = len(rowptr) - 1
    n = bb.shape[1]
    c = np.empty((m, n), np.float32)
    lib.oracle_csr_spmm_f32(_ptr(rowptr, ctypes.c_int32), _ptr(colidx, ctypes.c_int32),
                            _ptr(v, ctypes.c_float), m, n, _ptr(bb, ctypes.c_float),
                            _ptr(c, ctypes.c_float), threads)
    return c


def csr_spmm_f64(rowptr, colidx, values, b, threads: int = 0) -> np.ndarray:
    """The same product accumulated in fp64 (error measurement only)."""
    lib = _load()
    rowptr = np.ascontiguousarray(rowptr, np.int32)
    colidx = np.ascontiguousarray(colidx, np.int32)
    v = np.ascontiguousarray(values, np.float64)
    bb = np.ascontiguousarray(b, np.float64)
    m = len(rowptr) - 1
    n = bb.shape[1]
    c = np.empty((m, n), np.float64)
    lib.oracle_csr_spmm_f64(_ptr(rowptr, ctypes.c_int32), _ptr(colidx, ctypes.c_int32),
                            _ptr(v, ctypes.c_double), m, n, _ptr(bb, ctypes.c_double),
                            _ptr(c, ctypes.c_double), threads)
    return c


def dense_spmm(a, b, threads: int = 0) -> np.ndarray:
    """Literal reference naive_gemm (src/miscalleneous.cu:114-134) on fp32."""
    lib = _load()
    aa = np.ascontiguousarray(a, np.float32)
    bb = np.ascontiguousarray(b, np.float32)
    m, k = aa.shape
    n = bb.shape[1]
    c = np.empty((m, n), np.float32)
    lib.oracle_dense_spmm_f32(_ptr(aa, ctypes.c_float), _ptr(bb, ctypes.c_float),
                              _ptr(c, ctypes.c_float), m, n, k, threads)
    return c


def dense_to_bell(dense: np.ndarray, bsize: int):
    """Blocked-ELL of a dense M x K matrix as the reference builds it for
    cusparseCreateBlockedEll (src/spmm_cusparse.cu:201-342): M and K are
    padded to multiples of bsize (:201-211); a block counts the nonzero
    values in it (:261-269); block row i lists, ascending, the block columns
    with a nonzero count, padded with -1 to the longest list (:281-309);
    values[r][e * bsize + c] = A[r][colind[r / bsize][e] * bsize + c], zero
    for padding blocks (:311-332).  Returns (colind, values)."""
    m, k = dense.shape
    brows, bcols = -(-m // bsize), -(-k // bsize)
    pad = np.zeros((brows * bsize, bcols * bsize), dense.dtype)
    pad[:m, :k] = dense
    counts = [[int(np.count_nonzero(pad[i * bsize:(i + 1) * bsize, j * bsize:(j + 1) * bsize]
                                    .astype(np.float32)))
               for j in range(bcols)] for i in range(brows)]
    width = max([sum(1 for x in row if x > 0) for row in counts] + [0])
    colind = np.full((brows, width), -1, np.int32)
    for i in range(brows):
        e = 0
        for j in range(bcols):
            if counts[i][j] > 0:
                colind[i, e] = j
                e += 1
    values = np.zeros((brows * bsize, width * bsize), dense.dtype)
    for i in range(brows):
        for e in range(width):
            j = colind[i, e]
            if j >= 0:
                values[i * bsize:(i + 1) * bsize, e * bsize:(e + 1) * bsize] = \
                    pad[i * bsize:(i + 1) * bsize, j * bsize:(j + 1) * bsize]
    return colind, values


def bell_to_dense(colind: np.ndarray, values: np.ndarray, bsize: int, k: int) -> np.ndarray:
    """Dense (block-padded rows) x K matrix of a Blocked-ELL (the inverse of
    dense_to_bell; -1 blocks hold nothing)."""
    brows, width = colind.shape
    bcols = -(-k // bsize)
    out = np.zeros((brows * bsize, bcols * bsize), values.dtype)
    for i in range(brows):
        for e in range(width):
            j = colind[i, e]
            if j >= 0:
                out[i * bsize:(i + 1) * bsize, j * bsize:(j + 1) * bsize] = \
                    values[i * bsize:(i + 1) * bsize, e * bsize:(e + 1) * bsize]
    return out[:, :k]


def prune_24(dense: np.ndarray) -> np.ndarray:
    """2:4 pruning of a dense M x K matrix along its rows as the reference
    requests it from cusparseLtSpMMAPrune(CUSPARSELT_PRUNE_SPMMA_STRIP)
    (src/spmm_cusparse.cu:83-84): in every group of 4 consecutive columns
    keep the two entries of largest magnitude (the pair with the largest L1
    norm), zero the others; equal magnitudes keep the lower column."""
    out = np.zeros_like(dense)
    m, k = dense.shape
    for r in range(m):
        for g0 in range(0, k, 4):
            grp = dense[r, g0:g0 + 4].astype(np.float32)
            order = sorted((i for i in range(len(grp)) if grp[i] != 0), key=lambda i: (-abs(grp[i]), i))
            for i in order[:2]:
                out[r, g0 + i] = dense[r, g0 + i]
    return out


def decompress_24(vals: np.ndarray, meta: np.ndarray, k: int) -> np.ndarray:
    """Dense M x K matrix of a compressed 2:4 A (vals [M, Kp/2], meta
    [M, Kp/16]; word q covers columns 16 q .. 16 q + 15, group G's two
    values at vals[8 q + 2 G], [8 q + 2 G + 1] sit at positions bits
    4G..4G+1 and 4G+2..4G+3)."""
    m = vals.shape[0]
    kp = meta.shape[1] * 16
    out = np.zeros((m, kp), vals.dtype)
    for r in range(m):
        for q in range(meta.shape[1]):
            w = int(meta[r, q])
            for g in range(4):
                for s in range(2):
                    pos = (w >> (4 * g + 2 * s)) & 3
                    v = vals[r, 8 * q + 2 * g + s]
                    if v != 0:
                        out[r, 16 * q + 4 * g + pos] = v
    return out[:, :k]


def compare_mat(gold, cmp, tol: float = 1e-3):
    """Restates reference compare_mat<float> (src/general.cuh:71-123).

    Returns ``(success, fail_count, first_fail, max_rel)``; the scan stops at
    the 10th failure like the reference."""
    lib = _load()
    g = np.ascontiguousarray(gold, np.float32).ravel()
    c = np.ascontiguousarray(cmp, np.float32).ravel()
    assert g.size == c.size
    fc = ctypes.c_int64()
    ff = ctypes.c_int64()
    mr = ctypes.c_float()
    ok = lib.oracle_compare_mat(_ptr(g, ctypes.c_float), _ptr(c, ctypes.c_float), g.size, tol,
                                ctypes.byref(fc), ctypes.byref(ff), ctypes.byref(mr))
    return bool(ok), fc.value, ff.value, mr.value


# ------------------------------------------------ MatrixMarket coordinate
def _strtof(tok: str) -> np.float32:
    """A decimal rounded once to fp32, like the reference's `stream >> float`."""
    libc = ctypes.CDLL(None)
    libc.strtof.restype = ctypes.c_float
    libc.strtof.argtypes = [ctypes.c_char_p, ctypes.POINTER(ctypes.c_char_p)]
    return np.float32(libc.strtof(tok.encode(), None))


def parse_mtx(text: str, zero_based: bool, read_value: bool, missing: float):
    """(rows, cols, [(r, c, v), ...] in file order) of a MatrixMarket
    coordinate text, as the reference reads it (src/file_input.cu:63-112):
    '%' lines skipped, "rows cols nnz", then "r c [v]" per line, indices
    shifted down by one unless zero based, v = `missing` when absent (and
    not read at all unless read_value)."""
    lines = text.splitlines()
    i = 0
    while lines[i].startswith("%"):
        i += 1
    rows, cols, nnz = (int(t) for t in lines[i].split()[:3])
    ents = []
    for line in lines[i + 1:]:
        tok = line.split()
        if not tok or tok[0].startswith("%"):
            continue
        r, c = int(tok[0]), int(tok[1])
        v = _strtof(tok[2]) if read_value and len(tok) > 2 else np.float32(missing)
        if not zero_based:
            r, c = r - 1, c - 1
        ents.append((r, c, v))
    assert len(ents) == nnz
    return rows, cols, ents


def mtx_to_csr_file_order(text: str, pattern_only: bool, zero_based: bool):
    """The reference's mtx_input_to_CSR (src/file_input.cu:63-134): rows in
    ascending order, each row's entries in file order, duplicates kept;
    pattern_only: value 1, else a missing value is 0.  Returns (nrow, ncol,
    rowptr, colidx, values fp32)."""
    rows, cols, ents = parse_mtx(text, zero_based, not pattern_only, 1.0 if pattern_only else 0.0)
    per_row = [[] for _ in range(rows)]
    for r, c, v in ents:
        per_row[r].append((c, v))
    rowptr = np.zeros(rows + 1, np.int32)
    colidx, vals = [], []
    for r in range(rows):
        rowptr[r + 1] = rowptr[r] + len(per_row[r])
        for c, v in per_row[r]:
            colidx.append(c)
            vals.append(v)
    return rows, cols, rowptr, np.array(colidx, np.int32), np.array(vals, np.float32)


def mtx_to_dense(text: str, zero_based: bool) -> np.ndarray:
    """The reference's mtx_input_to_Dense (src/file_input.cu:8-62): a value
    read on every line (1 when missing), entries written in file order (a
    later duplicate overwrites an earlier one).  fp32 result."""
    rows, cols, ents = parse_mtx(text, zero_based, True, 1.0)
    d = np.zeros((rows, cols), np.float32)
    for r, c, v in ents:
        d[r, c] = v
    return d
