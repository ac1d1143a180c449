"""spmm_amd -- MI355X-native TCA-SpMM (C = A * B, A in CSR, B dense, C fp32).

Python side of the library: numpy-level wrappers of the C ABI in
``include/tca_spmm.h`` / ``include/tca_host.h`` (readers, generators,
validation) and :class:`Plan`, which runs the gfx950 kernels on device
buffers given as raw addresses or torch tensors.

Reference surface mirrored here (YaoLingF/SPMM):
  * ``CSR`` host struct            -- reference src/general.cuh:125-134
  * ``.smtx`` reader               -- reference src/file_input.cu:135-193
  * ``convert_dense_to_csr``       -- reference src/miscalleneous.cu:29-65
  * ``compare_mat`` verdict        -- reference src/general.cuh:71-123
  * ``our_spmm_balanced`` driver   -- reference src/our_spmm.cu:478-594
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from . import _lib
from ._lib import (TCA_BF16, TCA_F16, TCA_F32, TCA_PLAN_DEFAULT, TCA_PLAN_FORCE_MFMA, TCA_PLAN_MFMA_DENSE, TCA_PLAN_MFMA_PAIR, TCA_PLAN_MFMA_COMPACT, TCA_PLAN_NO_MFMA, TCA_PLAN_NO_PANELS, TCA_PLAN_FORCE_PANELS, TCA_PLAN_NO_SCRATCH, TCA_PLAN_KNOWN_FLAGS, TCA_PLAN_MFMA_SHORT, TCA_TILES_NONE, TCA_TILES_PAIR, TCA_TILES_DENSE, TCA_TILES_DENSE_K, TCA_TILES_COMPACT, TCA_TILES_SHORT,
                   TcaError,
                   call, lib, np_ptr)

__all__ = ["CSR", "Plan", "TcaError", "TCA_F16", "TCA_F32", "TCA_BF16", "TCA_PLAN_DEFAULT", "TCA_PLAN_NO_MFMA", "TCA_PLAN_NO_PANELS", "TCA_PLAN_FORCE_PANELS", "TCA_PLAN_NO_SCRATCH",
           "TCA_PLAN_FORCE_MFMA", "TCA_PLAN_MFMA_DENSE", "TCA_PLAN_MFMA_PAIR", "TCA_PLAN_MFMA_COMPACT", "TCA_PLAN_KNOWN_FLAGS", "TCA_PLAN_MFMA_SHORT", "TCA_TILES_NONE", "TCA_TILES_PAIR", "TCA_TILES_DENSE", "TCA_TILES_DENSE_K", "TCA_TILES_COMPACT", "TCA_TILES_SHORT", "read_smtx", "read_smtx_dense", "write_smtx", "read_mtx", "read_mtx_dense", "write_values", "write_csr_binary",
           "read_csr_binary", "launch_floor", "dense_to_csr", "csr_to_bell", "bell_spmm", "prune_24", "csr_to_24", "spmm_24",
           "csr_to_dense", "compare_mat", "gen_config", "gen_dense", "gen_bernoulli", "gen_lognormal_rows",
           "gen_rmat", "gen_zipf_rows", "naive_csr_spmm", "plan_row_tasks", "plan_mfma_windows", "our_spmm_balanced", "condense_windows", "np_dtype",
           "to_storage", "from_storage"]

# numpy storage type of each value type (fp16/bf16 are kept as 16-bit patterns)
_STORAGE = {TCA_F16: np.float16, TCA_F32: np.float32, TCA_BF16: np.uint16}


def np_dtype(dtype: int):
    return _STORAGE[dtype]


def to_storage(x: np.ndarray, dtype: int) -> np.ndarray:
    """fp32 values -> storage array of `dtype` (round to nearest even)."""
    x = np.ascontiguousarray(x, np.float32)
    if dtype == TCA_F32:
        return x.copy()
    out = np.empty(x.shape, _STORAGE[dtype])
    lib.tca_convert_array(np_ptr(x), TCA_F32, np_ptr(out), dtype, x.size)
    return out


def from_storage(x: np.ndarray, dtype: int) -> np.ndarray:
    """storage array of `dtype` -> fp32 values (exact)."""
    x = np.ascontiguousarray(x)
    if dtype == TCA_F32:
        return x.astype(np.float32)
    out = np.empty(x.shape, np.float32)
    lib.tca_convert_array(np_ptr(x), dtype, np_ptr(out), TCA_F32, x.size)
    return out


@dataclass
class CSR:
    """Host CSR matrix (int32 offsets and indices, values in storage type)."""
    nrow: int
    ncol: int
    rowptr: np.ndarray
    colidx: np.ndarray
    values: np.ndarray
    dtype: int

    @property
    def nnz(self) -> int:
        return int(self.rowptr[-1]) if len(self.rowptr) else 0

    def values_f32(self) -> np.ndarray:
        return from_storage(self.values, self.dtype)

    def as_struct(self) -> _lib.TcaCsr:
        """A tca_csr view of this matrix (valid while self is alive)."""
        self.rowptr = np.ascontiguousarray(self.rowptr, np.int32)
        self.colidx = np.ascontiguousarray(self.colidx, np.int32)
        self.values = np.ascontiguousarray(self.values, _STORAGE[self.dtype])
        return _lib.TcaCsr(self.nrow, self.ncol, self.nnz, np_ptr(self.rowptr, ctypes.c_int32),
                           np_ptr(self.colidx, ctypes.c_int32), self.values.ctypes.data, self.dtype)

    @staticmethod
    def from_struct(s: _lib.TcaCsr, free: bool = True) -> "CSR":
        """Copies a library-allocated tca_csr into numpy arrays (and frees it)."""
        m, nnz = s.nRow, s.nnz
        rowptr = np.ctypeslib.as_array(s.row_offset, shape=(m + 1,)).copy()
        colidx = np.ctypeslib.as_array(s.col_idx, shape=(nnz,)).copy() if nnz else np.zeros(0, np.int32)
        st = _STORAGE[s.dtype]
        if nnz:
            buf = (ctypes.c_char * (nnz * np.dtype(st).itemsize)).from_address(s.value)
            values = np.frombuffer(buf, dtype=st).copy()
        else:
            values = np.zeros(0, st)
        out = CSR(s.nRow, s.nCol, rowptr, colidx, values, s.dtype)
        if free:
            lib.tca_csr_free(ctypes.byref(s))
        return out

    def astype(self, dtype: int) -> "CSR":
        if dtype == self.dtype:
            return self
        return CSR(self.nrow, self.ncol, self.rowptr, self.colidx, to_storage(self.values_f32(), dtype), dtype)

    def validate(self) -> None:
        call("tca_csr_validate", np_ptr(np.ascontiguousarray(self.rowptr, np.int32), ctypes.c_int32),
             np_ptr(np.ascontiguousarray(self.colidx, np.int32), ctypes.c_int32), self.nrow, self.ncol, self.nnz)


# ------------------------------------------------------------------ I/O
def read_smtx(path: str, dtype: int = TCA_F16, values_path: str = None) -> CSR:
    """.smtx pattern (values 1.0), or with values from a values file."""
    s = _lib.TcaCsr()
    if values_path is None:
        call("tca_smtx_read_csr", path.encode(), dtype, ctypes.byref(s))
    else:
        call("tca_smtx_read_csr_values", path.encode(), values_path.encode(), dtype, ctypes.byref(s))
    return CSR.from_struct(s)


def write_values(path: str, a: CSR) -> None:
    """A's values as a values file (the sidecar of a .smtx pattern)."""
    v = np.ascontiguousarray(a.values, _STORAGE[a.dtype])
    call("tca_values_write", path.encode(), v.ctypes.data, a.nnz, a.dtype)


def write_csr_binary(path: str, a: CSR) -> None:
    s = a.as_struct()
    call("tca_csr_write_binary", path.encode(), ctypes.byref(s))


def read_csr_binary(path: str) -> CSR:
    s = _lib.TcaCsr()
    call("tca_csr_read_binary", path.encode(), ctypes.byref(s))
    return CSR.from_struct(s)


def read_smtx_dense(path: str, dtype: int = TCA_F16) -> np.ndarray:
    p = ctypes.c_void_p()
    m, k, nnz = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int32()
    call("tca_smtx_read_dense", path.encode(), dtype, ctypes.byref(p), ctypes.byref(m), ctypes.byref(k),
         ctypes.byref(nnz))
    st = _STORAGE[dtype]
    n = m.value * k.value
    buf = (ctypes.c_char * max(n * np.dtype(st).itemsize, 1)).from_address(p.value)
    out = np.frombuffer(buf, dtype=st, count=n).copy().reshape(m.value, k.value)
    lib.tca_free(p)
    return out


def write_smtx(path: str, a: CSR) -> None:
    s = a.as_struct()
    call("tca_smtx_write", path.encode(), ctypes.byref(s))


def read_mtx(path: str, pattern_only: bool = False, zero_based: bool = False, dtype: int = TCA_F16,
             file_order: bool = False) -> CSR:
    """MatrixMarket coordinate file -> CSR.  Default: entries sorted by
    (row, col), duplicates rejected (tca_mtx_read_csr).  file_order: the
    reference's CSR -- rows ascending, each row's entries in file order,
    duplicates kept (tca_mtx_read_csr_file_order, reference
    src/file_input.cu:63-134)."""
    s = _lib.TcaCsr()
    fn = "tca_mtx_read_csr_file_order" if file_order else "tca_mtx_read_csr"
    call(fn, path.encode(), int(pattern_only), int(zero_based), dtype, ctypes.byref(s))
    return CSR.from_struct(s)


def read_mtx_dense(path: str, zero_based: bool = False, dtype: int = TCA_F16) -> np.ndarray:
    """MatrixMarket coordinate file -> dense matrix, the reference's
    mtx_input_to_Dense (src/file_input.cu:8-62): a value on every line (1.0
    when missing), a later duplicate overwriting an earlier one."""
    p = ctypes.c_void_p()
    m, k, nnz = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int32()
    call("tca_mtx_read_dense", path.encode(), int(zero_based), dtype, ctypes.byref(p), ctypes.byref(m),
         ctypes.byref(k), ctypes.byref(nnz))
    st = _STORAGE[dtype]
    n = m.value * k.value
    buf = (ctypes.c_char * max(n * np.dtype(st).itemsize, 1)).from_address(p.value)
    out = np.frombuffer(buf, dtype=st, count=n).copy().reshape(m.value, k.value)
    lib.tca_free(p)
    return out


def csr_to_bell(a: CSR, bsize: int):
    """Blocked-ELL of A (tca_csr_to_bell): (colind [brows, ell_blocks] int32,
    values [brows * bsize, ell_blocks * bsize] in A's storage dtype)."""
    rp = np.ascontiguousarray(a.rowptr, np.int32)
    ci = np.ascontiguousarray(a.colidx, np.int32)
    v = np.ascontiguousarray(a.values)
    eb = ctypes.c_int32()
    call("tca_csr_to_bell", np_ptr(rp, ctypes.c_int32), np_ptr(ci, ctypes.c_int32), v.ctypes.data_as(ctypes.c_void_p),
         a.nrow, a.ncol, a.nnz, a.dtype, bsize, ctypes.byref(eb), None, None)
    brows = (a.nrow + bsize - 1) // bsize
    colind = np.zeros((brows, eb.value), np.int32)
    vals = np.zeros((brows * bsize, eb.value * bsize), v.dtype)
    call("tca_csr_to_bell", np_ptr(rp, ctypes.c_int32), np_ptr(ci, ctypes.c_int32), v.ctypes.data_as(ctypes.c_void_p),
         a.nrow, a.ncol, a.nnz, a.dtype, bsize, ctypes.byref(eb), np_ptr(colind, ctypes.c_int32),
         vals.ctypes.data_as(ctypes.c_void_p))
    return colind, vals


def bell_spmm(colind, values, m: int, k: int, n: int, bsize: int, dtype: int, b, c, stream=None) -> None:
    """C = A * B for a Blocked-ELL A on the device (tca_bell_spmm); colind,
    values, b, c are torch tensors or device addresses."""
    ell_blocks = int(colind.shape[1]) if hasattr(colind, "shape") else 0
    call("tca_bell_spmm", _addr(colind), _addr(values), m, k, n, bsize, ell_blocks, dtype, _addr(b), _addr(c),
         _addr(stream) if stream is not None else None)


def prune_24(a: CSR) -> CSR:
    """A pruned to 2:4 along its rows (tca_prune_24: the two largest |value|
    of every 4 consecutive columns, lower column on ties)."""
    rp = np.ascontiguousarray(a.rowptr, np.int32)
    ci = np.ascontiguousarray(a.colidx, np.int32)
    v = np.ascontiguousarray(a.values)
    s = _lib.TcaCsr()
    call("tca_prune_24", np_ptr(rp, ctypes.c_int32), np_ptr(ci, ctypes.c_int32), v.ctypes.data_as(ctypes.c_void_p),
         a.nrow, a.ncol, a.nnz, a.dtype, ctypes.byref(s))
    return CSR.from_struct(s)


def csr_to_24(a: CSR):
    """Compressed 2:4 form of a 2:4 matrix (tca_csr_to_24): (vals [M, Kp/2]
    uint16 storage, meta [M, Kp/16] uint16), Kp = K rounded up to 64."""
    rp = np.ascontiguousarray(a.rowptr, np.int32)
    ci = np.ascontiguousarray(a.colidx, np.int32)
    v = np.ascontiguousarray(a.values)
    kp = (a.ncol + 63) // 64 * 64
    vals = np.zeros((a.nrow, kp // 2), np.uint16)
    meta = np.zeros((a.nrow, kp // 16), np.uint16)
    call("tca_csr_to_24", np_ptr(rp, ctypes.c_int32), np_ptr(ci, ctypes.c_int32), v.ctypes.data_as(ctypes.c_void_p),
         a.nrow, a.ncol, a.nnz, a.dtype, vals.ctypes.data_as(ctypes.c_void_p), meta.ctypes.data_as(ctypes.c_void_p))
    return vals, meta


def spmm_24(vals, meta, m: int, k: int, n: int, dtype: int, b, c, stream=None) -> None:
    """C = A * B for a compressed 2:4 A on the device (tca_spmm_24)."""
    call("tca_spmm_24", _addr(vals), _addr(meta), m, k, n, dtype, _addr(b), _addr(c),
         _addr(stream) if stream is not None else None)


def dense_to_csr(dense: np.ndarray, dtype: int) -> CSR:
    d = np.ascontiguousarray(dense, _STORAGE[dtype])
    s = _lib.TcaCsr()
    call("tca_dense_to_csr", np_ptr(d), d.shape[0], d.shape[1], dtype, ctypes.byref(s))
    return CSR.from_struct(s)


def csr_to_dense(a: CSR) -> np.ndarray:
    out = np.empty((a.nrow, a.ncol), _STORAGE[a.dtype])
    s = a.as_struct()
    call("tca_csr_to_dense", ctypes.byref(s), np_ptr(out))
    return out


def csr_to_coo(a: CSR):
    """(row_idx, col_idx, values) of A in CSR order (tca_csr_to_coo)."""
    s = a.as_struct()
    o = _lib.TcaCoo()
    call("tca_csr_to_coo", ctypes.byref(s), ctypes.byref(o))
    try:
        n = o.nnz
        rows = np.ctypeslib.as_array(o.row_idx, shape=(n,)).copy() if n else np.zeros(0, np.int32)
        cols = np.ctypeslib.as_array(o.col_idx, shape=(n,)).copy() if n else np.zeros(0, np.int32)
        st = _STORAGE[o.dtype]
        if n:
            buf = (ctypes.c_char * (n * np.dtype(st).itemsize)).from_address(o.value)
            vals = np.frombuffer(buf, dtype=st).copy()
        else:
            vals = np.zeros(0, st)
    finally:
        lib.tca_coo_free(ctypes.byref(o))
    return rows, cols, vals


def coo_to_csr(nrow: int, ncol: int, rows, cols, values, dtype: int) -> CSR:
    """CSR of a COO matrix in any entry order (tca_coo_to_csr): rows, then
    columns ascending; duplicate or out-of-range entries raise TcaError."""
    r = np.ascontiguousarray(rows, np.int32)
    c = np.ascontiguousarray(cols, np.int32)
    v = np.ascontiguousarray(values, _STORAGE[dtype])
    if not (len(r) == len(c) == len(v)):
        raise ValueError("coo_to_csr: rows, cols and values differ in length")
    s = _lib.TcaCoo(nrow, ncol, len(r), np_ptr(r, ctypes.c_int32), np_ptr(c, ctypes.c_int32), v.ctypes.data, dtype)
    o = _lib.TcaCsr()
    call("tca_coo_to_csr", ctypes.byref(s), ctypes.byref(o))
    return CSR.from_struct(o)


def compare_mat(gold: np.ndarray, cmp: np.ndarray, tol: float = 1e-3, floor: float = 1e-6,
                verbose: bool = False) -> dict:
    g = np.ascontiguousarray(gold, np.float32).ravel()
    c = np.ascontiguousarray(cmp, np.float32).ravel()
    if g.size != c.size:
        raise ValueError("size mismatch")
    r = _lib.TcaCompareResult()
    call("tca_compare_mat", np_ptr(g, ctypes.c_float), np_ptr(c, ctypes.c_float), g.size, tol, floor, int(verbose),
         ctypes.byref(r))
    return {"success": bool(r.success), "fail_count": r.fail_count, "first_fail": r.first_fail,
            "max_rel": r.max_rel, "max_rel_floor": r.max_rel_floor}


def naive_csr_spmm(a: CSR, b: np.ndarray, threads: int = 0) -> np.ndarray:
    bb = np.ascontiguousarray(b, _STORAGE[a.dtype])
    n = bb.shape[1]
    c = np.empty((a.nrow, n), np.float32)
    s = a.as_struct()
    call("tca_naive_csr_spmm", ctypes.byref(s), np_ptr(bb), np_ptr(c, ctypes.c_float), n, threads)
    return c


def condense_windows(a: CSR, win: int = 16):
    nw = (a.nrow + win - 1) // win
    rp = np.ascontiguousarray(a.rowptr, np.int32)
    ci = np.ascontiguousarray(a.colidx, np.int32)
    uoff = np.zeros(nw + 1, np.int64)
    call("tca_condense_windows", np_ptr(rp, ctypes.c_int32), np_ptr(ci, ctypes.c_int32), a.nrow, a.nnz, win,
         np_ptr(uoff, ctypes.c_int64), None, None)
    ucols = np.zeros(int(uoff[-1]), np.int32)
    cpos = np.zeros(a.nnz, np.int32)
    call("tca_condense_windows", np_ptr(rp, ctypes.c_int32), np_ptr(ci, ctypes.c_int32), a.nrow, a.nnz, win,
         np_ptr(uoff, ctypes.c_int64), np_ptr(ucols, ctypes.c_int32), np_ptr(cpos, ctypes.c_int32))
    return uoff, ucols, cpos


def plan_row_tasks(a: CSR, n: int, dtype: int = None):
    """Host-only task list of the row kernel: (tasks int32[T,4], perm, longrows int32[L,4], geometry)."""
    dtype = a.dtype if dtype is None else dtype
    rp = np.ascontiguousarray(a.rowptr, np.int32)
    nt, npm, nl = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int32()
    geo = np.zeros(8, np.int32)
    call("tca_plan_row_tasks", np_ptr(rp, ctypes.c_int32), a.nrow, a.ncol, n, dtype, ctypes.byref(nt), ctypes.byref(npm),
         ctypes.byref(nl), None, None, None, np_ptr(geo, ctypes.c_int32))
    tasks = np.zeros((nt.value, 4), np.int32)
    perm = np.zeros(max(npm.value, 1), np.int32)
    longrows = np.zeros((max(nl.value, 1), 4), np.int32)
    call("tca_plan_row_tasks", np_ptr(rp, ctypes.c_int32), a.nrow, a.ncol, n, dtype, ctypes.byref(nt), ctypes.byref(npm),
         ctypes.byref(nl), np_ptr(tasks, ctypes.c_int32), np_ptr(perm, ctypes.c_int32),
         np_ptr(longrows, ctypes.c_int32), np_ptr(geo, ctypes.c_int32))
    keys = ("elems_per_lane", "lanes_per_row", "col_chunks", "seg_len", "chunk_lanes", "row_len", "wide_len",
            "multi_max")
    return tasks, perm[:npm.value], longrows[:nl.value], {k: int(v) for k, v in zip(keys, geo)}


def plan_mfma_windows(a: CSR, n: int, dtype: int = None, flags: int = TCA_PLAN_DEFAULT):
    """Host-only MFMA window plan: (windows int32[W,4], ucols int32[S*32], eoff int32[S+1], entries uint32)."""
    dtype = a.dtype if dtype is None else dtype
    rp = np.ascontiguousarray(a.rowptr, np.int32)
    ci = np.ascontiguousarray(a.colidx, np.int32)
    nw, ns, ne = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int64()
    call("tca_plan_mfma_windows", np_ptr(rp, ctypes.c_int32), np_ptr(ci, ctypes.c_int32), a.nrow, n, dtype, flags,
         ctypes.byref(nw), ctypes.byref(ns), ctypes.byref(ne), None, None, None, None)
    windows = np.zeros((max(nw.value, 1), 4), np.int32)
    ucols = np.zeros(max(ns.value * 32, 1), np.int32)
    eoff = np.zeros(ns.value + 1, np.int32)
    entries = np.zeros(max(ne.value, 1), np.uint32)
    call("tca_plan_mfma_windows", np_ptr(rp, ctypes.c_int32), np_ptr(ci, ctypes.c_int32), a.nrow, n, dtype, flags,
         ctypes.byref(nw), ctypes.byref(ns), ctypes.byref(ne), np_ptr(windows, ctypes.c_int32),
         np_ptr(ucols, ctypes.c_int32), np_ptr(eoff, ctypes.c_int32), np_ptr(entries, ctypes.c_uint32))
    return windows[:nw.value], ucols[:ns.value * 32], eoff, entries[:ne.value]


def plan_panels(a: CSR, n: int, flags: int = TCA_PLAN_DEFAULT, dtype: int = None) -> dict:
    """Host view of the panel plan (tca_plan_panels) as numpy arrays."""
    dtype = a.dtype if dtype is None else dtype
    rp = np.ascontiguousarray(a.rowptr, np.int32)
    ci = np.ascontiguousarray(a.colidx, np.int32)
    sizes = np.zeros(16, np.int64)
    args = (np_ptr(rp, ctypes.c_int32), np_ptr(ci, ctypes.c_int32), a.nrow, a.ncol, n, dtype, flags,
            np_ptr(sizes, ctypes.c_int64))
    call("tca_plan_panels", *args, None, None, None, None, None, None, None, None, None)
    (n_panels, n_tiles, n_units, n_long, R, P, waves, rpg, elems, chunks, nnz_p, staged, n_seg, n_rows,
     stride, max_dword) = (int(x) for x in sizes)
    out = dict(panels=n_panels, tiles=n_tiles, n_units=n_units, R=R, P=P, waves=waves, rpg=rpg, elems=elems,
               chunks=chunks, nnz=nnz_p, staged=staged, segments=n_seg, n_rows=n_rows, cnt_stride=stride,
               cnt_rows=stride // (4 * waves) if waves else 0, max_dword=max_dword,
               rows=np.zeros(max(n_panels * R, 1), np.int32), cols=np.zeros(max(n_tiles * P, 1), np.int32),
               width=np.zeros(max(n_tiles, 1), np.uint8),
               cnt=np.zeros(max(n_tiles * stride, 1), np.uint8), pos=np.zeros(max(a.nnz, 1), np.uint8),
               units=np.zeros((max(n_units, 1), 4), np.int32), panel_units=np.zeros(max(n_panels, 1), np.int32),
               ustart=np.zeros(max(n_units * R, 1), np.int32), longrows=np.zeros((max(n_long, 1), 4), np.int32))
    call("tca_plan_panels", *args, np_ptr(out["rows"], ctypes.c_int32), np_ptr(out["cols"], ctypes.c_int32),
         out["width"].ctypes.data, out["cnt"].ctypes.data, out["pos"].ctypes.data, np_ptr(out["units"], ctypes.c_int32),
         np_ptr(out["panel_units"], ctypes.c_int32), np_ptr(out["ustart"], ctypes.c_int32),
         np_ptr(out["longrows"], ctypes.c_int32))
    out["rows"] = out["rows"][:n_panels * R]
    out["cols"] = out["cols"][:n_tiles * P]
    out["width"] = out["width"][:n_tiles]
    out["cnt"] = out["cnt"][:n_tiles * stride]
    out["pos"] = out["pos"][:a.nnz]
    out["units"] = out["units"][:n_units]
    out["panel_units"] = out["panel_units"][:n_panels]
    out["ustart"] = out["ustart"][:n_units * R]
    out["longrows"] = out["longrows"][:n_long]
    return out


def plan_launch_orders(a: CSR, n: int, flags: int = TCA_PLAN_DEFAULT) -> dict:
    """Host view of the launch orders (tca_plan_launch_orders): panel workgroup ->
    unit, the row tasks [T, 4] and wavefront slot -> task (-1 idle)."""
    rp = np.ascontiguousarray(a.rowptr, np.int32)
    ci = np.ascontiguousarray(a.colidx, np.int32)
    nb, nt, ns = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int32()
    args = (np_ptr(rp, ctypes.c_int32), np_ptr(ci, ctypes.c_int32), a.nrow, a.ncol, n, a.dtype, flags)
    call("tca_plan_launch_orders", *args, ctypes.byref(nb), None, ctypes.byref(nt), None, ctypes.byref(ns), None)
    po = np.zeros(max(nb.value, 1), np.int32)
    tasks = np.zeros((max(nt.value, 1), 4), np.int32)
    ro = np.zeros(max(ns.value, 1), np.int32)
    call("tca_plan_launch_orders", *args, ctypes.byref(nb), np_ptr(po, ctypes.c_int32), ctypes.byref(nt),
         np_ptr(tasks, ctypes.c_int32), ctypes.byref(ns), np_ptr(ro, ctypes.c_int32))
    return dict(panel_order=po[:nb.value], tasks=tasks[:nt.value], row_order=ro[:ns.value])


# ----------------------------------------------------------- generators
def gen_dense(rows: int, cols: int, dist: int = 0, seed: int = 1, dtype: int = TCA_F16,
              sparsity: float = 0.0) -> np.ndarray:
    """dist 0 = U(-1,1), 1 = N(0,1), 2 = U(0,1), 3 = seeded prepare_cpu_matrix."""
    out = np.empty((rows, cols), _STORAGE[dtype])
    call("tca_gen_dense", rows, cols, dist, sparsity, seed, dtype, np_ptr(out))
    return out


def _gen(name, *args):
    s = _lib.TcaCsr()
    st = _lib.TcaGenStats()
    call(name, *args, ctypes.byref(s), ctypes.byref(st))
    return CSR.from_struct(s), st.as_dict()


def gen_bernoulli(m, k, p, sigma=0.02, seed=1, dtype=TCA_F16):
    return _gen("tca_gen_bernoulli", m, k, p, sigma, seed, dtype)


def gen_lognormal_rows(m, k, mean, s=1.0, sigma=0.02, seed=1, dtype=TCA_F16):
    return _gen("tca_gen_lognormal_rows", m, k, mean, s, sigma, seed, dtype)


def gen_rmat(scale, n, samples, a=0.57, b=0.19, c=0.19, symmetric=True, norm=0, seed=1, dtype=TCA_F32):
    return _gen("tca_gen_rmat", scale, n, samples, a, b, c, int(symmetric), norm, seed, dtype)


def gen_zipf_rows(m, k, total, s=1.5, cap=200000, seed=1, dtype=TCA_F16):
    return _gen("tca_gen_zipf_rows", m, k, total, s, cap, seed, dtype)


def gen_config(cfg: int, seed: int = 1, dtype: int = -1):
    """One of the five benchmark configurations; returns (A, N, stats)."""
    s = _lib.TcaCsr()
    st = _lib.TcaGenStats()
    n = ctypes.c_int32()
    call("tca_gen_config", cfg, seed, dtype, ctypes.byref(s), ctypes.byref(n), ctypes.byref(st))
    return CSR.from_struct(s), n.value, st.as_dict()


# ------------------------------------------------------------------ plans
def _addr(x) -> int:
    """Device address of a torch tensor or an int."""
    if isinstance(x, int):
        return x
    return int(x.data_ptr())


def launch_floor(stream=None, iters: int = 100) -> float:
    """Mean milliseconds per launch of an empty kernel (tca_launch_floor)."""
    ms = ctypes.c_float()
    call("tca_launch_floor", _addr(stream) if stream is not None else None, iters, ctypes.byref(ms))
    return ms.value


class Plan:
    """A planned SpMM for one sparsity structure and width N (tca_spmm_plan)."""

    def __init__(self, a: CSR, n: int, flags: int = TCA_PLAN_DEFAULT):
        self._p = ctypes.c_void_p()
        rp = np.ascontiguousarray(a.rowptr, np.int32)
        ci = np.ascontiguousarray(a.colidx, np.int32)
        call("tca_spmm_plan_create", np_ptr(rp, ctypes.c_int32), np_ptr(ci, ctypes.c_int32), a.nrow, a.ncol, a.nnz,
             n, a.dtype, flags, ctypes.byref(self._p))
        self.m, self.k, self.n, self.nnz, self.dtype = a.nrow, a.ncol, n, a.nnz, a.dtype

    @classmethod
    def from_device(cls, rowptr, colidx, m: int, k: int, nnz: int, n: int, dtype: int,
                    flags: int = TCA_PLAN_DEFAULT, stream=None) -> "Plan":
        """A plan built on the GPU from a device-resident CSR
        (tca_spmm_plan_create_device); rowptr / colidx are int32 torch
        tensors (or device addresses)."""
        self = cls.__new__(cls)
        self._p = ctypes.c_void_p()
        call("tca_spmm_plan_create_device", _addr(rowptr), _addr(colidx), m, k, nnz, n, dtype, flags,
             _addr(stream) if stream is not None else None, ctypes.byref(self._p))
        self.m, self.k, self.n, self.nnz, self.dtype = m, k, n, nnz, dtype
        return self

    def export_rows(self):
        """The row-kernel task list (tasks [T, 4], perm, longrows [L, 4]) as numpy arrays."""
        nt, npm, nl = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int32()
        call("tca_spmm_plan_export_rows", self._p, ctypes.byref(nt), ctypes.byref(npm), ctypes.byref(nl),
             None, None, None)
        tasks = np.zeros((max(nt.value, 1), 4), np.int32)
        perm = np.zeros(max(npm.value, 1), np.int32)
        longrows = np.zeros((max(nl.value, 1), 4), np.int32)
        call("tca_spmm_plan_export_rows", self._p, ctypes.byref(nt), ctypes.byref(npm), ctypes.byref(nl),
             np_ptr(tasks, ctypes.c_int32), np_ptr(perm, ctypes.c_int32), np_ptr(longrows, ctypes.c_int32))
        return tasks[:nt.value], perm[:npm.value], longrows[:nl.value]

    def export_order(self):
        """The row kernel's launch order (slot -> task, -1 idle); empty in task order."""
        ns = ctypes.c_int32()
        call("tca_spmm_plan_export_order", self._p, ctypes.byref(ns), None)
        order = np.zeros(max(ns.value, 1), np.int32)
        call("tca_spmm_plan_export_order", self._p, ctypes.byref(ns), np_ptr(order, ctypes.c_int32))
        return order[:ns.value]

    def export_tiles(self):
        """The dense-tile data (windows [W, 4], entry positions, entry CSR
        indices, B row offsets of condensed columns) as numpy arrays."""
        nw, ne, nu = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int32()
        call("tca_spmm_plan_export_tiles", self._p, ctypes.byref(nw), ctypes.byref(ne), ctypes.byref(nu),
             None, None, None, None)
        win = np.zeros((max(nw.value, 1), 4), np.int32)
        pos = np.zeros(max(ne.value, 1), np.uint32)
        src = np.zeros(max(ne.value, 1), np.int32)
        ucols = np.zeros(max(nu.value, 1), np.uint32)
        call("tca_spmm_plan_export_tiles", self._p, ctypes.byref(nw), ctypes.byref(ne), ctypes.byref(nu),
             np_ptr(win, ctypes.c_int32), np_ptr(pos, ctypes.c_uint32), np_ptr(src, ctypes.c_int32),
             np_ptr(ucols, ctypes.c_uint32))
        return win[:nw.value], pos[:ne.value], src[:ne.value], ucols[:nu.value]

    def export_panels(self) -> dict:
        """The plan's row panels as the panel kernel reads them
        (tca_spmm_plan_export_panels) as numpy arrays."""
        sizes = np.zeros(8, np.int64)
        call("tca_spmm_plan_export_panels", self._p, np_ptr(sizes, ctypes.c_int64), None, None, None, None, None,
             None, None, None, None, None)
        n_p, n_t, n_u, n_o, n_lr, R, P, n_pos = (int(x) for x in sizes)
        out = dict(panels=n_p, tiles=n_t, n_units=n_u, R=R, P=P,
                   rows=np.zeros(max(n_p * R, 1), np.int32), boff=np.zeros(max(n_t * P, 1), np.uint32),
                   cnt=np.zeros(max(n_t * 96, 1), np.uint32), pos=np.zeros(max(n_pos, 1), np.uint8),
                   units=np.zeros((max(n_u, 1), 4), np.int32), order=np.zeros(max(n_o, 1), np.int32),
                   panel_units=np.zeros(max(n_p, 1), np.int32), ustart=np.zeros(max(n_u * R, 1), np.int32),
                   longrows=np.zeros((max(n_lr, 1), 4), np.int32), window=np.zeros(max(n_p, 1), np.uint8))
        cnt_words = self.PANEL_CNT_DWORDS
        out["cnt"] = np.zeros(max(n_t * cnt_words, 1), np.uint32)
        call("tca_spmm_plan_export_panels", self._p, np_ptr(sizes, ctypes.c_int64), np_ptr(out["rows"], ctypes.c_int32),
             np_ptr(out["boff"], ctypes.c_uint32), np_ptr(out["cnt"], ctypes.c_uint32), out["pos"].ctypes.data,
             np_ptr(out["units"], ctypes.c_int32), np_ptr(out["order"], ctypes.c_int32),
             np_ptr(out["panel_units"], ctypes.c_int32), np_ptr(out["ustart"], ctypes.c_int32),
             np_ptr(out["longrows"], ctypes.c_int32), out["window"].ctypes.data)
        for k, n in (("rows", n_p * R), ("boff", n_t * P), ("cnt", n_t * cnt_words), ("pos", n_pos), ("units", n_u),
                     ("order", n_o), ("panel_units", n_p), ("ustart", n_u * R), ("longrows", n_lr),
                     ("window", n_p)):
            out[k] = out[k][:n]
        return out

    # count dwords of one panel tile: consumer wavefronts x count rows (planner.hpp)
    PANEL_CNT_DWORDS = 12 * 8

    def info(self) -> dict:
        i = _lib.TcaPlanInfo()
        call("tca_spmm_plan_info", self._p, ctypes.byref(i))
        return i.as_dict()

    def run(self, val, b, c, stream=None) -> None:
        """C = A * B on device; val/b/c are torch tensors or device addresses."""
        call("tca_spmm_run", self._p, _addr(val), _addr(b), _addr(c), _addr(stream) if stream is not None else None)

    def run_static(self, val, b, c, stream=None) -> None:
        """tca_spmm_run_static: the same run with the library's static partial-row scratch."""
        call("tca_spmm_run_static", self._p, _addr(val), _addr(b), _addr(c),
             _addr(stream) if stream is not None else None)

    def time(self, val, b, c, stream=None, warmup: int = 5, iters: int = 10) -> float:
        ms = ctypes.c_float()
        call("tca_spmm_time", self._p, _addr(val), _addr(b), _addr(c),
             _addr(stream) if stream is not None else None, warmup, iters, ctypes.byref(ms))
        return ms.value

    PHASES = ("pack", "tiles", "rows", "segments", "panels")

    def time_phases(self, val, b, c, stream=None, warmup: int = 5, iters: int = 10) -> dict:
        """Mean milliseconds of each phase (MFMA value pack, MFMA tiles, row
        kernel, segment sums of split rows, panel kernel) inside whole runs:
        `iters` runs back to back on the stream, each phase's kernel
        dispatched with start / stop timestamps of its own."""
        ms = (ctypes.c_float * (len(self.PHASES) + 1))()
        call("tca_spmm_time_phases", self._p, _addr(val), _addr(b), _addr(c),
             _addr(stream) if stream is not None else None, warmup, iters, ms, len(self.PHASES))
        return {k: float(ms[i]) for i, k in enumerate(self.PHASES)}

    def time_run_phases(self, val, b, c, stream=None, warmup: int = 5, iters: int = 10):
        """(mean milliseconds of a whole run, per-phase dict) from the same
        `iters` runs: the run time between hipEvents before the first run and
        after the last, each phase's kernel timed by its own dispatch."""
        n = len(self.PHASES) + 1
        ms = (ctypes.c_float * n)()
        call("tca_spmm_time_phases", self._p, _addr(val), _addr(b), _addr(c),
             _addr(stream) if stream is not None else None, warmup, iters, ms, n)
        return float(ms[n - 1]), {k: float(ms[i]) for i, k in enumerate(self.PHASES)}

    def phases(self) -> tuple:
        """Names of the phases in which the plan launches a kernel, in run order."""
        m = ctypes.c_uint32()
        call("tca_spmm_plan_phases", self._p, ctypes.byref(m))
        return tuple(k for k in ("pack", "tiles", "panels", "rows", "segments")
                     if m.value & (1 << self.PHASES.index(k)))

    def time_subset(self, val, b, c, phases, stream=None, warmup: int = 5, iters: int = 10) -> float:
        """Mean milliseconds of runs that launch only the named phases, back to
        back between two hipEvents (tca_spmm_time_subset); C holds a full
        product only when every phase the plan uses is named."""
        mask = 0
        for k in phases:
            mask |= 1 << self.PHASES.index(k)
        ms = ctypes.c_float()
        call("tca_spmm_time_subset", self._p, _addr(val), _addr(b), _addr(c),
             _addr(stream) if stream is not None else None, mask, warmup, iters, ctypes.byref(ms))
        return ms.value

    def close(self) -> None:
        if self._p:
            lib.tca_spmm_plan_destroy(self._p)
            self._p = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


def our_spmm_balanced(a: CSR, b: np.ndarray, n_iter: int = 10, verbose: bool = False):
    """Host-pointer driver (reference our_spmm_balanced, src/our_spmm.cu:478-594).
    Returns (C, mean ms per launch)."""
    bb = np.ascontiguousarray(b, _STORAGE[a.dtype])
    n = bb.shape[1]
    c = np.empty((a.nrow, n), np.float32)
    ms = ctypes.c_double()
    rp = np.ascontiguousarray(a.rowptr, np.int32)
    ci = np.ascontiguousarray(a.colidx, np.int32)
    vals = np.ascontiguousarray(a.values)
    call("tca_spmm_host", np_ptr(rp, ctypes.c_int32), np_ptr(ci, ctypes.c_int32), np_ptr(vals), a.nrow, a.ncol,
         a.nnz, np_ptr(bb), np_ptr(c, ctypes.c_float), n, a.dtype, n_iter, int(verbose), ctypes.byref(ms))
    return c, ms.value
