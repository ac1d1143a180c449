"""ctypes binding of libtcaspmm.so (the C ABI in include/tca_spmm.h and
include/tca_host.h).

The library is loaded from ``spmm_amd/lib/libtcaspmm.so`` inside the source
tree.  There is no fallback: if the library is missing or fails to load,
importing this module raises, so no caller can silently run something else.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "libtcaspmm.so")

TCA_F16, TCA_F32, TCA_BF16 = 0, 1, 2
DTYPE_NAMES = {TCA_F16: "f16", TCA_F32: "f32", TCA_BF16: "bf16"}
TCA_PLAN_DEFAULT, TCA_PLAN_NO_MFMA, TCA_PLAN_FORCE_MFMA = 0, 1, 2
TCA_PLAN_MFMA_DENSE = 16
TCA_PLAN_MFMA_PAIR = 64
TCA_PLAN_MFMA_COMPACT = 128
TCA_PLAN_NO_PANELS = 256
TCA_PLAN_FORCE_PANELS = 512
TCA_PLAN_NO_SCRATCH = 1024
TCA_PLAN_MFMA_SHORT = 2048
TCA_PLAN_KNOWN_FLAGS = (TCA_PLAN_NO_MFMA | TCA_PLAN_FORCE_MFMA | TCA_PLAN_MFMA_DENSE | TCA_PLAN_MFMA_PAIR |
                        TCA_PLAN_MFMA_COMPACT | TCA_PLAN_NO_PANELS | TCA_PLAN_FORCE_PANELS | TCA_PLAN_NO_SCRATCH |
                        TCA_PLAN_MFMA_SHORT)
# tile kernel of a plan (tca_plan_info.tile_kernel)
TCA_TILES_NONE, TCA_TILES_PAIR = 0, 3
TCA_TILES_DENSE, TCA_TILES_DENSE_K, TCA_TILES_COMPACT, TCA_TILES_SHORT = 4, 5, 7, 8

i32 = ctypes.c_int32
i64 = ctypes.c_int64
u32 = ctypes.c_uint32
u64 = ctypes.c_uint64
vp = ctypes.c_void_p
i32p = ctypes.POINTER(ctypes.c_int32)
u32p = ctypes.POINTER(ctypes.c_uint32)
i64p = ctypes.POINTER(ctypes.c_int64)
f32p = ctypes.POINTER(ctypes.c_float)


class TcaCsr(ctypes.Structure):
    _fields_ = [("nRow", i32), ("nCol", i32), ("nnz", i32), ("row_offset", i32p), ("col_idx", i32p),
                ("value", vp), ("dtype", i32)]


class TcaCoo(ctypes.Structure):
    _fields_ = [("nRow", i32), ("nCol", i32), ("nnz", i32), ("row_idx", i32p), ("col_idx", i32p),
                ("value", vp), ("dtype", i32)]


class TcaPlanInfo(ctypes.Structure):
    _fields_ = [("M", i32), ("K", i32), ("N", i32), ("nnz", i32), ("dtype", i32),
                ("elems_per_lane", i32), ("lanes_per_row", i32), ("col_chunks", i32),
                ("n_row_tasks", i32), ("n_multi_tasks", i32), ("n_seg_tasks", i32), ("n_long_rows", i32),
                ("n_windows_mfma", i32), ("rows_mfma", i32), ("nnz_mfma", i64), ("cond_cols_mfma", i64),
                ("row_blocks", i32), ("row_blockdim", i32), ("mfma_blocks", i32), ("mfma_blockdim", i32),
                ("mfma_lds_bytes", i32), ("seg_len", i32), ("scratch_bytes", i64), ("plan_ms", ctypes.c_double),
                ("n_wide_tasks", i32), ("chunk_lanes", i32), ("row_len", i32), ("wide_len", i32),
                ("tile_kernel", i32), ("n_panels", i32), ("n_panel_units", i32), ("rows_panels", i32),
                ("panel_blocks", i32), ("nnz_panels", i64), ("staged_panels", i64), ("panel_blockdim", i32),
                ("panel_lds_bytes", i32), ("panel_window", i32), ("rows_beside_panels", i32)]

    def as_dict(self):
        return {name: getattr(self, name) for name, _ in self._fields_}


class TcaCompareResult(ctypes.Structure):
    _fields_ = [("success", i32), ("fail_count", i64), ("first_fail", i64), ("max_rel", ctypes.c_float),
                ("max_rel_floor", ctypes.c_float)]


class TcaGenStats(ctypes.Structure):
    _fields_ = [("nnz", i64), ("max_row", i32), ("empty_rows", i32), ("rows_over_10k", i32),
                ("mean_row", ctypes.c_double), ("samples", i64)]

    def as_dict(self):
        return {name: getattr(self, name) for name, _ in self._fields_}


# name -> (restype, argtypes); every symbol declared in include/*.h
SIGNATURES = {
    # tca_spmm.h
    "tca_spmm_plan_create": (i32, [i32p, i32p, i32, i32, i32, i32, i32, u32, ctypes.POINTER(vp)]),
    "tca_spmm_run": (i32, [vp, vp, vp, vp, vp]),
    "tca_spmm_time": (i32, [vp, vp, vp, vp, vp, i32, i32, f32p]),
    "tca_spmm_time_phases": (i32, [vp, vp, vp, vp, vp, i32, i32, f32p, i32]),
    "tca_spmm_time_subset": (i32, [vp, vp, vp, vp, vp, u32, i32, i32, f32p]),
    "tca_spmm_plan_phases": (i32, [vp, u32p]),
    "tca_spmm_run_static": (i32, [vp, vp, vp, vp, vp]),
    "tca_sddmm": (i32, [vp, vp, vp, vp, vp]),
    "tca_launch_floor": (i32, [vp, i32, f32p]),
    "tca_gather_values": (i32, [vp, i32, vp, i32, vp, vp]),
    "tca_bell_spmm": (i32, [vp, vp, i32, i32, i32, i32, i32, i32, vp, vp, vp]),
    "tca_spmm_24": (i32, [vp, vp, i32, i32, i32, i32, vp, vp, vp]),
    "tca_spmm_plan_create_device": (i32, [vp, vp, i32, i32, i32, i32, i32, u32, vp, ctypes.POINTER(vp)]),
    "tca_spmm_plan_export_rows": (i32, [vp, i32p, i32p, i32p, i32p, i32p, i32p]),
    "tca_spmm_plan_export_order": (i32, [vp, i32p, i32p]),
    "tca_plan_launch_orders": (i32, [i32p, i32p, i32, i32, i32, i32, u32, i32p, i32p, i32p, i32p, i32p, i32p]),
    "tca_spmm_plan_export_tiles": (i32, [vp, i32p, i32p, i32p, i32p, u32p, i32p, u32p]),
    "tca_spmm_plan_export_panels": (i32, [vp, i64p, i32p, u32p, u32p, vp, i32p, i32p, i32p, i32p, i32p, vp]),
    "tca_spmm_plan_info": (i32, [vp, ctypes.POINTER(TcaPlanInfo)]),
    "tca_spmm_plan_destroy": (i32, [vp]),
    "tca_spmm_host": (i32, [i32p, i32p, vp, i32, i32, i32, vp, f32p, i32, i32, i32, i32,
                            ctypes.POINTER(ctypes.c_double)]),
    "tca_condense_windows": (i32, [i32p, i32p, i32, i32, i32, i64p, i32p, i32p]),
    "tca_plan_row_tasks": (i32, [i32p, i32, i32, i32, i32, i32p, i32p, i32p, i32p, i32p, i32p, i32p]),
    "tca_plan_mfma_windows": (i32, [i32p, i32p, i32, i32, i32, u32, i32p, i32p, i64p, i32p, i32p, i32p,
                                    ctypes.POINTER(ctypes.c_uint32)]),
    "tca_plan_panels": (i32, [i32p, i32p, i32, i32, i32, i32, u32, i64p, i32p, i32p, vp, vp, vp, i32p, i32p,
                              i32p, i32p]),
    "tca_status_string": (ctypes.c_char_p, [i32]),
    "tca_last_error": (ctypes.c_char_p, []),
    "tca_device_count": (i32, [i32p]),
    "tca_warm_up": (i32, []),
    "tca_version": (i32, []),
    # tca_host.h
    "tca_csr_free": (None, [ctypes.POINTER(TcaCsr)]),
    "tca_coo_free": (None, [ctypes.POINTER(TcaCoo)]),
    "tca_free": (None, [vp]),
    "tca_csr_validate": (i32, [i32p, i32p, i32, i32, i32]),
    "tca_smtx_read_csr": (i32, [ctypes.c_char_p, i32, ctypes.POINTER(TcaCsr)]),
    "tca_smtx_read_dense": (i32, [ctypes.c_char_p, i32, ctypes.POINTER(vp), i32p, i32p, i32p]),
    "tca_smtx_write": (i32, [ctypes.c_char_p, ctypes.POINTER(TcaCsr)]),
    "tca_mtx_read_csr": (i32, [ctypes.c_char_p, i32, i32, i32, ctypes.POINTER(TcaCsr)]),
    "tca_mtx_read_csr_file_order": (i32, [ctypes.c_char_p, i32, i32, i32, ctypes.POINTER(TcaCsr)]),
    "tca_debug_fail_allocs": (i32, [i64, i64]),
    "tca_mtx_read_dense": (i32, [ctypes.c_char_p, i32, i32, ctypes.POINTER(vp), i32p, i32p, i32p]),
    "tca_csr_write_binary": (i32, [ctypes.c_char_p, ctypes.POINTER(TcaCsr)]),
    "tca_csr_read_binary": (i32, [ctypes.c_char_p, ctypes.POINTER(TcaCsr)]),
    "tca_values_write": (i32, [ctypes.c_char_p, vp, i64, i32]),
    "tca_smtx_read_csr_values": (i32, [ctypes.c_char_p, ctypes.c_char_p, i32, ctypes.POINTER(TcaCsr)]),
    "tca_dense_to_csr": (i32, [vp, i32, i32, i32, ctypes.POINTER(TcaCsr)]),
    "tca_csr_to_dense": (i32, [ctypes.POINTER(TcaCsr), vp]),
    "tca_csr_to_coo": (i32, [ctypes.POINTER(TcaCsr), ctypes.POINTER(TcaCoo)]),
    "tca_coo_to_csr": (i32, [ctypes.POINTER(TcaCoo), ctypes.POINTER(TcaCsr)]),
    "tca_csr_transpose": (i32, [i32p, i32p, i32, i32, i32, i32p, i32p, i32p]),
    "tca_csr_convert": (i32, [ctypes.POINTER(TcaCsr), i32, ctypes.POINTER(TcaCsr)]),
    "tca_csr_to_bell": (i32, [i32p, i32p, vp, i32, i32, i32, i32, i32, i32p, i32p, vp]),
    "tca_prune_24": (i32, [i32p, i32p, vp, i32, i32, i32, i32, ctypes.POINTER(TcaCsr)]),
    "tca_csr_to_24": (i32, [i32p, i32p, vp, i32, i32, i32, i32, vp, vp]),
    "tca_f32_to_f16": (ctypes.c_uint16, [ctypes.c_float]),
    "tca_f16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
    "tca_f32_to_bf16": (ctypes.c_uint16, [ctypes.c_float]),
    "tca_bf16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
    "tca_convert_array": (None, [vp, i32, vp, i32, i64]),
    "tca_compare_mat": (i32, [f32p, f32p, i64, ctypes.c_float, ctypes.c_float, i32,
                              ctypes.POINTER(TcaCompareResult)]),
    "tca_naive_gemm": (i32, [vp, vp, f32p, i32, i32, i32, i32]),
    "tca_naive_csr_spmm": (i32, [ctypes.POINTER(TcaCsr), vp, f32p, i32, i32]),
    "tca_gen_dense": (i32, [i64, i64, i32, ctypes.c_float, u64, i32, vp]),
    "tca_gen_bernoulli": (i32, [i32, i32, ctypes.c_double, ctypes.c_double, u64, i32, ctypes.POINTER(TcaCsr),
                                ctypes.POINTER(TcaGenStats)]),
    "tca_gen_lognormal_rows": (i32, [i32, i32, ctypes.c_double, ctypes.c_double, ctypes.c_double, u64, i32,
                                     ctypes.POINTER(TcaCsr), ctypes.POINTER(TcaGenStats)]),
    "tca_gen_rmat": (i32, [i32, i32, i64, ctypes.c_double, ctypes.c_double, ctypes.c_double, i32, i32, u64, i32,
                           ctypes.POINTER(TcaCsr), ctypes.POINTER(TcaGenStats)]),
    "tca_gen_zipf_rows": (i32, [i32, i32, i64, ctypes.c_double, i32, u64, i32, ctypes.POINTER(TcaCsr),
                                ctypes.POINTER(TcaGenStats)]),
    "tca_gen_config": (i32, [i32, u64, i32, ctypes.POINTER(TcaCsr), i32p, ctypes.POINTER(TcaGenStats)]),
}


class TcaError(RuntimeError):
    """A libtcaspmm call returned a nonzero status."""

    def __init__(self, status: int, func: str, msg: str):
        super().__init__(f"{func}: status {status} ({msg})")
        self.status = status


def _preload_torch_hip_runtime() -> None:
    """Makes this process use PyTorch's HIP runtime when PyTorch is installed.

    PyTorch-ROCm ships its own libamdhip64.so (SONAME libamdhip64.so.7) and its
    libraries NEED it by the unversioned name from their own directory.  If
    libtcaspmm.so were loaded first, its NEEDED libamdhip64.so.7 would resolve
    to /opt/rocm/lib and a later `import torch` would load a second HIP
    runtime into the process; device pointers and streams from torch would
    then be foreign to this library.  Loading torch's copy first (by path,
    without importing torch) makes both resolve to one runtime.
    Set TCA_HIP_RUNTIME=system to skip this.
    """
    if os.environ.get("TCA_HIP_RUNTIME", "") == "system":
        return
    import importlib.util
    spec = importlib.util.find_spec("torch")
    if spec is None or not spec.submodule_search_locations:
        return
    path = os.path.join(list(spec.submodule_search_locations)[0], "lib", "libamdhip64.so")
    if os.path.exists(path):
        ctypes.CDLL(path, mode=ctypes.RTLD_GLOBAL)


def _load() -> ctypes.CDLL:
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"libtcaspmm.so not found at {LIB_PATH}; build it first (python -c 'import __graft_entry__ as g; g.build()' "
            "or make -C spmm_amd). There is no CPU fallback.")
    _preload_torch_hip_runtime()
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load()


def check(status: int, func: str = "tca") -> None:
    if status != 0:
        msg = lib.tca_last_error()
        raise TcaError(status, func, msg.decode() if msg else lib.tca_status_string(status).decode())


def call(name: str, *args):
    st = getattr(lib, name)(*args)
    check(st, name)
    return st


def np_ptr(a: np.ndarray, ctype=None):
    if ctype is None:
        return ctypes.c_void_p(a.ctypes.data)
    return a.ctypes.data_as(ctypes.POINTER(ctype))
