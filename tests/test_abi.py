"""The C-ABI library loads and exports every function include/*.h declares
(no compute call needs a GPU here)."""
import ctypes
import os
import re
import subprocess

import pytest

from conftest import ROOT

import spmm_amd._lib as L


def _declared():
    names = set()
    inc = os.path.join(ROOT, "include")
    for fn in sorted(os.listdir(inc)):
        if not fn.endswith(".h"):
            continue
        text = open(os.path.join(inc, fn)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        text = re.sub(r"//[^\n]*", "", text)
        for m in re.finditer(r"\b(tca_\w+)\s*\(", text):
            names.add(m.group(1))
    return names


def test_every_declared_symbol_is_exported():
    declared = _declared()
    assert len(declared) > 30
    lib = ctypes.CDLL(L.LIB_PATH)
    missing = [n for n in sorted(declared) if not hasattr(lib, n)]
    assert not missing, missing


def test_binding_covers_declarations():
    assert _declared() == set(L.SIGNATURES), _declared() ^ set(L.SIGNATURES)


def test_exports_are_c_linkage():
    out = subprocess.run(["nm", "-D", "--defined-only", L.LIB_PATH], capture_output=True, text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if line.strip()}
    for n in _declared():
        assert n in exported, n  # unmangled


def test_status_strings_and_errors_without_gpu():
    assert L.lib.tca_status_string(0) == b"ok"
    assert L.lib.tca_status_string(6) == b"malformed input"
    assert L.lib.tca_version() >= 100
    # argument errors are reported, never exit the process
    p = ctypes.c_void_p()
    st = L.lib.tca_spmm_plan_create(None, None, 4, 4, 0, 8, 0, 0, ctypes.byref(p))
    assert st == 1 and b"rowptr" in L.lib.tca_last_error()
    st = L.lib.tca_spmm_run(None, None, None, None, None)
    assert st == 1


def test_rejects_invalid_csr_before_touching_device():
    import numpy as np
    rp = np.array([0, 2, 1, 3], np.int32)  # decreasing offsets
    ci = np.array([0, 1, 2], np.int32)
    p = ctypes.c_void_p()
    st = L.lib.tca_spmm_plan_create(L.np_ptr(rp, ctypes.c_int32), L.np_ptr(ci, ctypes.c_int32), 3, 4, 3, 8, 0, 0,
                                    ctypes.byref(p))
    assert st == 1 and b"decreases" in L.lib.tca_last_error()
    rp = np.array([0, 2, 3, 3], np.int32)
    ci = np.array([1, 1, 2], np.int32)  # not strictly ascending
    st = L.lib.tca_spmm_plan_create(L.np_ptr(rp, ctypes.c_int32), L.np_ptr(ci, ctypes.c_int32), 3, 4, 3, 8, 0, 0,
                                    ctypes.byref(p))
    assert st == 1 and b"ascending" in L.lib.tca_last_error()


def test_device_plan_argument_checks_need_no_gpu():
    """Flags and NULL pointers are rejected before any device call."""
    import ctypes
    import spmm_amd as S
    p = ctypes.c_void_p()
    # the kernel whose layout only the host planner builds
    with pytest.raises(S.TcaError) as ei:
        S._lib.call("tca_spmm_plan_create_device", 16, 16, 4, 4, 4, 8, S.TCA_F16, S.TCA_PLAN_MFMA_PAIR, None,
                    ctypes.byref(p))
    assert ei.value.status == 4
    # bits outside TCA_PLAN_KNOWN_FLAGS (4, 8 and 32 once selected tile kernels)
    for flags in (4, 8, 32, 1 << 20):
        with pytest.raises(S.TcaError) as ei:
            S._lib.call("tca_spmm_plan_create_device", 16, 16, 4, 4, 4, 8, S.TCA_F16, flags, None, ctypes.byref(p))
        assert ei.value.status == 1 and b"unknown plan flags" in S._lib.lib.tca_last_error(), flags
    with pytest.raises(S.TcaError) as ei:
        S._lib.call("tca_spmm_plan_create_device", None, None, 4, 4, 4, 8, S.TCA_F32, 0, None, ctypes.byref(p))
    assert ei.value.status == 1


def test_python_constants_match_the_header():
    """Every TCA_PLAN_*, TCA_TILES_* and dtype #define of include/tca_spmm.h
    has the same value in the Python binding."""
    import re
    import spmm_amd as S
    head = open(os.path.join(ROOT, "include", "tca_spmm.h")).read()
    found = re.findall(r"#define (TCA_(?:PLAN|TILES)_\w+) (\d+)u?", head)
    assert len(found) >= 14
    for name, value in found:
        assert getattr(S, name) == int(value), name
    # TCA_PLAN_KNOWN_FLAGS: the OR of the flags its definition names
    m = re.search(r"#define TCA_PLAN_KNOWN_FLAGS\s*\\?\s*\(([^)]*)\)", head)
    names = re.findall(r"TCA_PLAN_\w+", m.group(1))
    assert len(names) == 9
    want = 0
    for name in names:
        want |= getattr(S, name)
    assert S.TCA_PLAN_KNOWN_FLAGS == want
