"""The Python mirrors of the C-ABI structs (spmm_amd/_lib.py) against the
headers: a small C program built with gcc from include/tca_spmm.h and
include/tca_host.h prints sizeof and every field's offset, and each must
equal ctypes' layout of the mirror (a field added to a header and not to the
mirror, or in another place, changes an offset or the size)."""
import ctypes
import os
import shutil
import subprocess

import pytest

from spmm_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

MIRRORS = {
    "tca_plan_info": _lib.TcaPlanInfo,
    "tca_csr": _lib.TcaCsr,
    "tca_coo": _lib.TcaCoo,
    "tca_compare_result": _lib.TcaCompareResult,
    "tca_gen_stats": _lib.TcaGenStats,
}


def _c_layout(tmp_path):
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "tca_spmm.h"', '#include "tca_host.h"',
             "int main(void) {"]
    for cname, py in MIRRORS.items():
        lines.append(f'    printf("{cname} sizeof %zu\\n", sizeof({cname}));')
        for field, _ in py._fields_:
            lines.append(f'    printf("{cname} {field} %zu\\n", offsetof({cname}, {field}));')
    lines += ["    return 0;", "}"]
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines) + "\n")
    exe = tmp_path / "layout"
    r = subprocess.run(["gcc", "-std=c11", "-Wall", "-Werror", "-I", os.path.join(ROOT, "include"), str(src), "-o",
                        str(exe)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60, check=True).stdout
    layout = {}
    for ln in out.splitlines():
        cname, field, value = ln.split()
        layout[(cname, field)] = int(value)
    return layout


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not on PATH")
def test_ctypes_mirrors_match_the_headers(tmp_path):
    layout = _c_layout(tmp_path)
    for cname, py in MIRRORS.items():
        assert ctypes.sizeof(py) == layout[(cname, "sizeof")], (cname, ctypes.sizeof(py), layout[(cname, "sizeof")])
        for field, _ in py._fields_:
            assert getattr(py, field).offset == layout[(cname, field)], (cname, field)
