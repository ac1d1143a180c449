"""The ./test harness (spmm_amd/bin/test) and the reference-named C++ API
example (spmm_amd/bin/compat_example).  Argument handling is checked on the
CPU (those paths exit before touching a GPU); runs are GPU tests."""
import json
import os
import subprocess

import pytest

from conftest import FIXTURE_SMTX, ROOT

BIN = os.path.join(ROOT, "spmm_amd", "bin")
TEST = os.path.join(BIN, "test")
EXAMPLE = os.path.join(BIN, "compat_example")


def run(args, timeout=120):
    return subprocess.run(args, capture_output=True, text=True, timeout=timeout)


def test_binaries_built():
    assert os.access(TEST, os.X_OK) and os.access(EXAMPLE, os.X_OK)


def test_usage_and_argument_errors():
    r = run([TEST])
    assert r.returncode != 0 and "Usage : ./test {matrix.smtx}" in r.stdout
    r = run([TEST, "-h"])
    assert r.returncode == 0 and "-n N" in r.stdout
    r = run([TEST, "/nonexistent.smtx"])
    assert r.returncode != 0 and "Input file not exists error" in r.stderr
    r = run([TEST, "-d", "2", FIXTURE_SMTX])
    assert r.returncode != 0 and "Not Implemented error for the specified dtype" in r.stderr
    r = run([EXAMPLE])
    assert r.returncode != 0 and "Usage" in r.stdout


@pytest.mark.gpu
def test_harness_on_reference_fixture(torch_cuda):
    r = run([TEST, FIXTURE_SMTX])
    print(r.stdout, r.stderr)
    assert r.returncode == 0, r.stdout + r.stderr
    out = r.stdout
    assert f"Input file - {FIXTURE_SMTX}" in out
    assert "preprocess " in out and "ms taken" in out
    assert "num_block: " in out and "blockdim: " in out and "shm: " in out
    # one line per kernel the plan launches, each with a non-empty grid
    launches = [l for l in out.splitlines() if l.startswith("num_block: ")]
    assert launches and any(l.endswith("(row_kernel)") for l in launches), launches
    assert all(int(l.split()[1]) > 0 for l in launches), launches
    assert "our: \x1b[36m[" in out and "validation failed" not in out


@pytest.mark.gpu
@pytest.mark.parametrize("args", [["-n", "64", "-d", "1"], ["-n", "512", "-d", "3", "-i", "3"], ["-n", "100"]])
def test_harness_flags(torch_cuda, args):
    r = run([TEST, *args, "-j", FIXTURE_SMTX])
    assert r.returncode == 0, r.stdout + r.stderr
    js = json.loads([l for l in r.stdout.splitlines() if l.startswith("{")][-1])
    assert js["valid"] and js["N"] == int(args[1]) and js["nnz"] == 1005


@pytest.mark.gpu
def test_harness_synthetic_and_mtx(torch_cuda, tmp_path):
    r = run([TEST, "-m", "300", "-k", "200", "-s", "0.9", "-n", "32", "-j"])
    assert r.returncode == 0, r.stdout + r.stderr
    js = json.loads([l for l in r.stdout.splitlines() if l.startswith("{")][-1])
    assert js["M"] == 300 and js["K"] == 200 and js["valid"]
    p = tmp_path / "a.mtx"
    p.write_text("%%MatrixMarket matrix coordinate real general\n4 5 5\n1 1 1.5\n1 5 -2\n2 2 0.25\n4 3 3\n4 4 1\n")
    r = run([TEST, "-b", "1", "-p", "0", "-n", "16", "-j", str(p)])
    assert r.returncode == 0, r.stdout + r.stderr
    js = json.loads([l for l in r.stdout.splitlines() if l.startswith("{")][-1])
    assert js["nnz"] == 5 and js["valid"]


@pytest.mark.gpu
def test_reference_api_example(torch_cuda):
    r = run([EXAMPLE, FIXTURE_SMTX, "256"])
    print(r.stdout, r.stderr)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "validation failed" not in r.stdout and "differs" not in r.stdout
