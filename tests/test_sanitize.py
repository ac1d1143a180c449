"""The host library under AddressSanitizer / UndefinedBehaviorSanitizer
(`make -C spmm_amd sanitize` -> spmm_amd/bin/host_sanitize, g++ builds of the
CPU sources, no GPU) over a corpus of valid, malformed and mutated input
files, plus allocation-failure injection through tca_debug_fail_allocs on
both the sanitized build and the production library."""
import os
import subprocess

import numpy as np
import pytest

from conftest import FIXTURE_SMTX, ROOT

import spmm_amd as S

EXE = os.path.join(ROOT, "spmm_amd", "bin", "host_sanitize")

CORPUS_TEXT = {
    "sorted.mtx": "%%MatrixMarket matrix coordinate real general\n% c\n3 4 4\n1 1 -1\n1 2 1.0\n2 3 4\n3 4 2.5\n",
    "unsorted_dups.mtx": "4 5 6\n2 3 1.5\n1 4 2\n2 1 -1\n3 2 0.1\n1 1 7\n2 3 5\n",
    "pattern.mtx": "3 3 3\n0 0\n1 2\n2 1\n",
    "count.mtx": "3 4 3\n1 1 1\n2 2 2\n",
    "range.mtx": "3 4 1\n4 1 1\n",
    "value.mtx": "3 4 1\n1 1 x\n",
    "huge_dense.mtx": "100000 100000 1\n1 1 1\n",
    "huge_nnz.mtx": "10 10 2000000000\n1 1 1\n",
    "empty.mtx": "",
    "crlf.mtx": "2 2 2\r\n1 1 1\r\n2 2 2\r\n",
    "bad_tokens.smtx": "2048, 512, 3\n0 1 2\n",
    "negative.smtx": "-5, 4, 1\n0 1\n0\n",
    "huge.smtx": "2000000000, 2000000000, 1\n0 1\n0\n",
    "short.smtx": "3, 3, 2\n0 1 2 2\n0 1\n",
}


def _corpus(tmp_path):
    d = tmp_path / "corpus"
    d.mkdir()
    for name, text in CORPUS_TEXT.items():
        (d / name).write_bytes(text.encode())
    (d / "fixture.smtx").write_bytes(open(FIXTURE_SMTX, "rb").read())
    a, _ = S.gen_bernoulli(30, 40, 0.1, seed=2, dtype=S.TCA_F16)
    S.write_csr_binary(str(d / "a.bin"), a)
    raw = open(str(d / "a.bin"), "rb").read()
    (d / "a_truncated.bin").write_bytes(raw[:len(raw) // 2])
    return d


def test_host_library_is_clean_under_asan_and_ubsan(tmp_path):
    """Every reader on every corpus file and on 24 deterministic mutations of
    each, generators, conversions, products and host planners, and the
    allocation-failure sweep: no sanitizer report, no leak, every status in
    range, every injected failure reported as TCA_ERR_ALLOC."""
    r = subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "spmm_amd"), "sanitize"], capture_output=True,
                       text=True, timeout=600)
    assert r.returncode == 0, r.stdout + r.stderr
    env = dict(os.environ)
    # allocations above 256 MiB return NULL (a dense reader asked for a
    # 100000 x 100000 matrix), which the library must report as
    # TCA_ERR_ALLOC; no reader sizes a container from a header alone
    env["ASAN_OPTIONS"] = "detect_leaks=1:halt_on_error=1:allocator_may_return_null=1:max_allocation_size_mb=256"
    env["UBSAN_OPTIONS"] = "halt_on_error=1:print_stacktrace=1"
    env["OMP_NUM_THREADS"] = "2"
    r = subprocess.run([EXE, str(_corpus(tmp_path))], capture_output=True, text=True, timeout=600, env=env)
    report = r.stdout + r.stderr
    assert r.returncode == 0, report[-4000:]
    # (allocator_may_return_null prints "WARNING: ... failed to allocate" for
    # the refused requests; reports are "ERROR: ...")
    assert "ERROR: AddressSanitizer" not in report and "ERROR: LeakSanitizer" not in report
    assert "runtime error" not in report
    assert "host sanitize ok" in r.stdout
    files = int(r.stdout.split("ok: ")[1].split(" files")[0])
    injected = int(r.stdout.split(", ")[-1].split(" injected")[0])
    assert files == len(CORPUS_TEXT) + 3 and injected >= 20, r.stdout


def _sweep(op):
    """Runs op() with its n-th host allocation failing, n = 0, 1, ... until it
    succeeds; returns the number of injected failures."""
    n = 0
    try:
        while True:
            S._lib.lib.tca_debug_fail_allocs(n, -1)
            try:
                op()
                return n
            except S.TcaError as e:
                assert e.status == 2, (n, e.status, str(e))  # TCA_ERR_ALLOC
            n += 1
            assert n < 100
    finally:
        S._lib.lib.tca_debug_fail_allocs(-1, -1)


def test_allocation_failures_are_reported_by_the_production_library(tmp_path):
    """The production library (not the sanitized build): every host
    allocation of a reader or a conversion can fail; each failure is
    TCA_ERR_ALLOC with nothing half-built returned, and the call then
    succeeds with the same result as without injection."""
    p = tmp_path / "m.mtx"
    p.write_text(CORPUS_TEXT["unsorted_dups.mtx"])
    want = S.read_mtx(str(p), dtype=S.TCA_F32, file_order=True)
    assert _sweep(lambda: S.read_mtx(str(p), dtype=S.TCA_F32, file_order=True)) == 3
    got = S.read_mtx(str(p), dtype=S.TCA_F32, file_order=True)
    assert np.array_equal(got.rowptr, want.rowptr) and np.array_equal(got.colidx, want.colidx)
    assert _sweep(lambda: S.read_mtx_dense(str(p))) == 1
    assert _sweep(lambda: S.read_smtx(FIXTURE_SMTX)) == 3
    a, _ = S.gen_bernoulli(40, 50, 0.2, seed=3, dtype=S.TCA_F16)
    assert _sweep(lambda: S.csr_to_coo(a)) == 3
    assert _sweep(lambda: S.gen_bernoulli(40, 50, 0.2, seed=3, dtype=S.TCA_F16)) == 3


@pytest.mark.gpu
def test_device_allocation_failures_release_everything(torch_cuda):
    """Plan creation (host and device planner) and the host driver with their
    n-th device allocation failing, for every n until they succeed: each
    failure is TCA_ERR_ALLOC and leaves the device's free memory where it was;
    the plan then built gives the oracle's product."""
    import ctypes
    from conftest import exact_dense, exact_values
    from oracle import oracle
    torch = torch_cuda
    rng = np.random.default_rng(9)
    a, _ = S.gen_lognormal_rows(600, 500, 30, seed=4, dtype=S.TCA_F16)
    a = S.CSR(a.nrow, a.ncol, a.rowptr, a.colidx, S.to_storage(exact_values(rng, a.nnz), S.TCA_F16), S.TCA_F16)
    n = 64
    b = S.to_storage(exact_dense(rng, (a.ncol, n)), S.TCA_F16)
    with S.Plan(a, n, S.TCA_PLAN_FORCE_MFMA):  # warm-up: runtime pools exist before the baseline
        pass
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    lib = S._lib.lib
    for flags in (S.TCA_PLAN_DEFAULT, S.TCA_PLAN_FORCE_MFMA, S.TCA_PLAN_NO_MFMA):
        k = 0
        while True:
            lib.tca_debug_fail_allocs(-1, k)
            try:
                plan = S.Plan(a, n, flags)
                lib.tca_debug_fail_allocs(-1, -1)
                break
            except S.TcaError as e:
                lib.tca_debug_fail_allocs(-1, -1)
                assert e.status == 2, (flags, k, e.status, str(e))  # TCA_ERR_ALLOC
                assert torch.cuda.mem_get_info()[0] == free0, (flags, k)
            k += 1
            assert k < 200
        assert k >= 3, (flags, k)
        dev = torch.device("cuda:0")
        val = torch.from_numpy(np.ascontiguousarray(a.values).view(np.int16)).to(dev)
        bd = torch.from_numpy(np.ascontiguousarray(b).view(np.int16)).to(dev)
        c = torch.empty((a.nrow, n), dtype=torch.float32, device=dev)
        plan.run(val, bd, c)
        torch.cuda.synchronize()
        assert np.array_equal(c.cpu().numpy(), oracle.csr_spmm(a.rowptr, a.colidx, S.from_storage(a.values, S.TCA_F16),
                                                                S.from_storage(b, S.TCA_F16)))
        plan.close()
        del val, bd, c
        torch.cuda.synchronize()
    # the host driver (copies in, plans, runs, copies out)
    cbuf = np.zeros((a.nrow, n), np.float32)
    k = 0
    while True:
        lib.tca_debug_fail_allocs(-1, k)
        st = lib.tca_spmm_host(a.rowptr.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)),
                               a.colidx.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)),
                               np.ascontiguousarray(a.values).ctypes.data, a.nrow, a.ncol, a.nnz,
                               np.ascontiguousarray(b).ctypes.data, cbuf.ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
                               n, S.TCA_F16, 1, 0, None)
        lib.tca_debug_fail_allocs(-1, -1)
        if st == 0:
            break
        assert st == 2 and torch.cuda.mem_get_info()[0] == free0, (k, st)
        k += 1
        assert k < 200
    assert k >= 3
