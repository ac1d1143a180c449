"""Writes the golden fixtures of tests/golden/ (run in the build container).

* scipy_spmm.npz -- small seeded CSR x dense products computed by
  scipy.sparse (fp64), an implementation independent of both the oracle and
  the HIP kernels.  Used to pin oracle.csr_spmm on the CPU and to check the
  GPU path directly against committed outputs.
* MANIFEST.json  -- the files here, with provenance.

The reference fixture body_decoder_layer_2_ffn_conv1.smtx is a verbatim copy
of the data file data/body_decoder_layer_2_ffn_conv1.smtx shipped by the
reference (data, not source).

Usage:  python tests/golden/make_golden.py
"""
import json
import os

import numpy as np
import scipy.sparse as sp

HERE = os.path.dirname(os.path.abspath(__file__))


def fixture_csr():
    with open(os.path.join(HERE, "body_decoder_layer_2_ffn_conv1.smtx")) as f:
        lines = f.read().split("\n")
    rowptr = np.array([int(t) for t in lines[1].split()], np.int32)
    colidx = np.array([int(t) for line in lines[2:] for t in line.split()], np.int32)
    return rowptr, colidx


def main():
    rng = np.random.default_rng(20261201)
    cases = {}

    def add(name, m, k, rowptr, colidx, values, b):
        a = sp.csr_matrix((values.astype(np.float64), colidx, rowptr), shape=(m, k))
        c = a @ b.astype(np.float64)
        cases[f"{name}__rowptr"] = rowptr.astype(np.int32)
        cases[f"{name}__colidx"] = colidx.astype(np.int32)
        cases[f"{name}__values"] = values
        cases[f"{name}__b"] = b
        cases[f"{name}__c"] = np.asarray(c)

    # the reference fixture (pattern -> value 1.0) with a seeded fp16 B, N = 256
    rp, ci = fixture_csr()
    b = rng.uniform(0, 1, (512, 256)).astype(np.float16)  # prepare_cpu_matrix-like U(0,1)
    add("fixture_n256", 2048, 512, rp, ci, np.ones(len(ci), np.float16), b)
    # random pruned-weight shapes, fp16 values N(0, 0.02), fp16 B U(-1,1)
    for name, m, k, n, p in [("bern_64x96_n64", 64, 96, 64, 0.1), ("bern_130x70_n40", 130, 70, 40, 0.3),
                             ("bern_33x500_n8", 33, 500, 8, 0.05)]:
        mask = rng.random((m, k)) < p
        rows, cols = np.nonzero(mask)
        rowptr = np.zeros(m + 1, np.int32)
        np.cumsum(np.bincount(rows, minlength=m), out=rowptr[1:])
        vals = (rng.standard_normal(len(rows)) * 0.02).astype(np.float16)
        vals[vals == 0] = np.float16(0.001)
        b = rng.uniform(-1, 1, (k, n)).astype(np.float16)
        add(name, m, k, rowptr, cols.astype(np.int32), vals, b)
    # fp32 graph-like case with one long row and empty rows
    m = k = 300
    lens = rng.integers(0, 6, m)
    lens[7] = 290
    lens[8:20] = 0
    rowptr = np.zeros(m + 1, np.int32)
    np.cumsum(lens, out=rowptr[1:])
    colidx = np.concatenate([np.sort(rng.choice(k, size=l, replace=False)) for l in lens]).astype(np.int32)
    vals = rng.standard_normal(len(colidx)).astype(np.float32)
    b = rng.standard_normal((k, 32)).astype(np.float32)
    add("graph_300_n32_f32", m, k, rowptr, colidx, vals, b)

    np.savez_compressed(os.path.join(HERE, "scipy_spmm.npz"), **cases)
    manifest = {
        "files": ["body_decoder_layer_2_ffn_conv1.smtx", "scipy_spmm.npz"],
        "scipy_spmm.npz": "scipy.sparse.csr_matrix @ dense in fp64; seed 20261201; written by make_golden.py",
        "body_decoder_layer_2_ffn_conv1.smtx": "copy of the reference's data/ fixture (pattern only)",
    }
    with open(os.path.join(HERE, "MANIFEST.json"), "w") as f:
        json.dump(manifest, f, indent=1)


if __name__ == "__main__":
    main()
