"""PyTorch-ROCm operator over the MI355X SpMM, with autograd.

    sm = SparseMatrix(a)                 # structure of A (host CSR), planned lazily per width
    c = spmm(sm, values, b)              # C = A * B, fp32, differentiable in values and B

The operator is registered with torch.library as torch.ops.spmm_amd.spmm
(schema: spmm(int handle, Tensor values, Tensor b) -> Tensor), with a fake
kernel (output shape and dtype only, for torch.compile and meta tracing)
and its autograd formula registered through register_autograd; `handle`
names a SparseMatrix (its structure and plans stay on the Python side, so
the op's arguments are plain ints and tensors).  Forward runs the library's
planned SpMM (tca_spmm_run) on the current torch stream.  Backward, through
the two companion ops spmm_amd::spmm_t and spmm_amd::sddmm:
    dB      = A^T * dC     -- an SpMM with a plan of the transpose (fp32; A's
                              values reordered on the device by tca_gather_values),
    dvalues = SDDMM(dC, B) -- <dC[row(j), :], B[col(j), :]> per nonzero (tca_sddmm).
All three are the library's HIP kernels; torch only supplies device memory
and the stream.  No counterpart in the reference, whose entry point
our_spmm_balanced (src/our_spmm.cuh:4) is forward-only; this is the operator
a GCN / GraphSAGE aggregation (C = A * X with A the normalised adjacency)
calls, forward and backward.

A plan owns device scratch that every run rewrites (packed MFMA entries,
partial rows of split rows), so one plan cannot serve two streams at once:
running a SparseMatrix's plan on a stream while its previous run on another
stream has not completed raises RuntimeError instead of racing.

Errors follow the library: TcaError with the library's message.  There is no
CPU fallback: the op needs the HIP library and a GPU.
"""
from __future__ import annotations

import ctypes
import itertools

import numpy as np
import torch

from . import (CSR, TCA_BF16, TCA_F16, TCA_F32, TCA_PLAN_DEFAULT, Plan, _addr, call, np_ptr)

__all__ = ["SparseMatrix", "spmm", "GCNConv", "SAGEMeanConv", "TORCH_DTYPES", "lookup"]

TORCH_DTYPES = {torch.float16: TCA_F16, torch.bfloat16: TCA_BF16, torch.float32: TCA_F32}


# SparseMatrix objects by handle (the int the registered ops take)
_REGISTRY: dict = {}
_HANDLES = itertools.count(1)


def lookup(handle: int) -> "SparseMatrix":
    sm = _REGISTRY.get(int(handle))
    if sm is None:
        raise ValueError(f"spmm_amd: no open SparseMatrix with handle {handle}")
    return sm


class SparseMatrix:
    """A fixed CSR sparsity structure A (M x K) for the operator.

    Holds the host structure, its transpose (computed once), and the plans of
    C = A * B (A's dtype) and of A^T * G (fp32) for every width N used, so a
    training loop plans once per layer width and reuses the plans."""

    def __init__(self, a: CSR, device="cuda:0", flags: int = TCA_PLAN_DEFAULT):
        self.a = a
        self.shape = (a.nrow, a.ncol)
        self.nnz = a.nnz
        self.dtype = a.dtype
        self.flags = flags
        self.device = torch.device(device)
        rp = np.ascontiguousarray(a.rowptr, np.int32)
        ci = np.ascontiguousarray(a.colidx, np.int32)
        rpt = np.zeros(a.ncol + 1, np.int32)
        cit = np.zeros(max(a.nnz, 1), np.int32)
        perm = np.zeros(max(a.nnz, 1), np.int32)
        call("tca_csr_transpose", np_ptr(rp, ctypes.c_int32), np_ptr(ci, ctypes.c_int32), a.nrow, a.ncol, a.nnz,
             np_ptr(rpt, ctypes.c_int32), np_ptr(cit, ctypes.c_int32), np_ptr(perm, ctypes.c_int32))
        self.at = CSR(a.ncol, a.nrow, rpt, cit[:a.nnz], np.zeros(a.nnz, np.float32), TCA_F32)
        self.perm = torch.from_numpy(perm[:a.nnz].copy()).to(self.device)
        self._plans: dict = {}
        self._plans_t: dict = {}
        self._inflight: dict = {}  # plan key -> (stream handle, event after its last run)
        self.handle = next(_HANDLES)
        _REGISTRY[self.handle] = self

    def plan(self, n: int) -> Plan:
        if n not in self._plans:
            self._plans[n] = Plan(self.a, n, self.flags)
        return self._plans[n]

    def plan_t(self, n: int) -> Plan:
        if n not in self._plans_t:
            self._plans_t[n] = Plan(self.at, n, self.flags)
        return self._plans_t[n]

    def values_tensor(self) -> torch.Tensor:
        """A's host values as a device tensor of the matching torch dtype."""
        v = torch.from_numpy(np.ascontiguousarray(self.a.values).view(
            {TCA_F16: np.float16, TCA_BF16: np.int16, TCA_F32: np.float32}[self.dtype]).copy())
        if self.dtype == TCA_BF16:
            v = v.view(torch.bfloat16)
        return v.to(self.device)

    def guarded(self, key, device) -> "_Guard":
        """Context for one run of the plan `key` on the current stream of
        `device`: raises RuntimeError if the plan's previous run was on
        another stream and has not completed; records its completion after."""
        return _Guard(self, key, torch.cuda.current_stream(device))

    def close(self) -> None:
        for p in list(self._plans.values()) + list(self._plans_t.values()):
            p.close()
        self._plans.clear()
        self._plans_t.clear()
        self._inflight.clear()
        _REGISTRY.pop(self.handle, None)


class _Guard:
    def __init__(self, sm: SparseMatrix, key, stream: torch.cuda.Stream):
        self.sm, self.key, self.stream = sm, key, stream

    def __enter__(self) -> int:
        prev = self.sm._inflight.get(self.key)
        if prev is not None and prev[0] != self.stream.cuda_stream and not prev[1].query():
            raise RuntimeError(f"spmm_amd: the plan {self.key} of SparseMatrix {self.sm.handle} is still running on "
                               f"another stream; a plan's scratch serves one run at a time (synchronise that stream, "
                               f"or use one SparseMatrix per stream)")
        return self.stream.cuda_stream

    def __exit__(self, exc_type, exc, tb) -> None:
        if exc_type is None:
            prev = self.sm._inflight.get(self.key)
            ev = prev[1] if prev is not None else torch.cuda.Event()
            ev.record(self.stream)
            self.sm._inflight[self.key] = (self.stream.cuda_stream, ev)


def _check(sm: SparseMatrix, values: torch.Tensor, b: torch.Tensor):
    if values.device.type != "cuda" or b.device.type != "cuda":
        raise ValueError("spmm: values and B must be GPU tensors (no CPU fallback)")
    if TORCH_DTYPES.get(values.dtype) != sm.dtype or TORCH_DTYPES.get(b.dtype) != sm.dtype:
        raise TypeError(f"spmm: values and B must have A's dtype ({sm.dtype}); got {values.dtype}, {b.dtype}")
    if values.dim() != 1 or values.numel() != sm.nnz:
        raise ValueError(f"spmm: values must be 1-D with {sm.nnz} entries")
    if b.dim() != 2 or b.shape[0] != sm.shape[1]:
        raise ValueError(f"spmm: B must be {sm.shape[1]} x N, got {tuple(b.shape)}")


@torch.library.custom_op("spmm_amd::spmm", mutates_args=())
def _spmm_op(handle: int, values: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """C = A * B in fp32, A = the structure of SparseMatrix `handle` with `values`."""
    sm = lookup(handle)
    _check(sm, values, b)
    values = values.contiguous()
    b = b.contiguous()
    n = b.shape[1]
    c = torch.empty((sm.shape[0], n), dtype=torch.float32, device=b.device)
    with sm.guarded(("A", n), b.device) as stream:
        sm.plan(n).run(values, b, c, stream=stream)
    return c


@_spmm_op.register_fake
def _spmm_fake(handle: int, values: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    sm = lookup(handle)
    return b.new_empty((sm.shape[0], b.shape[1]), dtype=torch.float32)


@torch.library.custom_op("spmm_amd::spmm_t", mutates_args=())
def _spmm_t_op(handle: int, values: torch.Tensor, g: torch.Tensor) -> torch.Tensor:
    """A^T * G in fp32 (G fp32, M x N): A's values reordered to the
    transpose's order on the device (tca_gather_values), then the planned
    SpMM of the transpose structure."""
    sm = lookup(handle)
    g = g.contiguous()
    n = g.shape[1]
    vt = torch.empty(sm.nnz, dtype=torch.float32, device=g.device)
    out = torch.empty((sm.shape[1], n), dtype=torch.float32, device=g.device)
    with sm.guarded(("AT", n), g.device) as stream:
        call("tca_gather_values", _addr(sm.perm), sm.nnz, _addr(values.contiguous()), sm.dtype, _addr(vt), stream)
        sm.plan_t(n).run(vt, g, out, stream=stream)
    return out


@_spmm_t_op.register_fake
def _spmm_t_fake(handle: int, values: torch.Tensor, g: torch.Tensor) -> torch.Tensor:
    sm = lookup(handle)
    return g.new_empty((sm.shape[1], g.shape[1]), dtype=torch.float32)


@torch.library.custom_op("spmm_amd::sddmm", mutates_args=())
def _sddmm_op(handle: int, g: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """Per nonzero j of A: <G[row(j), :], B[col(j), :]> in fp32 (tca_sddmm)."""
    sm = lookup(handle)
    g = g.contiguous()
    b = b.contiguous()
    n = b.shape[1]
    gv = torch.empty(sm.nnz, dtype=torch.float32, device=b.device)
    with sm.guarded(("A", n), b.device) as stream:
        call("tca_sddmm", sm.plan(n)._p, _addr(g), _addr(b), _addr(gv), stream)
    return gv


@_sddmm_op.register_fake
def _sddmm_fake(handle: int, g: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    sm = lookup(handle)
    return b.new_empty((sm.nnz,), dtype=torch.float32)


def _spmm_setup(ctx, inputs, output) -> None:
    handle, values, b = inputs
    ctx.handle = handle
    ctx.save_for_backward(values, b)


def _spmm_backward(ctx, gc):
    values, b = ctx.saved_tensors
    gc = gc.contiguous().to(torch.float32)
    grad_values = grad_b = None
    if ctx.needs_input_grad[1]:
        grad_values = torch.ops.spmm_amd.sddmm(ctx.handle, gc, b).to(values.dtype)
    if ctx.needs_input_grad[2]:
        grad_b = torch.ops.spmm_amd.spmm_t(ctx.handle, values, gc).to(b.dtype)
    return None, grad_values, grad_b


_spmm_op.register_autograd(_spmm_backward, setup_context=_spmm_setup)


def spmm(sm: SparseMatrix, values: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """C = A * B (fp32 result) with A's structure from `sm` and its values
    `values`; differentiable in `values` and `b` (torch.ops.spmm_amd.spmm)."""
    return torch.ops.spmm_amd.spmm(sm.handle, values, b)


class GCNConv(torch.nn.Module):
    """GCN layer: H' = A_hat (H W) + bias, A_hat the normalised adjacency
    D^-1/2 (A + I) D^-1/2 given as `sm` with values `a_values` (fp32 here)."""

    def __init__(self, sm: SparseMatrix, a_values: torch.Tensor, in_dim: int, out_dim: int, bias: bool = True):
        super().__init__()
        self.sm = sm
        self.register_buffer("a_values", a_values)
        self.lin = torch.nn.Linear(in_dim, out_dim, bias=False)
        self.bias = torch.nn.Parameter(torch.zeros(out_dim)) if bias else None

    def forward(self, h: torch.Tensor) -> torch.Tensor:
        out = spmm(self.sm, self.a_values, self.lin(h).to(self.a_values.dtype))
        return out + self.bias if self.bias is not None else out


class SAGEMeanConv(torch.nn.Module):
    """GraphSAGE (mean aggregator): H' = W_self H + W_neigh (A_mean H), A_mean
    the row-normalised adjacency (values 1/deg) given as `sm`, `a_values`."""

    def __init__(self, sm: SparseMatrix, a_values: torch.Tensor, in_dim: int, out_dim: int):
        super().__init__()
        self.sm = sm
        self.register_buffer("a_values", a_values)
        self.lin_self = torch.nn.Linear(in_dim, out_dim)
        self.lin_neigh = torch.nn.Linear(in_dim, out_dim, bias=False)

    def forward(self, h: torch.Tensor) -> torch.Tensor:
        agg = spmm(self.sm, self.a_values, h.to(self.a_values.dtype))
        return self.lin_self(h) + self.lin_neigh(agg)
