"""PyTorch-ROCm operator over the MI355X SpMM, with autograd.

    sm = SparseMatrix(a)                 # structure of A (host CSR), planned lazily per width
    c = spmm(sm, values, b)              # C = A * B, fp32, differentiable in values and B

Forward runs the library's planned SpMM (tca_spmm_run) on the current torch
stream.  Backward:
    dB      = A^T * dC     -- an SpMM with a plan of the transpose (fp32; A's
                              values reordered on the device by tca_gather_values),
    dvalues = SDDMM(dC, B) -- <dC[row(j), :], B[col(j), :]> per nonzero (tca_sddmm).
All three are the library's HIP kernels; torch only supplies device memory
and the stream.  No counterpart in the reference, whose entry point
our_spmm_balanced (src/our_spmm.cuh:4) is forward-only; this is the operator
a GCN / GraphSAGE aggregation (C = A * X with A the normalised adjacency)
calls, forward and backward.

Errors follow the library: TcaError with the library's message.  There is no
CPU fallback: the op needs the HIP library and a GPU.
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import (CSR, TCA_BF16, TCA_F16, TCA_F32, TCA_PLAN_DEFAULT, Plan, _addr, call, np_ptr)

__all__ = ["SparseMatrix", "spmm", "GCNConv", "SAGEMeanConv", "TORCH_DTYPES"]

TORCH_DTYPES = {torch.float16: TCA_F16, torch.bfloat16: TCA_BF16, torch.float32: TCA_F32}


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


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

    def close(self) -> None:
        for p in list(self._plans.values()) + list(self._plans_t.values()):
            p.close()
        self._plans.clear()
        self._plans_t.clear()


def _check(sm: SparseMatrix, values: torch.Tensor, b: torch.Tensor):
    if values.device.type != "cuda" or b.device.type != "cuda":
        raise ValueError("spmm: values and B must be GPU tensors (no CPU fallback)")
    if TORCH_DTYPES.get(values.dtype) != sm.dtype or TORCH_DTYPES.get(b.dtype) != sm.dtype:
        raise TypeError(f"spmm: values and B must have A's dtype ({sm.dtype}); got {values.dtype}, {b.dtype}")
    if values.dim() != 1 or values.numel() != sm.nnz:
        raise ValueError(f"spmm: values must be 1-D with {sm.nnz} entries")
    if b.dim() != 2 or b.shape[0] != sm.shape[1]:
        raise ValueError(f"spmm: B must be {sm.shape[1]} x N, got {tuple(b.shape)}")


class _SpMM(torch.autograd.Function):
    @staticmethod
    def forward(ctx, values, b, sm):
        _check(sm, values, b)
        values = values.contiguous()
        b = b.contiguous()
        n = b.shape[1]
        c = torch.empty((sm.shape[0], n), dtype=torch.float32, device=b.device)
        sm.plan(n).run(values, b, c, stream=_stream())
        ctx.sm = sm
        ctx.save_for_backward(values, b)
        return c

    @staticmethod
    def backward(ctx, gc):
        sm = ctx.sm
        values, b = ctx.saved_tensors
        gc = gc.contiguous().to(torch.float32)
        n = b.shape[1]
        grad_values = grad_b = None
        if ctx.needs_input_grad[1]:
            vt = torch.empty(sm.nnz, dtype=torch.float32, device=b.device)
            call("tca_gather_values", _addr(sm.perm), sm.nnz, _addr(values), sm.dtype, _addr(vt), _stream())
            gb = torch.empty((sm.shape[1], n), dtype=torch.float32, device=b.device)
            sm.plan_t(n).run(vt, gc, gb, stream=_stream())
            grad_b = gb.to(b.dtype)
        if ctx.needs_input_grad[0]:
            gv = torch.empty(sm.nnz, dtype=torch.float32, device=b.device)
            call("tca_sddmm", sm.plan(n)._p, _addr(gc), _addr(b), _addr(gv), _stream())
            grad_values = gv.to(values.dtype)
        return grad_values, grad_b, None


def spmm(sm: SparseMatrix, values: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """C = A * B (fp32 result) with A's structure from `sm` and its values
    `values`; differentiable in `values` and `b`."""
    return _SpMM.apply(values, b, sm)


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
