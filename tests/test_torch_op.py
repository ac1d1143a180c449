"""The PyTorch-ROCm operator (spmm_amd.torch_ops): forward and backward against
a plain PyTorch fp32 dense reference, exact cases against the oracle, a
small GCN / GraphSAGE training run, the torch.library registration (schemas,
fake kernels, opcheck, torch.compile) and the one-stream-per-plan guard."""
import numpy as np
import pytest

from conftest import exact_dense, exact_values
from oracle import oracle

import spmm_amd as S


def test_no_cpu_fallback():
    """The operator refuses CPU tensors instead of computing on the host."""
    import torch
    from spmm_amd.torch_ops import SparseMatrix, spmm
    a, _ = S.gen_bernoulli(30, 20, 0.2, seed=1, dtype=S.TCA_F32)
    sm = SparseMatrix(a, device="cpu")
    v = torch.from_numpy(a.values.copy())
    b = torch.zeros(20, 8)
    with pytest.raises(ValueError):
        spmm(sm, v, b)


def _dense_ref(torch, a, values, b):
    """Plain PyTorch fp32 reference of C = A * B, differentiable in values and B."""
    dev = b.device
    rows = torch.from_numpy(np.repeat(np.arange(a.nrow), np.diff(a.rowptr)).astype(np.int64)).to(dev)
    cols = torch.from_numpy(a.colidx.astype(np.int64)).to(dev)
    dense = torch.zeros((a.nrow, a.ncol), dtype=torch.float32, device=dev)
    dense = dense.index_put((rows, cols), values.float())
    return dense @ b.float()


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [S.TCA_F32, S.TCA_F16, S.TCA_BF16])
def test_forward_backward_match_a_dense_fp32_reference(torch_cuda, dtype):
    torch = torch_cuda
    from spmm_amd.torch_ops import TORCH_DTYPES, SparseMatrix, spmm
    tdt = {v: k for k, v in TORCH_DTYPES.items()}[dtype]
    dev = torch.device("cuda:0")
    a, _ = S.gen_bernoulli(300, 200, 0.05, seed=3, dtype=dtype)
    sm = SparseMatrix(a)
    for n in (16, 64, 136):
        v = sm.values_tensor().requires_grad_(True)
        b = torch.randn(200, n, device=dev).to(tdt).requires_grad_(True)
        c = spmm(sm, v, b)
        g = torch.randn_like(c)
        (c * g).sum().backward()
        v2 = v.detach().clone().requires_grad_(True)
        b2 = b.detach().clone().requires_grad_(True)
        c2 = _dense_ref(torch, a, v2, b2)
        (c2 * g).sum().backward()
        tol = 1e-5 if dtype == S.TCA_F32 else 2e-3
        torch.testing.assert_close(c, c2, rtol=tol, atol=tol)
        # gradients are returned in the inputs' dtype
        assert v.grad.dtype == tdt and b.grad.dtype == tdt
        torch.testing.assert_close(v.grad.float(), v2.grad.float(), rtol=2e-2 if dtype != S.TCA_F32 else 1e-5,
                                   atol=2e-2 if dtype != S.TCA_F32 else 1e-4)
        torch.testing.assert_close(b.grad.float(), b2.grad.float(), rtol=2e-2 if dtype != S.TCA_F32 else 1e-5,
                                   atol=2e-2 if dtype != S.TCA_F32 else 1e-4)
    sm.close()


@pytest.mark.gpu
def test_exact_inputs_give_bit_exact_gradients(torch_cuda):
    """With exact-arithmetic inputs the forward output, dB = A^T dC and
    dvalues = SDDMM(dC, B) are bit-equal to the oracle / an fp64 numpy product."""
    torch = torch_cuda
    from spmm_amd.torch_ops import SparseMatrix, spmm
    rng = np.random.default_rng(5)
    dev = torch.device("cuda:0")
    a, _ = S.gen_bernoulli(129, 77, 0.1, seed=4, dtype=S.TCA_F32)
    a = S.CSR(a.nrow, a.ncol, a.rowptr, a.colidx, exact_values(rng, a.nnz), S.TCA_F32)
    n = 72
    bh = exact_dense(rng, (77, n))
    gh = exact_dense(rng, (129, n))
    sm = SparseMatrix(a)
    v = torch.from_numpy(a.values.copy()).to(dev).requires_grad_(True)
    b = torch.from_numpy(bh).to(dev).requires_grad_(True)
    c = spmm(sm, v, b)
    c.backward(torch.from_numpy(gh).to(dev))
    assert np.array_equal(c.detach().cpu().numpy(), oracle.csr_spmm(a.rowptr, a.colidx, a.values, bh))
    dense = S.csr_to_dense(a).astype(np.float64)
    assert np.array_equal(b.grad.cpu().numpy(), (dense.T @ gh.astype(np.float64)).astype(np.float32))
    rows = np.repeat(np.arange(a.nrow), np.diff(a.rowptr))
    want_v = np.einsum("jn,jn->j", gh[rows].astype(np.float64), bh[a.colidx].astype(np.float64))
    assert np.array_equal(v.grad.cpu().numpy(), want_v.astype(np.float32))
    sm.close()


@pytest.mark.gpu
def test_gcn_and_sage_layers_train(torch_cuda):
    """A 2-layer GCN and a GraphSAGE-mean layer on an R-MAT graph: forward
    matches the dense reference and a few Adam steps lower the loss."""
    torch = torch_cuda
    from spmm_amd.torch_ops import GCNConv, SAGEMeanConv, SparseMatrix
    torch.manual_seed(0)
    dev = torch.device("cuda:0")
    a_gcn, _ = S.gen_rmat(10, 1000, 6000, norm=0, seed=2)     # D^-1/2 (A + I) D^-1/2
    a_sage, _ = S.gen_rmat(10, 1000, 6000, norm=1, seed=2)    # 1 / deg
    x = torch.randn(1000, 32, device=dev)
    y = torch.randint(0, 4, (1000,), device=dev)
    for a, kind in ((a_gcn, "gcn"), (a_sage, "sage")):
        sm = SparseMatrix(a)
        vals = sm.values_tensor()
        if kind == "gcn":
            model = torch.nn.Sequential(GCNConv(sm, vals, 32, 16), torch.nn.ReLU(), GCNConv(sm, vals, 16, 4)).to(dev)
            ref = _dense_ref(torch, a, vals, model[0].lin(x)) + model[0].bias
            torch.testing.assert_close(model[0](x), ref, rtol=1e-5, atol=1e-5)
        else:
            model = SAGEMeanConv(sm, vals, 32, 4).to(dev)
            ref = model.lin_self(x) + model.lin_neigh(_dense_ref(torch, a, vals, x))
            torch.testing.assert_close(model(x), ref, rtol=1e-5, atol=1e-5)
        opt = torch.optim.Adam(model.parameters(), lr=0.02)
        losses = []
        for _ in range(30):
            opt.zero_grad()
            loss = torch.nn.functional.cross_entropy(model(x), y)
            loss.backward()
            opt.step()
            losses.append(loss.item())
        assert losses[-1] < losses[0] * 0.9, (kind, losses[0], losses[-1])
        sm.close()


# ------------------------------------------------ torch.library registration
def test_ops_are_registered_with_torch_library():
    """spmm, spmm_t and sddmm are torch.library ops of namespace spmm_amd
    with plain int / tensor schemas."""
    import torch
    import spmm_amd.torch_ops  # noqa: F401  (registers the ops)
    schemas = {name: str(getattr(torch.ops.spmm_amd, name).default._schema) for name in ("spmm", "spmm_t", "sddmm")}
    assert schemas["spmm"] == "spmm_amd::spmm(SymInt handle, Tensor values, Tensor b) -> Tensor"
    assert schemas["spmm_t"] == "spmm_amd::spmm_t(SymInt handle, Tensor values, Tensor g) -> Tensor"
    assert schemas["sddmm"] == "spmm_amd::sddmm(SymInt handle, Tensor g, Tensor b) -> Tensor"


def test_fake_kernels_give_output_shapes_without_a_gpu():
    """The fake kernels (what torch.compile traces with) give each op's output
    shape and dtype from the SparseMatrix handle alone: on meta tensors and
    under FakeTensorMode, no kernel runs."""
    import torch
    from torch._subclasses.fake_tensor import FakeTensorMode
    from spmm_amd.torch_ops import SparseMatrix
    a, _ = S.gen_bernoulli(30, 20, 0.2, seed=1, dtype=S.TCA_F16)
    sm = SparseMatrix(a, device="meta")
    v = torch.empty(a.nnz, dtype=torch.float16, device="meta")
    b = torch.empty(20, 8, dtype=torch.float16, device="meta")
    g = torch.empty(30, 8, dtype=torch.float32, device="meta")
    c = torch.ops.spmm_amd.spmm(sm.handle, v, b)
    assert c.shape == (30, 8) and c.dtype == torch.float32 and c.device.type == "meta"
    assert torch.ops.spmm_amd.spmm_t(sm.handle, v, g).shape == (20, 8)
    assert torch.ops.spmm_amd.sddmm(sm.handle, g, b).shape == (a.nnz,)
    with FakeTensorMode():
        fv = torch.empty(a.nnz, dtype=torch.float16)
        fb = torch.empty(20, 40, dtype=torch.float16)
        fc = torch.ops.spmm_amd.spmm(sm.handle, fv, fb)
        assert fc.shape == (30, 40) and fc.dtype == torch.float32
    sm.close()


def test_closed_matrix_handle_is_rejected():
    import torch
    from spmm_amd.torch_ops import SparseMatrix, lookup
    a, _ = S.gen_bernoulli(10, 10, 0.3, seed=2, dtype=S.TCA_F32)
    sm = SparseMatrix(a, device="meta")
    assert lookup(sm.handle) is sm
    sm.close()
    with pytest.raises(ValueError, match="no open SparseMatrix"):
        torch.ops.spmm_amd.spmm(sm.handle, torch.empty(a.nnz, device="meta"), torch.empty(10, 4, device="meta"))


@pytest.mark.gpu
def test_registered_op_forward_backward_bit_exact(torch_cuda):
    """torch.ops.spmm_amd.spmm called directly: forward and both gradients
    bit-equal to the oracle / fp64 products on exact-arithmetic inputs, and
    torch.library.opcheck passes (schema, fake kernel, autograd registration)."""
    torch = torch_cuda
    from spmm_amd.torch_ops import SparseMatrix
    rng = np.random.default_rng(15)
    dev = torch.device("cuda:0")
    a, _ = S.gen_bernoulli(150, 90, 0.08, seed=6, dtype=S.TCA_F32)
    a = S.CSR(a.nrow, a.ncol, a.rowptr, a.colidx, exact_values(rng, a.nnz), S.TCA_F32)
    n = 40
    bh = exact_dense(rng, (90, n))
    gh = exact_dense(rng, (150, n))
    sm = SparseMatrix(a)
    v = torch.from_numpy(a.values.copy()).to(dev).requires_grad_(True)
    b = torch.from_numpy(bh).to(dev).requires_grad_(True)
    c = torch.ops.spmm_amd.spmm(sm.handle, v, b)
    c.backward(torch.from_numpy(gh).to(dev))
    assert np.array_equal(c.detach().cpu().numpy(), oracle.csr_spmm(a.rowptr, a.colidx, a.values, bh))
    dense = S.csr_to_dense(a).astype(np.float64)
    assert np.array_equal(b.grad.cpu().numpy(), (dense.T @ gh.astype(np.float64)).astype(np.float32))
    rows = np.repeat(np.arange(a.nrow), np.diff(a.rowptr))
    want_v = np.einsum("jn,jn->j", gh[rows].astype(np.float64), bh[a.colidx].astype(np.float64))
    assert np.array_equal(v.grad.cpu().numpy(), want_v.astype(np.float32))
    args = (sm.handle, v.detach().requires_grad_(True), b.detach().requires_grad_(True))
    torch.library.opcheck(torch.ops.spmm_amd.spmm.default, args,
                          test_utils=("test_schema", "test_autograd_registration", "test_faketensor"))
    sm.close()


@pytest.mark.gpu
def test_gcn_layer_under_torch_compile(torch_cuda):
    """A 2-layer GCN compiled with torch.compile (fullgraph: the op is one
    opaque node, traced through its fake kernel; backend aot_eager, so
    dynamo and AOTAutograd trace the forward and the registered backward
    and no code is generated) gives the eager model's output and gradients."""
    torch = torch_cuda
    from spmm_amd.torch_ops import GCNConv, SparseMatrix
    torch.manual_seed(1)
    dev = torch.device("cuda:0")
    a, _ = S.gen_rmat(9, 512, 3000, norm=0, seed=3)
    sm = SparseMatrix(a)
    vals = sm.values_tensor()
    model = torch.nn.Sequential(GCNConv(sm, vals, 32, 16), torch.nn.ReLU(), GCNConv(sm, vals, 16, 4)).to(dev)
    x = torch.randn(512, 32, device=dev)
    compiled = torch.compile(model, fullgraph=True, backend="aot_eager")
    out_e = model(x)
    out_e.square().sum().backward()
    grads_e = [p.grad.clone() for p in model.parameters()]
    model.zero_grad()
    out_c = compiled(x)
    out_c.square().sum().backward()
    torch.testing.assert_close(out_c, out_e, rtol=1e-5, atol=1e-5)
    for p, ge in zip(model.parameters(), grads_e):
        torch.testing.assert_close(p.grad, ge, rtol=1e-4, atol=1e-5)
    sm.close()


@pytest.mark.gpu
def test_plan_in_flight_on_another_stream_raises(torch_cuda):
    """A plan whose run is still queued on one stream cannot be run on a
    second stream (its scratch would be shared): RuntimeError, not a race.
    Once that stream has drained, the second stream may use it."""
    torch = torch_cuda
    from spmm_amd.torch_ops import SparseMatrix, spmm
    dev = torch.device("cuda:0")
    a, _ = S.gen_bernoulli(200, 100, 0.05, seed=8, dtype=S.TCA_F32)
    sm = SparseMatrix(a)
    v = sm.values_tensor()
    b = torch.randn(100, 16, device=dev)
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    want = spmm(sm, v, b)
    torch.cuda.synchronize()
    with torch.cuda.stream(s1):
        torch.cuda._sleep(200_000_000)  # keeps s1 busy (~0.1 s): the run below stays queued
        c1 = spmm(sm, v, b)
    with torch.cuda.stream(s2):
        with pytest.raises(RuntimeError, match="still running on another stream"):
            spmm(sm, v, b)
    s1.synchronize()
    with torch.cuda.stream(s2):
        c2 = spmm(sm, v, b)
    s2.synchronize()
    assert torch.equal(c1, want) and torch.equal(c2, want)
    sm.close()
