"""Operands that are one-column (or one-row) views of wider tensors, through
every surface that derives a leading dimension from a tensor: the five torch
forwards and csrspmm_auto (B), csrspmm_spmm_out and CsrSpmmPlan (B and C),
dense_to_csr (the dense input), and the ctypes view of the C ABI.  A view
X[:, k:k+1] of a [R, W] tensor has strides (W, 1): its rows are W floats
apart, and the product must read (or write) exactly those elements, leaving
the parent's other columns untouched.  Checked against the oracle.

The shapes the reference derives are kept (torch_csrspmm/torch_csrspmm_naive.cpp:27-46:
M = rowptr.size(0) - 1, K = B.size(0), N = B.size(1)); its forwards ignore
strides, this surface honours them."""
import numpy as np
import pytest
import torch

import torch_csrspmm as tc
import oracle
from csrspmm_amd import capi

pytestmark = pytest.mark.gpu

NAMES = ["csrspmm_naive", "csrspmm_warp_per_row", "csrspmm_warp_per_row_smem",
         "csrspmm_warp_per_row_fp4", "csrspmm_warp_per_row_smem_fp4", "csrspmm_auto"]


def call(name, rp, ci, va, mx, B, alpha, beta):
    fn = getattr(tc, name)
    if "smem" in name:
        return fn(rp, ci, va, mx, B, alpha, beta)
    return fn(rp, ci, va, B, alpha, beta)


def csr(M, K, density, seed):
    rng = np.random.default_rng(seed)
    dense = rng.uniform(-1, 1, (M, K)).astype(np.float32) * (rng.random((M, K)) < density)
    return oracle.dense2csr(dense, 0.0)


def to(gpu, x):
    return torch.from_numpy(np.ascontiguousarray(x)).to(gpu)


def expect(C, rp, ci, va, B, alpha=1.0, beta=0.0, C0=None, c0_zero=False, what=""):
    R, S = oracle.spmm_f64(rp, ci, va, np.ascontiguousarray(B), C0, alpha, beta, c0_zero=c0_zero)
    bad, ratio, _, _ = oracle.check(np.ascontiguousarray(C), R, S, 1e-5)
    assert bad == 0, f"{what}: {bad} elements off, max ratio {ratio}"


# Small (one launch, no plan) and planned (M + nnz >= 65536: plan, segments,
# combine) problems.
SHAPES = [(70, 40, 0.3), (3000, 600, 0.04)]


@pytest.mark.parametrize("name", NAMES)
@pytest.mark.parametrize("shape", SHAPES, ids=["small", "planned"])
def test_forward_one_column_B_view(name, shape, gpu):
    M, K, dens = shape
    rp, ci, va, mx = csr(M, K, dens, 17)
    X = np.random.default_rng(4).uniform(-1, 1, (K, 5)).astype(np.float32)
    dX = to(gpu, X)
    for k in (0, 3, 4):
        Bv = dX[:, k:k + 1]
        assert Bv.stride() == (5, 1)
        C = call(name, to(gpu, rp), to(gpu, ci), to(gpu, va), mx, Bv, 1.25, 0.0)
        assert C.shape == (M, 1)
        expect(C.cpu().numpy(), rp, ci, va, X[:, k:k + 1], 1.25, 0.0, what=f"{name} column {k}")


@pytest.mark.parametrize("algo", ["Auto", "Naive", "NaiveSmem", "WarpPerRow", "WarpPerRowFp4",
                                  "WarpPerRowSmem", "WarpPerRowSmemFp4"])
@pytest.mark.parametrize("shape", SHAPES, ids=["small", "planned"])
def test_spmm_out_one_column_C_view(algo, shape, gpu):
    """C = Y[:, j:j+1] of a [M, 4] tensor: the product lands in column j and
    the other three columns keep their bits; B is a one-column view too."""
    M, K, dens = shape
    rp, ci, va, _ = csr(M, K, dens, 23)
    rng = np.random.default_rng(8)
    X = rng.uniform(-1, 1, (K, 3)).astype(np.float32)
    Y = rng.uniform(-1, 1, (M, 4)).astype(np.float32)
    dX, dY = to(gpu, X), to(gpu, Y)
    for j, k in ((1, 2), (3, 0)):
        Cv = dY[:, j:j + 1]
        assert Cv.stride() == (4, 1)
        before = dY.clone()
        out = tc.csrspmm_spmm_out(to(gpu, rp), to(gpu, ci), to(gpu, va), dX[:, k:k + 1], Cv,
                                  0.5, -1.5, algo=algo)
        assert out.data_ptr() == Cv.data_ptr()
        got = dY.cpu().numpy()
        expect(got[:, j:j + 1], rp, ci, va, X[:, k:k + 1], 0.5, -1.5,
               C0=before.cpu().numpy()[:, j:j + 1], what=f"spmm_out {algo} C[:, {j}]")
        others = [c for c in range(4) if c != j]
        assert torch.equal(dY[:, others], before[:, others]), f"{algo}: other columns changed"


def test_plan_one_column_views(gpu):
    M, K, dens = SHAPES[1]
    rp, ci, va, _ = csr(M, K, dens, 29)
    rng = np.random.default_rng(9)
    X = rng.uniform(-1, 1, (K, 6)).astype(np.float32)
    Y = rng.uniform(-1, 1, (M, 3)).astype(np.float32)
    dX, dY = to(gpu, X), to(gpu, Y)
    for algo in ("Auto", "WarpPerRowFp4", "Naive"):
        plan = tc.CsrSpmmPlan(to(gpu, rp), to(gpu, ci), to(gpu, va), K, algo=algo, n_hint=1)
        C = plan.spmm(dX[:, 5:6], 2.0, 0.0)
        expect(C.cpu().numpy(), rp, ci, va, X[:, 5:6], 2.0, 0.0, what=f"plan.spmm {algo}")
        before = dY.clone()
        plan.spmm_out(dX[:, 1:2], dY[:, 0:1], 1.0, 0.25)
        expect(dY.cpu().numpy()[:, 0:1], rp, ci, va, X[:, 1:2], 1.0, 0.25,
               C0=before.cpu().numpy()[:, 0:1], what=f"plan.spmm_out {algo}")
        assert torch.equal(dY[:, 1:], before[:, 1:])


def test_dense_to_csr_one_column_view(gpu):
    """K = 1: a column of a wider dense tensor, through the torch entry point
    and the C ABI, bit-exact against the oracle's dense2csr."""
    rng = np.random.default_rng(12)
    D = rng.uniform(-1, 1, (500, 7)).astype(np.float32)
    D[rng.random((500, 7)) < 0.5] = 0.0
    dD = to(gpu, D)
    for k in (0, 6):
        want = oracle.dense2csr(np.ascontiguousarray(D[:, k:k + 1]), 0.0)
        for got in (tc.dense_to_csr(dD[:, k:k + 1]), capi.dense2csr(dD[:, k:k + 1])):
            for g, w in zip(got, want[:3]):
                assert np.array_equal(g.cpu().numpy(), w), f"column {k}"


@pytest.mark.parametrize("algo", ["Auto", "Naive", "WarpPerRow", "WarpPerRowSmemFp4"])
def test_capi_one_column_views(algo, gpu):
    """The ctypes view of the C ABI: B and C one-column views, and a plan."""
    M, K, dens = SHAPES[1]
    rp, ci, va, _ = csr(M, K, dens, 31)
    rng = np.random.default_rng(10)
    X = rng.uniform(-1, 1, (K, 4)).astype(np.float32)
    Y = rng.uniform(-1, 1, (M, 2)).astype(np.float32)
    dX, dY = to(gpu, X), to(gpu, Y)
    before = dY.clone()
    capi.spmm(algo, to(gpu, rp), to(gpu, ci), to(gpu, va), dX[:, 2:3], dY[:, 1:2], 1.0, 0.5)
    torch.cuda.synchronize()
    expect(dY.cpu().numpy()[:, 1:2], rp, ci, va, X[:, 2:3], 1.0, 0.5,
           C0=before.cpu().numpy()[:, 1:2], what=f"capi.spmm {algo}")
    assert torch.equal(dY[:, 0], before[:, 0])
    plan = capi.Plan(algo, to(gpu, rp), to(gpu, ci), to(gpu, va), K)
    before = dY.clone()
    plan.spmm(dX[:, 0:1], dY[:, 0:1], 1.0, 0.0)
    torch.cuda.synchronize()
    expect(dY.cpu().numpy()[:, 0:1], rp, ci, va, X[:, 0:1], what=f"capi.Plan {algo}")
    assert torch.equal(dY[:, 1], before[:, 1])
    plan.close()


def test_overlapping_rows_rejected(gpu):
    rp = torch.tensor([0, 1, 2], dtype=torch.int32, device=gpu)
    ci = torch.tensor([0, 1], dtype=torch.int32, device=gpu)
    va = torch.ones(2, device=gpu)
    Bx = torch.ones(1, 4, device=gpu).expand(2, 4)  # stride (0, 1)
    with pytest.raises(RuntimeError, match="row stride"):
        tc.csrspmm_warp_per_row(rp, ci, va, Bx, 1.0, 0.0)
    Cx = torch.zeros(1, 4, device=gpu).expand(2, 4)
    with pytest.raises(RuntimeError, match="row stride"):
        tc.csrspmm_spmm_out(rp, ci, va, torch.ones(2, 4, device=gpu), Cx, 1.0, 0.0)
    with pytest.raises(ValueError, match="row stride"):
        capi.spmm("Auto", rp, ci, va, Bx, torch.zeros(2, 4, device=gpu), 1.0, 0.0)
