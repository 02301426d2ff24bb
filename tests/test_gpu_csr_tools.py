"""Device-side CSR tooling against the oracle: dense -> CSR (the reference's
host dense2csr rule, src/host/csr_utils.cpp:70-111, bit-exact arrays), the
longest row, int64 -> int32 index narrowing, and torch.sparse_csr input to
the SpMM with no host sync."""
import numpy as np
import pytest
import torch

import torch_csrspmm as tc
import oracle
from csrspmm_amd import capi

pytestmark = pytest.mark.gpu


def special_dense(M, K, density, rng):
    D = rng.uniform(-1, 1, (M, K)).astype(np.float32)
    D[rng.random((M, K)) > density] = 0.0
    flat = D.reshape(-1)
    picks = rng.choice(flat.size, size=min(flat.size, 40), replace=False)
    specials = np.array([-0.0, np.nan, np.inf, -np.inf, 1e-30, -1e-30, 0.25, -0.25], np.float32)
    flat[picks] = specials[np.arange(picks.size) % specials.size]
    if M > 3:
        D[3, :] = 0.0  # an empty row
    return D


@pytest.mark.parametrize("M,K,density,tol", [
    (1, 1, 1.0, 0.0), (7, 63, 0.5, 0.0), (40, 65, 0.3, 0.0), (33, 200, 0.2, 0.25),
    (20000, 9, 0.6, 0.0),   # > 4096 rows: several scan steps
    (300, 5000, 0.01, 0.0), (5, 0, 0.0, 0.0),
])
def test_dense2csr_matches_oracle(M, K, density, tol, gpu):
    rng = np.random.default_rng(M * 31 + K)
    D = special_dense(M, K, density, rng) if K > 0 else np.zeros((M, 0), np.float32)
    rp, ci, va, mx = oracle.dense2csr(D, tol)
    drp, dci, dva = capi.dense2csr(torch.from_numpy(D).to(gpu), tol)
    assert np.array_equal(drp.cpu().numpy(), rp)
    assert np.array_equal(dci.cpu().numpy(), ci)
    assert np.array_equal(dva.cpu().numpy().view(np.uint32), va.view(np.uint32))
    assert int(capi.max_row_nnz(drp).item()) == mx
    # the torch entry gives the same arrays, also from a padded row-major view
    Dp = torch.zeros((M, K + 5), device=gpu)
    Dp[:, :K] = torch.from_numpy(D).to(gpu)
    t_rp, t_ci, t_va = tc.dense_to_csr(Dp[:, :K], tol)
    assert torch.equal(t_rp.cpu(), torch.from_numpy(rp))
    assert torch.equal(t_ci.cpu(), torch.from_numpy(ci))
    assert np.array_equal(t_va.cpu().numpy().view(np.uint32), va.view(np.uint32))


def test_max_row_nnz_without_sync(gpu):
    rng = np.random.default_rng(2)
    lens = rng.integers(0, 3000, 100000)
    lens[12345] = 77777
    rp = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    out = tc.csr_max_row_nnz(torch.from_numpy(rp).to(gpu))
    assert out.is_cuda and out.dtype == torch.int32 and int(out.item()) == 77777
    assert int(tc.csr_max_row_nnz(torch.zeros(1, dtype=torch.int32, device=gpu)).item()) == 0


def test_narrow_indices_and_overflow_flag(gpu):
    src = torch.tensor([0, 5, 2**31 - 1, -7, 123456789], dtype=torch.int64, device=gpu)
    dst, flag = capi.narrow_indices(src)
    assert dst.tolist() == [0, 5, 2**31 - 1, -7, 123456789] and int(flag.item()) == 0
    big = torch.arange(100000, dtype=torch.int64, device=gpu)
    big[77] = 2**31
    dst, flag = capi.narrow_indices(big)
    assert int(flag.item()) == 1
    assert dst[:77].tolist() == list(range(77))


@pytest.mark.filterwarnings("ignore:Sparse CSR tensor support")
@pytest.mark.parametrize("index_dtype", [torch.int64, torch.int32])
def test_sparse_csr_input(index_dtype, gpu):
    rng = np.random.default_rng(9)
    M, K, N = 3000, 2000, 96
    D = rng.uniform(-1, 1, (M, K)).astype(np.float32)
    D[rng.random((M, K)) > 0.02] = 0.0
    D[5, :] = rng.uniform(-1, 1, K)  # one long row (split path)
    Dt = torch.from_numpy(D).to(gpu)
    A = Dt.to_sparse_csr()
    if index_dtype == torch.int32:
        A = torch.sparse_csr_tensor(A.crow_indices().to(torch.int32),
                                    A.col_indices().to(torch.int32), A.values(), A.shape)
    B = rng.uniform(-1, 1, (K, N)).astype(np.float32)
    rowptr, colidx, vals, K2 = tc.from_sparse_csr(A)
    assert K2 == K and rowptr.dtype == torch.int32 and colidx.dtype == torch.int32
    if index_dtype == torch.int32:  # zero-copy
        assert rowptr.data_ptr() == A.crow_indices().data_ptr()
        assert colidx.data_ptr() == A.col_indices().data_ptr()
    C = tc.csrspmm_sparse(A, torch.from_numpy(B).to(gpu), 0.5, 2.0)
    rp, ci, va, _ = oracle.dense2csr(D, 0.0)
    R, S = oracle.spmm_f64(rp, ci, va, B, None, 0.5, 2.0, c0_zero=True)
    bad, ratio, _, _ = oracle.check(C.cpu().numpy(), R, S, 1e-5)
    assert bad == 0, ratio
    with pytest.raises(RuntimeError, match="torch.sparse_csr"):
        tc.from_sparse_csr(Dt)
