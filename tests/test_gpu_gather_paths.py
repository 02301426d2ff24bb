"""The two ways the warp-per-row kernels gather B (rowgroup.hip): through a
buffer resource with 32-bit offsets (row * ldb * 4 computed by one
v_mad_u32_u24), taken whenever B's rows and row stride fit 24 bits and its
extent stays below 3 GiB (buf_gathers_ok), and 64-bit global loads
otherwise.  The parity tests run the first; these shapes force the second,
by a row stride of more than 2^22 floats and by more than 2^24 rows of B,
and check every variant against the oracle on every row."""
import numpy as np
import pytest
import torch

import oracle
from csrspmm_amd import capi

pytestmark = pytest.mark.gpu

ALGOS = ["Auto", "Naive", "NaiveSmem", "WarpPerRow", "WarpPerRowFp4", "WarpPerRowSmem",
         "WarpPerRowSmemFp4"]


def random_csr(M, K, per_row, seed, high=0):
    """Rows of up to per_row distinct sorted columns; with `high`, half of
    each row's columns come from the top `high` rows of B."""
    rng = np.random.default_rng(seed)
    lens = rng.integers(0, per_row + 1, M)
    rowptr = np.zeros(M + 1, dtype=np.int32)
    rowptr[1:] = np.cumsum(lens)
    cols = []
    for n in lens:
        if high:
            lo = rng.choice(K - high, size=n // 2, replace=False)
            hi = K - high + rng.choice(high, size=n - n // 2, replace=False)
            c = np.concatenate([lo, hi])
        else:
            c = rng.choice(K, size=n, replace=False)
        cols.append(np.sort(c).astype(np.int32))
    colidx = np.concatenate(cols)
    vals = rng.uniform(-1, 1, rowptr[-1]).astype(np.float32)
    return rowptr, colidx, vals


def to(gpu, x):
    return torch.from_numpy(np.ascontiguousarray(x)).to(gpu)


def check(C, rp, ci, va, B, alpha, beta, C0, what):
    R, S = oracle.spmm_f64(rp, ci, va, np.ascontiguousarray(B), C0, alpha, beta)
    bad, ratio, _, _ = oracle.check(np.ascontiguousarray(C), R, S, 1e-5)
    assert bad == 0, f"{what}: {bad} elements off, max ratio {ratio}"


@pytest.mark.parametrize("algo", ALGOS)
def test_row_stride_beyond_24_bits(algo, gpu):
    """B = the first 128 columns of a [16, 2^22 + 128] tensor: a row stride of
    16 MiB + 512 bytes, beyond the 24-bit offsets of the buffer path.  10000
    rows of up to 16 nonzeros (a planned problem)."""
    K, N, W = 16, 128, (1 << 22) + 128
    M = 10000
    rp, ci, va = random_csr(M, K, 16, 31)
    rng = np.random.default_rng(32)
    Bw = torch.empty((K, W), device=gpu)
    Bsub = rng.uniform(-1, 1, (K, N)).astype(np.float32)
    Bw[:, :N] = to(gpu, Bsub)
    C0 = rng.uniform(-1, 1, (M, N)).astype(np.float32)
    dC = to(gpu, C0)
    capi.spmm(algo, to(gpu, rp), to(gpu, ci), to(gpu, va), Bw[:, :N], dC, 1.25, -0.5)
    torch.cuda.synchronize()
    check(dC.cpu().numpy(), rp, ci, va, Bsub, 1.25, -0.5, C0, f"{algo} ldb {W}")


@pytest.mark.parametrize("algo", ["Auto", "WarpPerRow", "WarpPerRowFp4", "WarpPerRowSmem",
                                  "WarpPerRowSmemFp4"])
def test_more_than_2_pow_24_rows_of_B(algo, gpu):
    """K = 2^24 + 3 rows of B (N = 4, 256 MiB): row indices beyond 24 bits,
    half of every row's columns among the top 1000 rows."""
    K, N, M = (1 << 24) + 3, 4, 6000
    rp, ci, va = random_csr(M, K, 24, 33, high=1000)
    rng = np.random.default_rng(34)
    B = rng.uniform(-1, 1, (K, N)).astype(np.float32)
    dC = torch.zeros((M, N), device=gpu)
    capi.spmm(algo, to(gpu, rp), to(gpu, ci), to(gpu, va), to(gpu, B), dC, 1.0, 0.0)
    torch.cuda.synchronize()
    check(dC.cpu().numpy(), rp, ci, va, B, 1.0, 0.0, None, f"{algo} K {K}")
