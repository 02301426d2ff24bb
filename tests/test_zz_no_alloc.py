"""csrspmm_spmm_f32_noalloc through the C ABI: its output against
csrspmm_spmm_f32_ex's on the same inputs (bit for bit: the same kernels on
the same workspace layout) and against the oracle, on two calls in a row, the
second with a smaller input, so that the second call runs on a scratch the
first one left full; device memory unchanged across calls; a problem whose
base workspace exceeds the 128 MiB scratch rejected before anything runs."""
import numpy as np
import pytest
import torch

import oracle
from csrspmm_amd import capi, configs, gen

pytestmark = pytest.mark.gpu

SCRATCH_TOO_SMALL = -6


def upload(gpu, a, B):
    t = lambda x: torch.from_numpy(x).to(gpu)  # noqa: E731
    return t(a.rowptr), t(a.colidx), t(a.vals), t(B)


def sample_rows(a, every):
    longest = np.argsort(np.diff(a.rowptr))[-64:]
    return np.unique(np.concatenate([longest, np.arange(0, a.M, every)])).astype(np.int32)


def run_pair(algo, a, B, d, C0, alpha, beta, hint=-1):
    """(noalloc output, _ex output) of one product, C starting from C0."""
    rp, ci, va, dB = d
    C_na = C0.clone()
    C_ex = C0.clone()
    capi.spmm(algo, rp, ci, va, dB, C_na, alpha, beta, hint=hint, noalloc=True)
    capi.spmm(algo, rp, ci, va, dB, C_ex, alpha, beta, hint=hint)
    torch.cuda.synchronize()
    return C_na, C_ex


@pytest.mark.parametrize("algo", ["Auto", "WarpPerRowFp4", "WarpPerRowSmem", "Naive"])
def test_noalloc_matches_ex_on_two_calls(algo, gpu):
    big = configs.CONFIGS["xl"]
    a1 = big.csr()
    B1 = big.B(a1.K)
    a2 = gen.ragged(5000, 3000, 0, 700, seed=77)  # smaller: empty, short and split rows
    B2 = gen.dense(77, gen.TAG_B, a2.K, 64)
    cases = [(a1, B1, 1.0, 0.0), (a2, B2, 0.5, -2.0)]
    for i, (a, B, alpha, beta) in enumerate(cases):
        d = upload(gpu, a, B)
        N = B.shape[1]
        C0 = torch.from_numpy(gen.dense(5 + i, gen.TAG_C0, a.M, N)).to(gpu)
        C_na, C_ex = run_pair(algo, a, B, d, C0, alpha, beta)
        assert torch.equal(C_na, C_ex), f"{algo} call {i + 1}: noalloc differs from _ex"
        rows = sample_rows(a, 97 if a.M > 100000 else 1)
        R, S = oracle.spmm_f64(a.rowptr, a.colidx, a.vals, B, C0.cpu().numpy(), alpha, beta,
                               rows=rows)
        bad, ratio, _, _ = oracle.check(C_na.cpu().numpy()[rows], R, S, 1e-5)
        assert bad == 0, f"{algo} call {i + 1}: {bad} elements off, max ratio {ratio}"


def test_noalloc_allocates_nothing(gpu):
    a = gen.ragged(20000, 8000, 0, 3000, seed=78)
    B = gen.dense(78, gen.TAG_B, a.K, 128)
    d = upload(gpu, a, B)
    C = torch.empty(a.M, 128, device=gpu)
    algos = ("Auto", "WarpPerRow", "WarpPerRowSmemFp4", "NaiveSmem")
    # first calls: the scratch's address lookup and the lazy loading of each
    # kernel's code object happen here, outside the measured window
    for algo in algos:
        capi.spmm(algo, *d[:3], d[3], C, 1.0, 0.0, noalloc=True)
    torch.cuda.synchronize()
    free0, _ = torch.cuda.mem_get_info()
    reserved0 = torch.cuda.memory_reserved()
    for _ in range(3):
        for algo in algos:
            capi.spmm(algo, *d[:3], d[3], C, 1.0, 0.0, noalloc=True)
    torch.cuda.synchronize()
    free1, _ = torch.cuda.mem_get_info()
    assert free1 == free0 and torch.cuda.memory_reserved() == reserved0


def test_noalloc_rejects_beyond_scratch(gpu):
    """Base workspace above 128 MiB (segment partials of 8M nonzeros x 1100
    columns): rejected, C untouched."""
    M, K, N, nnz = 1024, 1, 1100, 8_000_000
    lib = capi.hip()
    assert lib.csrspmm_workspace_bytes(capi.ALGO["Auto"], M, N, nnz) > 128 << 20
    rowptr = (torch.arange(M + 1, dtype=torch.int64, device=gpu) * nnz // M).to(torch.int32)
    colidx = torch.zeros(nnz, dtype=torch.int32, device=gpu)
    vals = torch.ones(nnz, device=gpu)
    B = torch.ones(K, N, device=gpu)
    C = torch.full((M, N), 7.0, device=gpu)
    with pytest.raises(capi.CsrspmmError) as e:
        capi.spmm("Auto", rowptr, colidx, vals, B, C, 1.0, 0.0, noalloc=True)
    assert e.value.status == SCRATCH_TOO_SMALL
    assert "no-allocation scratch" in str(e.value)
    torch.cuda.synchronize()
    assert bool((C == 7.0).all())


def test_noalloc_hinted_one_launch(gpu):
    """A max_row_nnz hint that makes a mid-sized call one launch (rows of at
    most 256, M < 32768, no column slices) needs no workspace, even where
    the unhinted plan's partials would exceed the scratch (rows of 200 on
    1024 x 256 with N = 16384: segments of 32, 419 MB of partials): the call
    runs, bit for bit as _ex, within the bar of the oracle, twice in a row."""
    M, K, N = 1024, 256, 16384
    a = gen.uniform(M, K, 200, 23)
    lib = capi.hip()
    assert lib.csrspmm_workspace_bytes(capi.ALGO["Auto"], M, N, a.nnz) > 128 << 20
    assert lib.csrspmm_workspace_bytes_ex(capi.ALGO["Auto"], M, K, N, a.nnz, 200) == 0
    B = gen.dense(23, gen.TAG_B, K, N)
    d = upload(gpu, a, B)
    C0 = torch.zeros((M, N), device=gpu)
    rows = np.arange(0, M, 16).astype(np.int32)
    R, S = oracle.spmm_f64(a.rowptr, a.colidx, a.vals, B, None, 1.0, 0.0, rows=rows)
    for _ in range(2):
        C_na, C_ex = run_pair("Auto", a, B, d, C0, 1.0, 0.0, hint=200)
        assert torch.equal(C_na, C_ex)
        bad, ratio, _, _ = oracle.check(C_na.cpu().numpy()[rows], R, S, 1e-5)
        assert bad == 0, f"max ratio {ratio}"
