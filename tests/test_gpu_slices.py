"""GPU parity of column slices.

On a B much larger than the L2s (>= 32 MiB, a 64-column band of <= 16 MiB
or a B of >= 1 GiB) with N >= 256 (or N = 128 when no column panels apply),
a warp-per-row call runs its main work as ceil(N / 64) column slices, one
launch per slice (>= 32 nonzeros per row on average) or all in one launch in
slice order (sparser rows), sharing the plan and the combine.  These
tests cover a last partial slice, long rows on segments, the beta epilogue,
padded leading dimensions and the scalar-column kernels, against the fp64
oracle at the 1e-5 bar and bitwise against the fp32 CSR-order restatement on
the rows summed whole (csr_cases.whole_row_max).
"""
import numpy as np
import pytest
import torch

import oracle
from csrspmm_amd import ALGORITHMS, capi, gen
from csr_cases import csr_from_lengths, mixed_lengths, whole_row_limit, whole_row_max

pytestmark = pytest.mark.gpu

TOL = 1e-5
ROWGROUP = ["WarpPerRow", "WarpPerRowFp4", "WarpPerRowSmem", "WarpPerRowSmemFp4", "Auto"]


def check(algo, C, rowptr, colidx, vals, B, C0=None, alpha=1.0, beta=0.0, what=""):
    assert not np.isnan(C).any(), f"{algo} {what}: unwritten output"
    R, S = oracle.spmm_f64(rowptr, colidx, vals, B, C0, alpha, beta)
    bad, ratio, _, _ = oracle.check(C, R, S, TOL)
    assert bad == 0, f"{algo} {what}: {bad} elements off (max ratio {ratio:.3g})"
    F = oracle.spmm_f32_seq(rowptr, colidx, vals, B, C0, alpha, beta)
    whole = np.diff(rowptr) <= whole_row_limit(algo, rowptr, B.shape[0], B.shape[1])
    assert np.array_equal(C[whole].view(np.uint32), F[whole].view(np.uint32)), \
        f"{algo} {what}: short rows differ from the fp32 restatement"


@pytest.mark.parametrize("empty_rows", [0, 6000])
@pytest.mark.parametrize("N", [256, 200, 132, 128])
@pytest.mark.parametrize("algo", ROWGROUP)
def test_slices_mixed_rows(algo, N, empty_rows, gpu):
    # ~52 nonzeros per row: one launch per slice; with 6000 more empty rows
    # (~13 per row): all slices in one launch
    K = 65536  # B of 33-64 MiB, 16 MiB per 64-column band
    lens = np.concatenate([mixed_lengths(90 + N, M=2000), np.zeros(empty_rows, np.int64)])
    np.random.default_rng(N).shuffle(lens)
    rowptr, colidx, vals = csr_from_lengths(lens, K, seed=N)
    B = gen.dense(21, gen.TAG_B, K, N)
    print(f"[slices] {algo} N={N} M={lens.size} nnz={colidx.size}", flush=True)
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(gpu)  # noqa: E731
    dC = torch.full((lens.size, N), float("nan"), device=gpu)
    capi.spmm(algo, t(rowptr), t(colidx), t(vals), t(B), dC, 1.0, 0.0)
    torch.cuda.synchronize()
    C = dC.cpu().numpy()
    check(algo, C, rowptr, colidx, vals, B, what=f"N={N}")
    # the same product through the caller-workspace entry, twice: bit-identical
    C2 = torch.full_like(dC, float("nan"))
    capi.spmm(algo, t(rowptr), t(colidx), t(vals), t(B), C2, 1.0, 0.0)
    capi.spmm(algo, t(rowptr), t(colidx), t(vals), t(B), C2, 1.0, 0.0)
    torch.cuda.synchronize()
    assert np.array_equal(C.view(np.uint32), C2.cpu().numpy().view(np.uint32))


@pytest.mark.parametrize("algo", ["WarpPerRowSmem", "WarpPerRowSmemFp4", "Auto"])
def test_slices_epilogue_and_padded_operands(algo, gpu):
    K, N = 65536, 256
    lens = mixed_lengths(77, M=1200)
    rowptr, colidx, vals = csr_from_lengths(lens, K, seed=77)
    Bw = gen.dense(22, gen.TAG_B, K, N + 8)
    Cw = gen.dense(22, gen.TAG_C0, lens.size, N + 4)
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(gpu)  # noqa: E731
    dB = t(Bw)[:, :N]
    dCw = t(Cw)
    dC = dCw[:, :N]
    capi.spmm(algo, t(rowptr), t(colidx), t(vals), dB, dC, -0.5, 2.0)
    torch.cuda.synchronize()
    out = dCw.cpu().numpy()
    assert np.array_equal(out[:, N:].view(np.uint32), Cw[:, N:].view(np.uint32)), "padding written"
    check(algo, np.ascontiguousarray(out[:, :N]), rowptr, colidx, vals, np.ascontiguousarray(Bw[:, :N]),
          np.ascontiguousarray(Cw[:, :N]), -0.5, 2.0, what="beta != 0, ldb = N + 8, ldc = N + 4")


def test_slices_stored_plan(gpu):
    K, N = 65536, 256
    lens = mixed_lengths(88, M=2500)
    rowptr, colidx, vals = csr_from_lengths(lens, K, seed=88)
    B = gen.dense(23, gen.TAG_B, K, N)
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(gpu)  # noqa: E731
    drp, dci, dv = t(rowptr), t(colidx), t(vals)
    for algo in ("WarpPerRowSmemFp4", "WarpPerRow"):
        plan = capi.Plan(algo, drp, dci, dv, K, n_hint=N)
        dC = torch.full((lens.size, N), float("nan"), device=gpu)
        plan.spmm(t(B), dC, 1.0, 0.0)
        torch.cuda.synchronize()
        check(algo, dC.cpu().numpy(), rowptr, colidx, vals, B, what="stored plan, sliced")
        plan.close()


@pytest.mark.parametrize("per_row", [3, 9, 20, 40, 70])
@pytest.mark.parametrize("algo", ["WarpPerRowFp4", "WarpPerRowSmemFp4"])
def test_sliced_merge_blocks_sized_to_rows(algo, per_row, gpu):
    """A per-call float4 call with slices and fewer than 65536 rows sizes its
    merge blocks from the mean row (16, 16, 16, 32 and 64 items here), and a
    stored plan for that width does the same.  Rows are summed whole, so the
    two agree bit for bit (and with the fp32 restatement), including the
    empty rows spread among them and rows longer than the block."""
    K, N, M = 40000, 256, 20000  # B of 39 MiB: four 64-column slices
    rng = np.random.default_rng(per_row)
    lens = np.minimum(rng.integers(0, 2 * per_row + 1, M), 128).astype(np.int64)  # no long rows
    lens[rng.choice(M, M // 10, replace=False)] = 0
    rowptr, colidx, vals = csr_from_lengths(lens, K, seed=per_row)
    B = gen.dense(24, gen.TAG_B, K, N)
    print(f"[slices] merge blocks {algo} per_row={per_row} nnz={colidx.size}", flush=True)
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(gpu)  # noqa: E731
    drp, dci, dv, dB = t(rowptr), t(colidx), t(vals), t(B)
    dC = torch.full((M, N), float("nan"), device=gpu)
    capi.spmm(algo, drp, dci, dv, dB, dC, 1.0, 0.0)
    plan = capi.Plan(algo, drp, dci, dv, K, n_hint=N)
    dP = torch.full((M, N), float("nan"), device=gpu)
    plan.spmm(dB, dP, 1.0, 0.0)
    torch.cuda.synchronize()
    plan.close()
    C = dC.cpu().numpy()
    check(algo, C, rowptr, colidx, vals, B, what=f"merge blocks, {per_row} per row")
    assert np.array_equal(C.view(np.uint32), dP.cpu().numpy().view(np.uint32)), \
        f"{algo}: per-call and stored-plan results differ"
