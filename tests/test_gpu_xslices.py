"""GPU parity of XCD slices and of the combine's early exit.

XCD slices: a float4 call whose B is larger than one XCD's 4 MiB L2 while
each 64-column band of it fits one (K <= 16384), with 2, 4 or 8 such bands
(N of 65-128, 193-256 or 449-512) and no other column slices, runs all its
bands in one launch with block b on band b mod the band count, so each XCD
gathers from one band (medium, 16384^2 at N = 128, takes this path).  The
cases: two and four bands, a last partial band (N = 124), long rows on
segments and the combine, the beta epilogue, a stored plan, and the scalar
variants on the same shapes (which keep the unsliced path).

A single long row: plan_kernel handles rows in blocks of 256 (grid-strided
past 4096 blocks), zeroing each split row's segment counter and flagging
its block for the combine of a stored plan; per call the row is summed in
the main launch by the wave whose segment counts last.  The cases put the
row in the first, a middle and the last row block, and in a grid-strided
block of a matrix of over 2^20 rows.

Bar: 1e-5 against the fp64 oracle on every element; rows summed whole
(csr_cases.whole_row_max) bit for bit against the fp32 restatement.
"""
import numpy as np
import pytest
import torch

import oracle
from csrspmm_amd import capi, gen
from csr_cases import csr_from_lengths, mixed_lengths, whole_row_limit

pytestmark = pytest.mark.gpu

TOL = 1e-5
ROWGROUP = ["WarpPerRow", "WarpPerRowFp4", "WarpPerRowSmem", "WarpPerRowSmemFp4", "Auto"]


def t(x, dev):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


def run(algo, rowptr, colidx, vals, B, dev, C0=None, alpha=1.0, beta=0.0, hint=-1):
    M, N = rowptr.size - 1, B.shape[1]
    dC = t(C0, dev) if C0 is not None else torch.full((M, N), float("nan"), device=dev)
    capi.spmm(algo, t(rowptr, dev), t(colidx, dev), t(vals, dev), t(B, dev), dC, alpha, beta,
              hint=hint)
    torch.cuda.synchronize()
    return dC.cpu().numpy()


def check(algo, C, rowptr, colidx, vals, B, C0=None, alpha=1.0, beta=0.0, what=""):
    assert not np.isnan(C).any(), f"{algo} {what}: unwritten output"
    R, S = oracle.spmm_f64(rowptr, colidx, vals, B, C0, alpha, beta)
    bad, ratio, _, _ = oracle.check(C, R, S, TOL)
    assert bad == 0, f"{algo} {what}: {bad} elements off (max ratio {ratio:.3g})"
    F = oracle.spmm_f32_seq(rowptr, colidx, vals, B, C0, alpha, beta)
    whole = np.diff(rowptr) <= whole_row_limit(algo, rowptr, B.shape[0], B.shape[1])
    assert np.array_equal(C[whole].view(np.uint32), F[whole].view(np.uint32)), \
        f"{algo} {what}: rows summed whole differ from the fp32 restatement"


@pytest.mark.parametrize("K,N", [(16384, 128), (16384, 124), (16384, 256), (12000, 96)])
@pytest.mark.parametrize("algo", ROWGROUP)
def test_xslices_mixed_rows(algo, K, N, gpu):
    """Short, long and empty rows (segments and the combine) on 2 or 4 bands."""
    lens = np.minimum(mixed_lengths(K + N, M=3000), K)
    rowptr, colidx, vals = csr_from_lengths(lens, K, seed=N)
    B = gen.dense(N, gen.TAG_B, K, N)
    print(f"[xslices] {algo} K={K} N={N} M={lens.size} nnz={colidx.size}", flush=True)
    C = run(algo, rowptr, colidx, vals, B, gpu)
    check(algo, C, rowptr, colidx, vals, B, what=f"K={K} N={N}")
    C2 = run(algo, rowptr, colidx, vals, B, gpu)
    assert np.array_equal(C.view(np.uint32), C2.view(np.uint32)), "not deterministic"


@pytest.mark.parametrize("algo", ["WarpPerRowFp4", "WarpPerRowSmemFp4"])
def test_xslices_short_rows_epilogue(algo, gpu):
    """Rows of 40-90 (no segment, no combine work) with beta, and a stored
    plan of the same product."""
    K, N, M = 16384, 128, 6000
    lens = np.random.default_rng(3).integers(40, 91, M)
    rowptr, colidx, vals = csr_from_lengths(lens, K, seed=3)
    B = gen.dense(3, gen.TAG_B, K, N)
    C0 = gen.dense(3, gen.TAG_C0, M, N)
    C = run(algo, rowptr, colidx, vals, B, gpu, C0=C0, alpha=0.5, beta=-2.0)
    check(algo, C, rowptr, colidx, vals, B, C0, 0.5, -2.0, what="beta")
    plan = capi.Plan(algo, t(rowptr, gpu), t(colidx, gpu), t(vals, gpu), K, n_hint=N)
    dC = torch.full((M, N), float("nan"), device=gpu)
    plan.spmm(t(B, gpu), dC, 1.0, 0.0)
    torch.cuda.synchronize()
    Cp = dC.cpu().numpy()
    plan.close()
    check(algo, Cp, rowptr, colidx, vals, B, what="stored plan")
    Cc = run(algo, rowptr, colidx, vals, B, gpu)
    assert np.array_equal(Cp.view(np.uint32), Cc.view(np.uint32)), "plan and per-call differ"


@pytest.mark.parametrize("where", ["first", "middle", "last", "strided"])
@pytest.mark.parametrize("algo", ["WarpPerRow", "WarpPerRowFp4", "WarpPerRowSmemFp4"])
def test_combine_single_long_row(algo, where, gpu):
    """One row of 3000 nonzeros among rows of 0-3, split into segments and
    summed in the main launch."""
    K, N = 4096, 64
    M = 1_100_000 if where == "strided" else 60000
    rng = np.random.default_rng(9)
    lens = rng.integers(0, 4, M)
    # row block b = row // 256 (grid-strided: blocks beyond 4096 reuse
    # 0..4095, so row 4097 * 256 + 5 is in the second pass of block 1)
    row = {"first": 3, "middle": M // 2 + 17, "last": M - 1, "strided": 4097 * 256 + 5}[where]
    lens[row] = 3000
    rowptr = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    # sorted columns per row (short rows may repeat one: duplicates are valid)
    rid = np.repeat(np.arange(M), lens)
    cols = rng.integers(0, K, rid.size)
    cols[rowptr[row]:rowptr[row + 1]] = np.sort(rng.choice(K, 3000, replace=False))
    colidx = cols[np.lexsort((cols, rid))].astype(np.int32)
    vals = (rng.integers(0, 1 << 24, size=colidx.size) * 2.0 ** -23 - 1.0).astype(np.float32)
    B = gen.dense(9, gen.TAG_B, K, N)
    print(f"[combine] {algo} {where} M={M} nnz={colidx.size} long row {row}", flush=True)
    C = run(algo, rowptr, colidx, vals, B, gpu)
    check(algo, C, rowptr, colidx, vals, B, what=f"long row {where}")


@pytest.mark.parametrize("algo", ["WarpPerRowFp4", "Auto"])
def test_xslices_plan_across_widths(algo, gpu):
    """One stored plan (hinted at N = 64, no XCD slices) called at N = 128
    and 256 (two and four XCD bands) and 512 (ordinary column slices), with
    a long row among short ones: each call bit-identical to the per-call
    product and within the oracle's bar."""
    K, M = 16384, 5000
    lens = np.random.default_rng(13).integers(10, 120, M)
    lens[1234] = 6000  # a long row: segments and the combine
    rowptr, colidx, vals = csr_from_lengths(lens, K, seed=13)
    plan = capi.Plan(algo, t(rowptr, gpu), t(colidx, gpu), t(vals, gpu), K, n_hint=64)
    for N in (128, 256, 512, 64):
        B = gen.dense(N + 1, gen.TAG_B, K, N)
        dC = torch.full((M, N), float("nan"), device=gpu)
        plan.spmm(t(B, gpu), dC, 1.0, 0.0)
        torch.cuda.synchronize()
        Cp = dC.cpu().numpy()
        Cc = run(plan.algorithm, rowptr, colidx, vals, B, gpu)
        check(plan.algorithm, Cp, rowptr, colidx, vals, B, what=f"plan N={N}")
        short = np.diff(rowptr) <= 128
        assert np.array_equal(Cp[short].view(np.uint32), Cc[short].view(np.uint32)), \
            f"N={N}: plan and per-call differ on rows summed whole"
    plan.close()
