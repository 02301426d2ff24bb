"""GPU parity of the XCD shares (csrspmm_call_shares).

On a B whose 64-column band is at least 64 MiB, with no column panels and
2^20 nonzeros or more, a per-call product sums its long rows XCD by XCD:
the columns are cut into eight ranges from a per-call sample, a row of
129-2047 nonzeros is split into eight parts (one per range, each summed on
its own XCD into a partial row) and a longer row's segments are each summed
on the XCD of their middle column.  The parts partition every row's
positions whatever the boundaries, so every row must meet the 1e-5 bar
against the fp64 oracle; rows of at most 128 nonzeros are still summed whole
in CSR order and must equal the fp32 restatement bit for bit, and equal a
call without shares (a base-size workspace) bit for bit.

The cases: power-law rows (short, split and whole rows) with an unsorted
split row, an unsorted whole row and duplicate columns, on the scalar
variants at N = 64 (the float4 ones take column panels there); the beta and
C_IS_ZERO epilogues; a max_row_nnz hint below the true longest row (rows of
any length in one segment, split whole); and column slices of the float4
variants, one launch per slice (rows averaging 98) and all slices in one
launch (rows averaging 25), on a 1 GiB B.
"""
import functools

import numpy as np
import pytest
import torch

import oracle
from csrspmm_amd import capi, gen

pytestmark = pytest.mark.gpu

TOL = 1e-5
K = 262144  # a 64-column band of B is 64 MiB
# At N = 64 the float4 variants (and Auto, which picks them for rows of 24
# or more on average) take the column panels on such a B, which exclude the
# shares; the scalar ones have no panels below N = 128.  Float4 calls meet
# the shares in column slices (test_shares_column_slices).
SCALAR = ["WarpPerRow", "WarpPerRowSmem"]


@functools.lru_cache(maxsize=2)
def matrix(M, shift, seed):
    """Power-law rows (Zipf exponent 1.5, the given shift, at most 9000 per
    row), uniform sorted columns, then one split row and one whole row
    shuffled and a duplicated column in another long row."""
    a = gen.powerlaw(M, K, 1.5, shift, 9000, seed)
    rowptr, colidx, vals = a.rowptr, a.colidx.copy(), a.vals
    lens = np.diff(rowptr)
    rng = np.random.default_rng(seed)
    split = np.nonzero((lens > 128) & (lens < 2048))[0]
    whole = np.nonzero(lens >= 2048)[0]
    assert split.size >= 3 and whole.size >= 1
    for r in (split[0], whole[0]):
        rng.shuffle(colidx[rowptr[r]:rowptr[r + 1]])
    r = split[1]
    colidx[rowptr[r] + 5] = colidx[rowptr[r] + 4]  # a duplicate (still sorted)
    return rowptr, colidx, vals


def run(algo, rowptr, colidx, vals, B, dev, C0=None, alpha=1.0, beta=0.0, hint=-1, flags=0,
        base=False):
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(dev)  # noqa: E731
    M, N = rowptr.size - 1, B.shape[1]
    lib = capi.hip()
    a = capi.ALGO[algo]
    nbytes = (lib.csrspmm_workspace_bytes(a, M, N, int(vals.size)) if base else
              lib.csrspmm_workspace_bytes_ex(a, M, K, N, int(vals.size), hint))
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
    dC = t(C0) if C0 is not None else torch.full((M, N), float("nan"), device=dev)
    drp, dci = t(rowptr), t(colidx)
    capi.spmm(algo, drp, dci, t(vals), t(B), dC, alpha, beta, hint=hint, flags=flags, workspace=ws)
    torch.cuda.synchronize()
    assert torch.equal(dci.cpu(), torch.from_numpy(colidx)), "colidx modified"
    return dC.cpu().numpy()


def check(algo, C, rowptr, colidx, vals, B, C0=None, alpha=1.0, beta=0.0, rows=None, c0_zero=False,
          what=""):
    Cs = C if rows is None else C[rows]
    assert not np.isnan(Cs).any(), f"{algo} {what}: unwritten output"
    R, S = oracle.spmm_f64(rowptr, colidx, vals, B, C0, alpha, beta, c0_zero=c0_zero, rows=rows)
    bad, ratio, _, _ = oracle.check(Cs, R, S, TOL)
    assert bad == 0, f"{algo} {what}: {bad} elements off (max ratio {ratio:.3g})"
    F = oracle.spmm_f32_seq(rowptr, colidx, vals, B, C0, alpha, beta, c0_zero=c0_zero, rows=rows)
    ridx = np.arange(rowptr.size - 1) if rows is None else np.asarray(rows)
    short = (rowptr[ridx + 1] - rowptr[ridx]) <= 128
    assert np.array_equal(Cs[short].view(np.uint32), F[short].view(np.uint32)), \
        f"{algo} {what}: rows of at most 128 nonzeros differ from the fp32 restatement"


@pytest.mark.parametrize("algo", SCALAR)
def test_shares_every_row(algo, gpu):
    rowptr, colidx, vals = matrix(60000, 0.7, 7)
    M, N = rowptr.size - 1, 64
    assert capi.call_shares(algo, M, K, N, int(vals.size))
    B = gen.dense(7, gen.TAG_B, K, N)
    print(f"[shares] {algo} M={M} nnz={vals.size} N={N}", flush=True)
    C = run(algo, rowptr, colidx, vals, B, gpu)
    check(algo, C, rowptr, colidx, vals, B, what="shares")
    C2 = run(algo, rowptr, colidx, vals, B, gpu)
    assert np.array_equal(C.view(np.uint32), C2.view(np.uint32)), "not deterministic"
    # a base-size workspace runs without shares: short rows agree bit for bit
    Cb = run(algo, rowptr, colidx, vals, B, gpu, base=True)
    check(algo, Cb, rowptr, colidx, vals, B, what="base workspace")
    short = np.diff(rowptr) <= 128
    assert np.array_equal(C[short].view(np.uint32), Cb[short].view(np.uint32))


@pytest.mark.parametrize("algo", SCALAR)
def test_shares_epilogues_and_hint(algo, gpu):
    rowptr, colidx, vals = matrix(60000, 0.7, 7)
    M, N = rowptr.size - 1, 64
    B = gen.dense(8, gen.TAG_B, K, N)
    C0 = gen.dense(8, gen.TAG_C0, M, N)
    C = run(algo, rowptr, colidx, vals, B, gpu, C0=C0, alpha=0.5, beta=-1.25)
    check(algo, C, rowptr, colidx, vals, B, C0, 0.5, -1.25, what="beta")
    C = run(algo, rowptr, colidx, vals, B, gpu, C0=C0, alpha=1.5, beta=0.25, flags=capi.FLAG_C_IS_ZERO)
    check(algo, C, rowptr, colidx, vals, B, None, 1.5, 0.25, c0_zero=True, what="c_is_zero")
    # a hint of 300 (the longest row holds 9000): one segment per long row,
    # so every long row is split in eight parts whatever its length
    assert capi.call_shares(algo, M, K, N, int(vals.size), 300)
    C = run(algo, rowptr, colidx, vals, B, gpu, hint=300)
    check(algo, C, rowptr, colidx, vals, B, what="hint 300")
    # a hint of at most 128 rules out long rows: no shares
    assert not capi.call_shares(algo, M, K, N, int(vals.size), 128)


@pytest.mark.parametrize("algo", ["WarpPerRowFp4", "WarpPerRowSmemFp4"])
@pytest.mark.parametrize("M,shift", [(20000, 0.0), (60000, 0.7)])
def test_shares_column_slices(M, shift, algo, gpu):
    """N = 1024 on a 1 GiB B: 16 column slices of 64, whose bands are 64
    MiB.  Rows averaging 98 (shift 0) run one launch per slice, rows
    averaging 25 all slices in one launch; the parts and segment partials
    of every slice meet in one combine."""
    rowptr, colidx, vals = matrix(M, shift, 11)
    N = 1024
    assert capi.call_shares(algo, M, K, N, int(vals.size))
    B = gen.dense(11, gen.TAG_B, K, N)
    lens = np.diff(rowptr)
    rng = np.random.default_rng(5)
    rows = np.unique(np.concatenate([np.nonzero(lens > 128)[0][:1500],
                                     rng.choice(M, 1500, replace=False)])).astype(np.int32)
    print(f"[shares] slices {algo} M={M} nnz={vals.size} N={N} checked rows={rows.size}", flush=True)
    C = run(algo, rowptr, colidx, vals, B, gpu)
    check(algo, C, rowptr, colidx, vals, B, rows=rows, what="slices")
