"""The band sweep of column slices (rowgroup.hip sweep_rows): float4 calls
whose B is sliced (B of at least 32 MiB, N >= 128, a 64-column band of at
most 16 MiB), whose rows average at least two nonzeros per band and which
have enough rows for 8192 waves (M >= 65536) keep two rows' accumulators
per 16-lane group while all groups walk B in bands.  Every shape below meets
those conditions (K = 32768 or 49152, bands of 16384 B rows).  Each case is
checked against the oracle on every row, against the scalar-column variant
(WarpPerRow), which keeps the merge blocks, and against the LDS-staged
float4 variant (WarpPerRowSmemFp4), which sweeps through its LDS stage: all
sum every short row whole in CSR order and the long rows in the same
segments, so they must agree bit for bit.

Covered: ragged rows with empty ones, rows above the long-row limit (summed
by segments, skipped by the sweep), rows with unsorted columns (all of a row
in band 0), a last slice narrower than 64 columns, alpha/beta with C read,
strided B and C, max_row_nnz hints (exact, and too small so that the sweep
sums a long row whole), and a stored plan."""
import numpy as np
import pytest
import torch

import oracle
from csrspmm_amd import capi

pytestmark = pytest.mark.gpu


def rows_csr(lengths, K, seed, unsorted=()):
    """CSR with the given row lengths, distinct columns per row (sorted,
    except the rows listed in `unsorted`, whose columns are shuffled)."""
    rng = np.random.default_rng(seed)
    rowptr = np.zeros(len(lengths) + 1, dtype=np.int32)
    rowptr[1:] = np.cumsum(lengths)
    cols = []
    for r, n in enumerate(lengths):
        c = np.sort(rng.choice(K, size=n, replace=False)).astype(np.int32)
        if r in unsorted:
            rng.shuffle(c)
        cols.append(c)
    colidx = np.concatenate(cols) if cols else np.zeros(0, np.int32)
    vals = rng.uniform(-1, 1, rowptr[-1]).astype(np.float32)
    return rowptr, colidx, vals


def lengths_for(M, seed, long_rows=()):
    rng = np.random.default_rng(seed)
    n = rng.integers(0, 100, M)
    n[rng.choice(M, M // 50, replace=False)] = 0  # empty rows
    for r, L in long_rows:
        n[r] = L
    return n


def to(gpu, x):
    return torch.from_numpy(np.ascontiguousarray(x)).to(gpu)


def check_all(C, rp, ci, va, B, alpha, beta, C0, what):
    R, S = oracle.spmm_f64(rp, ci, va, np.ascontiguousarray(B), C0, alpha, beta)
    bad, ratio, _, _ = oracle.check(np.ascontiguousarray(C), R, S, 1e-5)
    assert bad == 0, f"{what}: {bad} elements off, max ratio {ratio}"


def run(algo, gpu, rp, ci, va, B, C0, alpha, beta, hint=-1):
    dC = to(gpu, C0)
    capi.spmm(algo, to(gpu, rp), to(gpu, ci), to(gpu, va), to(gpu, B), dC, alpha, beta,
              hint=hint)
    torch.cuda.synchronize()
    return dC


MS = 65536  # rows: 8192 waves of two rows per 16-lane group

CASES = {
    # id: (M, K, N, long rows (row, length), unsorted rows)
    "ragged": (MS, 32768, 256, (), ()),
    "long_rows": (MS, 32768, 256, ((7, 300), (1500, 2500), (MS - 1, 129)), ()),
    "unsorted": (MS, 32768, 256, ((11, 700),), (3, 4, 11, 2000)),
    "narrow_last_slice": (MS, 49152, 200, ((5, 400),), (9,)),
}


@pytest.mark.parametrize("case", sorted(CASES))
def test_sweep_against_oracle_and_merge_blocks(case, gpu):
    M, K, N, longs, unsorted = CASES[case]
    rp, ci, va = rows_csr(lengths_for(M, 5, longs), K, 6, unsorted)
    rng = np.random.default_rng(7)
    B = rng.uniform(-1, 1, (K, N)).astype(np.float32)
    C0 = rng.uniform(-1, 1, (M, N)).astype(np.float32)
    alpha, beta = 1.5, -0.5
    sweep = run("WarpPerRowFp4", gpu, rp, ci, va, B, C0, alpha, beta)
    check_all(sweep.cpu().numpy(), rp, ci, va, B, alpha, beta, C0, f"{case} sweep")
    merge = run("WarpPerRow", gpu, rp, ci, va, B, C0, alpha, beta)
    assert torch.equal(sweep, merge), f"{case}: sweep and merge blocks differ"
    lds = run("WarpPerRowSmemFp4", gpu, rp, ci, va, B, C0, alpha, beta)
    assert torch.equal(sweep, lds), f"{case}: the LDS-staged sweep differs"
    auto = run("Auto", gpu, rp, ci, va, B, C0, alpha, beta)
    assert torch.equal(sweep, auto), f"{case}: Auto differs from WarpPerRowFp4"


@pytest.mark.parametrize("hint", ["exact", "too_small"])
def test_sweep_with_hints(hint, gpu):
    """max_row_nnz = the true longest row (>= 128: segments as without a
    hint), and a hint of 90 with rows up to 300 long: every row is then summed
    whole, the long ones by the sweep itself."""
    M, K, N = MS, 32768, 256
    rp, ci, va = rows_csr(lengths_for(M, 9, ((17, 300), (2400, 250))), K, 10)
    rng = np.random.default_rng(11)
    B = rng.uniform(-1, 1, (K, N)).astype(np.float32)
    C0 = np.zeros((M, N), np.float32)
    h = int(np.diff(rp).max()) if hint == "exact" else 90
    C = run("WarpPerRowFp4", gpu, rp, ci, va, B, C0, 1.0, 0.0, hint=h)
    check_all(C.cpu().numpy(), rp, ci, va, B, 1.0, 0.0, None, f"hint {hint}")
    for other in ("WarpPerRow", "WarpPerRowSmemFp4"):
        assert torch.equal(C, run(other, gpu, rp, ci, va, B, C0, 1.0, 0.0, hint=h)), other


def test_sweep_strided_operands(gpu):
    """B and C as column windows of wider tensors (ldb, ldc > N)."""
    M, K, N = MS, 32768, 256
    rp, ci, va = rows_csr(lengths_for(M, 12, ((40, 333),)), K, 13)
    rng = np.random.default_rng(14)
    Bw = rng.uniform(-1, 1, (K, N + 12)).astype(np.float32)
    Cw = rng.uniform(-1, 1, (M, N + 20)).astype(np.float32)
    dB, dC = to(gpu, Bw), to(gpu, Cw)
    Bv, Cv = dB[:, 8:8 + N], dC[:, 4:4 + N]
    capi.spmm("WarpPerRowFp4", to(gpu, rp), to(gpu, ci), to(gpu, va), Bv, Cv, 0.75, 0.25)
    torch.cuda.synchronize()
    got = dC.cpu().numpy()
    check_all(got[:, 4:4 + N], rp, ci, va, Bw[:, 8:8 + N], 0.75, 0.25, Cw[:, 4:4 + N], "strided")
    assert np.array_equal(got[:, :4], Cw[:, :4]) and np.array_equal(got[:, 4 + N:], Cw[:, 4 + N:])


def test_sweep_stored_plan(gpu):
    """A stored plan of a matrix whose long rows stay below the panel
    threshold (1024): the plan's calls slice and sweep like the per-call path
    and must match it bit for bit."""
    M, K, N = MS, 32768, 256
    rp, ci, va = rows_csr(lengths_for(M, 15, ((100, 900), (101, 140))), K, 16, (50,))
    rng = np.random.default_rng(17)
    B = rng.uniform(-1, 1, (K, N)).astype(np.float32)
    drp, dci, dva, dB = to(gpu, rp), to(gpu, ci), to(gpu, va), to(gpu, B)
    plan = capi.Plan("WarpPerRowFp4", drp, dci, dva, K, n_hint=N)
    try:
        C = torch.empty((M, N), device=gpu)
        for _ in range(2):
            plan.spmm(dB, C, 1.0, 0.0)
        torch.cuda.synchronize()
    finally:
        plan.close()
    check_all(C.cpu().numpy(), rp, ci, va, B, 1.0, 0.0, None, "plan")
    per_call = run("WarpPerRowFp4", gpu, rp, ci, va, B, np.zeros((M, N), np.float32), 1.0, 0.0)
    assert torch.equal(C, per_call)


def test_sweep_wide_band_with_hint(gpu):
    """A 64-column band wider than 16 MiB (K = 81920: 20 MiB) is sliced only
    when the call sweeps with at least 4 nonzeros per band and no column
    panels can apply, as with a max_row_nnz hint below 1024.  Checked against
    the oracle and, bit for bit, against the LDS-staged float4 variant, which
    sweeps too, and the scalar-column variant, which stays unsliced there:
    on its 80 MiB B it splits the long rows by XCD (capi.call_shares), so
    against it only rows of at most 128 nonzeros, summed whole by both, are
    compared bit for bit."""
    M, K, N = MS, 81920, 256
    rp, ci, va = rows_csr(lengths_for(M, 18, ((3, 300), (MS - 1, 700))), K, 19, (8,))
    rng = np.random.default_rng(20)
    B = rng.uniform(-1, 1, (K, N)).astype(np.float32)
    C0 = rng.uniform(-1, 1, (M, N)).astype(np.float32)
    h = int(np.diff(rp).max())
    C = run("WarpPerRowFp4", gpu, rp, ci, va, B, C0, -1.25, 0.5, hint=h)
    check_all(C.cpu().numpy(), rp, ci, va, B, -1.25, 0.5, C0, "wide band")
    assert not capi.call_shares("WarpPerRowFp4", M, K, N, int(va.size), h)
    for other in ("WarpPerRow", "WarpPerRowSmemFp4"):
        Co = run(other, gpu, rp, ci, va, B, C0, -1.25, 0.5, hint=h)
        if capi.call_shares(other, M, K, N, int(va.size), h):
            check_all(Co.cpu().numpy(), rp, ci, va, B, -1.25, 0.5, C0, f"wide band {other}")
            short = torch.from_numpy(np.diff(rp) <= 128).to(gpu)
            assert torch.equal(C[short], Co[short]), other
        else:
            assert torch.equal(C, Co), other


@pytest.mark.parametrize("N", [128, 64])
def test_unsliced_sweep_with_hint(N, gpu):
    """Float4 calls of up to 128 columns also sweep when B exceeds 4 MiB, the
    max_row_nnz hint rules out skewed rows (at most 128, or 4x the mean) and
    the rows fill enough waves (M = 16384 with 32-lane groups, 65536 with
    16-lane ones):
    K = 32768 gives a 16 MiB (N = 128) or 8 MiB (N = 64) B in 4 MiB bands.
    Rows of 50-149 nonzeros with one of 300 (segments, skipped by the sweep;
    the hint 300 is below 4x the mean) and one unsorted.  Against the oracle
    and bit for bit against the merge blocks (WarpPerRow) and the LDS-staged
    sweep."""
    M, K = (16384 if N == 128 else MS), 32768  # 4096 / 8192 waves
    rng = np.random.default_rng(22)
    lens = rng.integers(50, 150, M)
    lens[17] = 300
    rp, ci, va = rows_csr(lens, K, 23, (40,))
    B = rng.uniform(-1, 1, (K, N)).astype(np.float32)
    C0 = rng.uniform(-1, 1, (M, N)).astype(np.float32)
    h = int(np.diff(rp).max())
    C = run("WarpPerRowFp4", gpu, rp, ci, va, B, C0, 0.5, -2.0, hint=h)
    check_all(C.cpu().numpy(), rp, ci, va, B, 0.5, -2.0, C0, f"unsliced N={N}")
    for other in ("WarpPerRow", "WarpPerRowSmemFp4"):
        assert torch.equal(C, run(other, gpu, rp, ci, va, B, C0, 0.5, -2.0, hint=h)), other
    no_hint = run("WarpPerRowFp4", gpu, rp, ci, va, B, C0, 0.5, -2.0)
    assert torch.equal(C, no_hint)


@pytest.mark.parametrize("seed,M,K,N", [(31, 70000, 48000, 192), (32, 66000, 30000, 320),
                                        (33, 80000, 65000, 132)])
def test_sweep_random_shapes(seed, M, K, N, gpu):
    """Seeded shapes off the powers of two (rows and slices that do not
    divide evenly, a last slice of 4 columns at N = 132), with a few long
    and unsorted rows: bit for bit against the merge blocks (WarpPerRow) and
    the LDS-staged sweep, and against the oracle on sampled rows."""
    rng = np.random.default_rng(seed)
    lens = rng.integers(0, 2 * (seed % 5 + 20), M)
    for r in rng.choice(M, 6, replace=False):
        lens[r] = int(rng.integers(129, 3000))
    rp, ci, va = rows_csr(lens, K, seed + 100, tuple(int(x) for x in rng.choice(M, 4, replace=False)))
    B = rng.uniform(-1, 1, (K, N)).astype(np.float32)
    C0 = rng.uniform(-1, 1, (M, N)).astype(np.float32)
    C = run("WarpPerRowFp4", gpu, rp, ci, va, B, C0, 1.0, 1.0)
    for other in ("WarpPerRow", "WarpPerRowSmemFp4"):
        assert torch.equal(C, run(other, gpu, rp, ci, va, B, C0, 1.0, 1.0)), other
    rows = np.unique(np.concatenate([rng.choice(M, 3000, replace=False), np.nonzero(lens > 128)[0]]))
    R, S = oracle.spmm_f64(rp, ci, va, B, C0, 1.0, 1.0, rows=rows)
    bad, ratio, _, _ = oracle.check(C.cpu().numpy()[rows], R, S, 1e-5)
    assert bad == 0, f"{bad} elements off, max ratio {ratio}"
