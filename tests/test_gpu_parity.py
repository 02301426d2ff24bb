"""GPU parity: every variant of libcsrspmm_hip.so, called through the C ABI,
against the CPU oracle on the same seeded inputs.

Bar: |C - R| <= 1e-5 * max(|R|, S) elementwise
against the fp64 oracle R (S = |alpha| sum |a b| + |beta c0|), CSR arrays
byte-identical after the call.  Rows the kernels sum whole (every row for
Naive/NaiveSmem, rows shorter than two segments for the warp-per-row
family: under 512 nonzeros on matrices of a million nonzeros or more,
under 64..511 on smaller ones, csr_cases.whole_row_max) must also equal the
oracle's fp32 CSR-order fma restatement bit for bit, since the kernels use
the same order; longer rows are split into near-equal segments whose partial
sums are added in a fixed order, which is within the tolerance but not
bitwise.

Every BASELINE config is checked on every element of C, for Auto and each
variant: the fp64 oracle and the fp32 restatement are OpenMP loops over rows
(R-MAT at N = 64, 16 M nonzeros: about 0.6 s on 8 cores), computed once per
config and shared by its variants.
"""
import functools

import numpy as np
import pytest
import torch

import oracle
from csrspmm_amd import ALGORITHMS, capi, configs, gen
from csr_cases import csr_from_lengths, whole_row_limit, whole_row_max
from golden_cases import load, names

pytestmark = pytest.mark.gpu

TOL = 1e-5
WHOLE_ROW_ALGOS = {"Naive", "NaiveSmem"}


def dev_t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def run_spmm(algo, rowptr, colidx, vals, B, dev, C0=None, alpha=1.0, beta=0.0, hint=-1, flags=0,
             owned=False, N=None):
    drp, dci, dv = dev_t(rowptr, dev), dev_t(colidx, dev), dev_t(vals, dev)
    dB = dev_t(B, dev)
    M = rowptr.size - 1
    N = B.shape[1] if N is None else N
    if C0 is not None:
        dC = dev_t(C0, dev)
    else:
        dC = torch.full((M, N), float("nan"), dtype=torch.float32, device=dev)
    capi.spmm(algo, drp, dci, dv, dB, dC, alpha, beta, hint=hint, flags=flags, owned_workspace=owned)
    torch.cuda.synchronize()
    # A must be untouched
    assert torch.equal(drp.cpu(), torch.from_numpy(rowptr))
    assert torch.equal(dci.cpu(), torch.from_numpy(colidx))
    assert torch.equal(dv.cpu().view(torch.int32), torch.from_numpy(vals).view(torch.int32))
    return dC.cpu().numpy()


def assert_parity(algo, C, rowptr, colidx, vals, B, C0, alpha, beta, rows=None, c0_zero=False,
                  what="", hint=-1, shares=None, ref=None):
    """ref: (R, S, F) of these inputs, already computed, or None."""
    if ref is None:
        R, S = oracle.spmm_f64(rowptr, colidx, vals, B, C0, alpha, beta, c0_zero=c0_zero, rows=rows)
        F = oracle.spmm_f32_seq(rowptr, colidx, vals, B, C0, alpha, beta, c0_zero=c0_zero, rows=rows)
    else:
        R, S, F = ref
    Cs = C if rows is None else C[rows]
    bad, ratio, plain, worst = oracle.check(Cs, R, S, TOL)
    assert bad == 0, f"{algo} {what}: {bad} elements out of tolerance (max ratio {ratio:.3g})"
    # bitwise against the fp32 restatement on rows summed whole
    ridx = np.arange(rowptr.size - 1) if rows is None else np.asarray(rows)
    lens = rowptr[ridx + 1] - rowptr[ridx]
    whole = (np.ones_like(lens, dtype=bool) if algo in WHOLE_ROW_ALGOS
             else lens <= whole_row_limit(algo, rowptr, B.shape[0], B.shape[1], hint, shares))
    a = Cs[whole].view(np.uint32)
    b = F[whole].view(np.uint32)
    # +0 and -0 only differ in sign bits; NaN payloads are not compared.
    same = (a == b) | ((Cs[whole] == 0) & (F[whole] == 0)) | (np.isnan(Cs[whole]) & np.isnan(F[whole]))
    assert same.all(), f"{algo} {what}: {np.count_nonzero(~same)} whole-row elements differ from the fp32 restatement"
    return ratio, plain


# ---------------------------------------------------------------- golden fixtures

@pytest.mark.parametrize("algo", ALGORITHMS)
@pytest.mark.parametrize("name", names())
def test_golden_fixture(algo, name, gpu):
    g = load(name)
    C = run_spmm(algo, g["rowptr"], g["colidx"], g["vals"], g["B"], gpu, C0=g["C0"],
                 alpha=g["alpha"], beta=g["beta"])
    bad, ratio, _, _ = oracle.check(C, g["R"], g["S"], TOL)
    assert bad == 0, f"{algo}/{name}: max ratio {ratio}"
    assert_parity(algo, C, g["rowptr"], g["colidx"], g["vals"], g["B"], g["C0"], g["alpha"],
                  g["beta"], what=name)
    if name.startswith("integer"):
        assert np.array_equal(C.astype(np.float64), g["R"])


# ---------------------------------------------------------------- BASELINE configs

@functools.lru_cache(maxsize=2)
def config_data(name):
    cfg = configs.CONFIGS[name]
    a = cfg.csr()
    B = cfg.B(a.K)
    return cfg, a, B


@functools.lru_cache(maxsize=1)
def config_ref(name):
    """(R, S, F) over every row of a config (one config held at a time: the
    tests below run config by config)."""
    cfg, a, B = config_data(name)
    R, S = oracle.spmm_f64(a.rowptr, a.colidx, a.vals, B)
    F = oracle.spmm_f32_seq(a.rowptr, a.colidx, a.vals, B)
    return R, S, F


def sample_rows(a, full):
    if full:
        return None
    rng = np.random.default_rng(123)
    lens = np.diff(a.rowptr)
    longest = np.argsort(lens)[-64:]
    empty = np.nonzero(lens == 0)[0][:64]
    rnd = rng.choice(a.M, size=4096, replace=False)
    return np.unique(np.concatenate([longest, empty, rnd])).astype(np.int32)


# algo varies fastest, so each config's oracle is computed once
@pytest.mark.parametrize("algo", ("Auto",) + ALGORITHMS)
@pytest.mark.parametrize("cfg_name", ["host", "medium", "large", "xl", "xl98", "rmat", "rmat512"])
def test_config(cfg_name, algo, gpu):
    """Every element of C against the fp64 oracle (and, on rows summed
    whole, the fp32 restatement bit for bit)."""
    cfg, a, B = config_data(cfg_name)
    print(f"[parity] {cfg_name} {algo} M={a.M} nnz={a.nnz} N={cfg.N} (every row)", flush=True)
    C = run_spmm(algo, a.rowptr, a.colidx, a.vals, B, gpu, alpha=1.0, beta=0.0)
    assert not np.isnan(C).any(), "unwritten output elements"
    assert_parity(algo, C, a.rowptr, a.colidx, a.vals, B, None, 1.0, 0.0, what=cfg_name,
                  ref=config_ref(cfg_name))


def test_xl_deterministic_and_hint_independent(gpu):
    cfg, a, B = config_data("xl")
    C1 = run_spmm("WarpPerRowFp4", a.rowptr, a.colidx, a.vals, B, gpu)
    C2 = run_spmm("WarpPerRowFp4", a.rowptr, a.colidx, a.vals, B, gpu)
    assert np.array_equal(C1.view(np.uint32), C2.view(np.uint32))
    # a wrong "short rows only" hint skips the split plan: still correct
    C3 = run_spmm("WarpPerRowSmemFp4", a.rowptr, a.colidx, a.vals, B, gpu, hint=8)
    rows = sample_rows(a, False)
    assert_parity("WarpPerRowSmemFp4", C3, a.rowptr, a.colidx, a.vals, B, None, 1.0, 0.0,
                  rows=rows, what="xl hint=8", hint=8)
    # the library-owned workspace path gives the same bits
    C4 = run_spmm("WarpPerRowFp4", a.rowptr, a.colidx, a.vals, B, gpu, owned=True)
    assert np.array_equal(C1.view(np.uint32), C4.view(np.uint32))


# ---------------------------------------------------------------- epilogue and edge cases

@pytest.mark.parametrize("algo", ALGORITHMS)
def test_epilogue_modes(algo, gpu):
    a = gen.ragged(300, 800, 0, 600, seed=77)
    B = gen.dense(77, gen.TAG_B, 800, 40)
    C0 = gen.dense(77, gen.TAG_C0, 300, 40)
    # accumulate into C0
    C = run_spmm(algo, a.rowptr, a.colidx, a.vals, B, gpu, C0=C0, alpha=0.75, beta=-1.5)
    assert_parity(algo, C, a.rowptr, a.colidx, a.vals, B, C0, 0.75, -1.5, what="beta")
    # beta == 0 overwrites NaN
    nan0 = np.full_like(C0, np.nan)
    C = run_spmm(algo, a.rowptr, a.colidx, a.vals, B, gpu, C0=nan0, alpha=2.0, beta=0.0)
    assert_parity(algo, C, a.rowptr, a.colidx, a.vals, B, None, 2.0, 0.0, what="beta0")
    # C_IS_ZERO: C0 never read, beta scales +0
    C = run_spmm(algo, a.rowptr, a.colidx, a.vals, B, gpu, C0=nan0, alpha=1.0, beta=0.5,
                 flags=capi.FLAG_C_IS_ZERO)
    assert_parity(algo, C, a.rowptr, a.colidx, a.vals, B, None, 1.0, 0.5, c0_zero=True,
                  what="c_is_zero")


@pytest.mark.parametrize("algo", ALGORITHMS)
@pytest.mark.parametrize("N", [1, 3, 4, 31, 64, 96, 130, 1100])
def test_column_counts(algo, N, gpu):
    a = gen.ragged(97, 401, 0, 300, seed=N)
    B = gen.dense(N, gen.TAG_B, 401, N)
    C = run_spmm(algo, a.rowptr, a.colidx, a.vals, B, gpu)
    assert_parity(algo, C, a.rowptr, a.colidx, a.vals, B, None, 1.0, 0.0, what=f"N={N}")


@pytest.mark.parametrize("algo", ALGORITHMS)
def test_strided_b_and_split_boundaries(algo, gpu):
    # rows of exactly 256, 257, 511, 512, 767, 768 and 20000 nonzeros around short ones
    K = 30000
    lens = np.array([0, 256, 1, 257, 511, 512, 767, 768, 0, 20000, 3, 255], dtype=np.int64)
    rng = np.random.default_rng(5)
    rowptr = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    colidx = np.concatenate([np.sort(rng.choice(K, L, replace=False)) for L in lens]).astype(np.int32)
    vals = rng.uniform(-1, 1, colidx.size).astype(np.float32)
    Bfull = rng.uniform(-1, 1, (K, 72)).astype(np.float32)
    dev = gpu
    N = 64
    drp, dci, dv = dev_t(rowptr, dev), dev_t(colidx, dev), dev_t(vals, dev)
    dB = dev_t(Bfull, dev)[:, :N]  # ldb = 72 > N
    dC = torch.full((lens.size, N), float("nan"), device=dev)
    capi.spmm(algo, drp, dci, dv, dB, dC, 1.0, 0.0)
    torch.cuda.synchronize()
    C = dC.cpu().numpy()
    assert_parity(algo, C, rowptr, colidx, vals, Bfull[:, :N].copy(), None, 1.0, 0.0, what="strided")


@pytest.mark.parametrize("algo", ["WarpPerRow", "WarpPerRowFp4", "WarpPerRowSmem", "WarpPerRowSmemFp4"])
@pytest.mark.parametrize("hint", [-1, 60, 128, 300, 2000, 5000])
def test_row_hint(algo, hint, gpu):
    """The max_row_nnz hint only steers the plan: at most 128 drops the
    segment phase (the merge blocks sum every row whole), below 512 drops
    split rows (one segment per long row).  A hint below the true longest
    row (2000 here) gives the right result, only slower."""
    rng = np.random.default_rng(7)
    K = 6000
    short = rng.integers(0, 6, 30000)
    long_ = np.array([100, 129, 200, 255, 256, 400, 511, 512, 600, 1200, 2000])
    lens = short.copy()
    lens[rng.choice(lens.size, long_.size, replace=False)] = long_
    rowptr = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    colidx = np.concatenate([np.sort(rng.choice(K, L, replace=False)) for L in lens]).astype(np.int32)
    vals = rng.uniform(-1, 1, colidx.size).astype(np.float32)
    B = rng.uniform(-1, 1, (K, 64)).astype(np.float32)
    C = run_spmm(algo, rowptr, colidx, vals, B, gpu, hint=hint)
    assert_parity(algo, C, rowptr, colidx, vals, B, None, 1.0, 0.0, what=f"hint={hint}", hint=hint)
    C0 = rng.uniform(-1, 1, (lens.size, 64)).astype(np.float32)
    C = run_spmm(algo, rowptr, colidx, vals, B, gpu, C0=C0, alpha=0.5, beta=2.0, hint=hint)
    assert_parity(algo, C, rowptr, colidx, vals, B, C0, 0.5, 2.0, what=f"hint={hint} beta", hint=hint)


@functools.lru_cache(maxsize=None)
def short_row_problem(shape):
    M, K, per, N = shape
    rng = np.random.default_rng(M + per)
    lens = rng.integers(per // 2, per + per // 2 + 1, M)
    lens[::97] = 0
    rowptr, colidx, vals = csr_from_lengths(lens, K, seed=M + per)
    B = rng.uniform(-1, 1, (K, N)).astype(np.float32)
    C0 = rng.uniform(-1, 1, (M, N)).astype(np.float32)
    return lens, rowptr, colidx, vals, B, C0


@pytest.mark.parametrize("algo", ["Auto", "WarpPerRow", "WarpPerRowFp4", "WarpPerRowSmem", "WarpPerRowSmemFp4"])
@pytest.mark.parametrize("shape", [(4096, 4096, 41, 128), (16384, 16384, 60, 256), (8192, 4096, 41, 96),
                                   (2048, 4096, 150, 256)])
def test_hinted_short_rows_one_launch(algo, shape, gpu):
    """A hint of at most 256 on a mid-sized problem (under 2^20 rows +
    nonzeros and 32768 rows, no column slices) skips the plan: one group per
    row, one launch, no workspace.  Every row against the oracle and bit for
    bit against the fp32 restatement, every row being summed whole, with the
    hint at the longest row and at 256, and with beta != 0."""
    M, K, per, N = shape
    lens, rowptr, colidx, vals, B, C0 = short_row_problem(shape)
    for hint in (int(lens.max()), 256):
        assert capi.hip().csrspmm_workspace_bytes_ex(capi.ALGO[algo], M, K, N, colidx.size, hint) == 0
        print(f"[parity] one launch {algo} M={M} K={K} N={N} hint={hint}", flush=True)
        C = run_spmm(algo, rowptr, colidx, vals, B, gpu, hint=hint)
        assert_parity(algo, C, rowptr, colidx, vals, B, None, 1.0, 0.0, what=f"hint={hint}", hint=hint)
        F = oracle.spmm_f32_seq(rowptr, colidx, vals, B, None, 1.0, 0.0)
        assert np.array_equal(C.view(np.uint32), F.view(np.uint32)), "rows summed whole"
    C = run_spmm(algo, rowptr, colidx, vals, B, gpu, C0=C0, alpha=0.5, beta=-1.5, hint=int(lens.max()))
    assert_parity(algo, C, rowptr, colidx, vals, B, C0, 0.5, -1.5, what="beta", hint=int(lens.max()))


@pytest.mark.parametrize("algo", ALGORITHMS)
@pytest.mark.parametrize("N", [1, 3, 5, 130])
def test_split_rows_odd_columns(algo, N, gpu):
    """Split rows at column counts that are not a multiple of 4, with C rows
    that are not 16-byte aligned: the combine reads partials four columns at
    a time and stores C column by column.  Runs of consecutive long rows put
    several split rows in one scan chunk of the combine, and many rows with
    long table ranges (merge-block starts, segment slots) in one wave of the
    per-call plan."""
    K = 20000
    lens = np.concatenate([[20000, 0, 3], np.full(40, 520), [700, 1, 0], np.full(70, 600),
                           np.arange(64) % 5, [1500, 9000]]).astype(np.int64)
    rng = np.random.default_rng(100 + N)
    rowptr = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    colidx = np.concatenate([np.sort(rng.choice(K, L, replace=False)) for L in lens]).astype(np.int32)
    vals = rng.uniform(-1, 1, colidx.size).astype(np.float32)
    B = rng.uniform(-1, 1, (K, N)).astype(np.float32)
    M = lens.size
    dev = gpu
    drp, dci, dv, dB = dev_t(rowptr, dev), dev_t(colidx, dev), dev_t(vals, dev), dev_t(B, dev)
    if N == 1:
        dC = torch.full((M, 1), float("nan"), device=dev)  # 4-byte rows
    else:
        ldc = N + 1 if (N + 1) % 4 else N + 2
        dC = torch.full((M, ldc), float("nan"), device=dev)[:, :N]
    capi.spmm(algo, drp, dci, dv, dB, dC, 1.0, 0.0)
    torch.cuda.synchronize()
    C = dC.cpu().numpy()
    assert_parity(algo, C, rowptr, colidx, vals, B, None, 1.0, 0.0, what=f"split N={N}")


@pytest.mark.parametrize("algo", ALGORITHMS)
def test_empty_and_degenerate(algo, gpu):
    # nnz = 0 with beta != 0 and with beta == 0
    M, K, N = 50, 40, 12
    rowptr = np.zeros(M + 1, dtype=np.int32)
    z = np.zeros(0, dtype=np.int32)
    zf = np.zeros(0, dtype=np.float32)
    B = gen.dense(3, gen.TAG_B, K, N)
    C0 = gen.dense(3, gen.TAG_C0, M, N)
    C = run_spmm(algo, rowptr, z, zf, B, gpu, C0=C0, alpha=1.0, beta=0.5)
    np.testing.assert_array_equal(C, np.float32(0.5) * C0)
    C = run_spmm(algo, rowptr, z, zf, B, gpu, C0=np.full_like(C0, np.nan), alpha=1.0, beta=0.0)
    assert np.all(C == 0.0)
    # M = 0 and N = 0 are no-ops
    r0 = np.zeros(1, dtype=np.int32)
    C = run_spmm(algo, r0, z, zf, B, gpu, C0=np.zeros((0, N), np.float32))
    assert C.shape == (0, N)


@pytest.mark.parametrize("algo", ALGORITHMS)
def test_duplicates_unsorted_and_nonfinite_b(algo, gpu):
    rng = np.random.default_rng(8)
    M, K, N = 40, 30, 16
    lens = rng.integers(0, 700, M)
    rowptr = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    colidx = rng.integers(0, K, int(lens.sum())).astype(np.int32)  # unsorted, duplicates
    vals = rng.uniform(-1, 1, colidx.size).astype(np.float32)
    B = rng.uniform(-1, 1, (K, N)).astype(np.float32)
    C = run_spmm(algo, rowptr, colidx, vals, B, gpu)
    assert_parity(algo, C, rowptr, colidx, vals, B, None, 1.0, 0.0, what="dup")
    # Inf / NaN in B propagate exactly like the oracle's classes
    B2 = B.copy()
    B2[3, 5] = np.inf
    B2[7, 1] = np.nan
    C = run_spmm(algo, rowptr, colidx, vals, B2, gpu)
    R, S = oracle.spmm_f64(rowptr, colidx, vals, B2)
    with np.errstate(invalid="ignore"):
        assert oracle.check(C, R, S, TOL)[0] == 0


def test_validator(gpu):
    a = gen.ragged(1000, 300, 0, 80, seed=4)
    flags, mx = capi.validate(dev_t(a.rowptr, gpu), dev_t(a.colidx, gpu), a.K)
    assert flags == 0 and mx == a.max_row_nnz
    bad_cols = a.colidx.copy()
    bad_cols[10] = a.K
    flags, _ = capi.validate(dev_t(a.rowptr, gpu), dev_t(bad_cols, gpu), a.K)
    assert flags & 8
    bad_rp = a.rowptr.copy()
    bad_rp[500] = bad_rp[501] + 1
    flags, _ = capi.validate(dev_t(bad_rp, gpu), dev_t(a.colidx, gpu), a.K)
    assert flags & 4
    unsorted = a.colidx.copy()
    r = int(np.argmax(np.diff(a.rowptr)))
    s = a.rowptr[r]
    unsorted[s], unsorted[s + 1] = unsorted[s + 1], unsorted[s]
    flags, _ = capi.validate(dev_t(a.rowptr, gpu), dev_t(unsorted, gpu), a.K)
    assert flags == 16
    end = a.rowptr.copy()
    end[-1] -= 1
    flags, _ = capi.validate(dev_t(end, gpu), dev_t(a.colidx[:-1].copy(), gpu), a.K)
    assert flags == 0
    flags, _ = capi.validate(dev_t(end, gpu), dev_t(a.colidx, gpu), a.K)
    assert flags & 2


def test_reference_harness_known_answer(gpu):
    """The reference's default test_csrspmm inputs (constant -5 matrices from
    its re-seeding dense_init_random, dense A) give C = 25597.5 everywhere."""
    A = oracle.dense_init_random_ref(1024, 1024, -10.0, 10.0, 0.7, True)
    rowptr, colidx, vals, mx = oracle.dense2csr(A, 0.0)
    B = np.full((1024, 1024), -5.0, dtype=np.float32)
    C0 = np.full((1024, 1024), -5.0, dtype=np.float32)
    for algo in ALGORITHMS:
        C = run_spmm(algo, rowptr, colidx, vals, B, gpu, C0=C0, alpha=1.0, beta=0.5, hint=mx)
        assert np.all(C == np.float32(25597.5)), algo


@pytest.mark.parametrize("per_row", [12, 40])
@pytest.mark.parametrize("algo", ["WarpPerRowFp4", "WarpPerRowSmemFp4"])
def test_unsliced_row_sized_merge_blocks(algo, per_row, gpu):
    """An unsliced per-call float4 call of fewer than 65536 rows takes merge
    blocks sized to its mean row (16 or 32 items here) when at least 16384
    of them remain, and so does a stored plan for that width.  Rows are
    summed whole: the two agree bit for bit, and with the oracle."""
    K, N, M = 20000, 128, 40000  # B of 10 MiB: no slices, no panels
    rng = np.random.default_rng(200 + per_row)
    lens = np.minimum(rng.integers(0, 2 * per_row + 1, M), 128).astype(np.int64)
    rowptr, colidx, vals = csr_from_lengths(lens, K, seed=per_row)
    B = gen.dense(25, gen.TAG_B, K, N)
    print(f"[parity] row-sized merge blocks {algo} per_row={per_row} nnz={colidx.size}", flush=True)
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
    assert_parity(algo, C, rowptr, colidx, vals, B, None, 1.0, 0.0, what=f"row-sized blocks {per_row}")
    assert np.array_equal(C.view(np.uint32), dP.cpu().numpy().view(np.uint32)), \
        f"{algo}: per-call and stored-plan results differ"
