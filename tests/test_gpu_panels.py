"""GPU parity of the per-call column panels.

With float4 columns (WarpPerRowFp4 / WarpPerRowSmemFp4), or scalar ones
from N = 128 (WarpPerRow / WarpPerRowSmem, Auto), a B wide enough for 32
panels (>= 64 MiB) and N <= 256, every SpMM call cuts rows of >= 1024
nonzeros with sorted columns at column-panel boundaries on the device, sums
the pieces panel by panel (each XCD walking its own panels) and adds a
row's pieces in column order.  These tests put such rows next to the cases
that must fall back to the ordinary long-row segments (unsorted columns,
skewed panel loads, a workspace sized without the panel tables) and check
every row against the fp64 oracle at the 1e-5 bar, plus bitwise agreement
with the fp32 CSR-order restatement on the rows summed whole.
"""
import numpy as np
import pytest
import torch

import oracle
from csrspmm_amd import ALGORITHMS, capi, gen
from csr_cases import csr_from_lengths, mixed_lengths, whole_row_limit, whole_row_max

pytestmark = pytest.mark.gpu

TOL = 1e-5
PANEL_ALGOS = ["WarpPerRowFp4", "WarpPerRowSmemFp4", "Auto", "WarpPerRow", "WarpPerRowSmem"]


def expects_panels(algo, N, M=None, K=None, nnz=None):
    """Whether a per-call product on a 64 MiB+ B with N <= 256 takes panels:
    float4 columns at any N, scalar columns from N = 128.  Auto is resolved
    from the shape by the library (below N = 128 it takes float4 columns
    when rows average 24 nonzeros or more)."""
    if algo == "Auto":
        lib = capi.hip()
        algo = lib.csrspmm_algorithm_name(
            lib.csrspmm_resolve_algorithm_ex(capi.ALGO["Auto"], M, K, N, nnz, -1)).decode()
    return algo in ("WarpPerRowFp4", "WarpPerRowSmemFp4") or (
        algo in ("WarpPerRow", "WarpPerRowSmem") and N >= 128)


def run(algo, rowptr, colidx, vals, B, dev, C0=None, alpha=1.0, beta=0.0, workspace_bytes=None):
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(dev)  # noqa: E731
    drp, dci, dv, dB = t(rowptr), t(colidx), t(vals), t(B)
    M, N = rowptr.size - 1, B.shape[1]
    dC = t(C0) if C0 is not None else torch.full((M, N), float("nan"), device=dev)
    ws = None
    if workspace_bytes is not None:
        ws = torch.empty(max(workspace_bytes, 1), dtype=torch.uint8, device=dev)
    capi.spmm(algo, drp, dci, dv, dB, dC, alpha, beta, workspace=ws)
    torch.cuda.synchronize()
    assert torch.equal(dci.cpu(), torch.from_numpy(colidx))
    return dC.cpu().numpy()


def check(algo, C, rowptr, colidx, vals, B, C0=None, alpha=1.0, beta=0.0, what=""):
    assert not np.isnan(C).any(), f"{algo} {what}: unwritten output"
    R, S = oracle.spmm_f64(rowptr, colidx, vals, B, C0, alpha, beta)
    bad, ratio, _, _ = oracle.check(C, R, S, TOL)
    assert bad == 0, f"{algo} {what}: {bad} elements off (max ratio {ratio:.3g})"
    F = oracle.spmm_f32_seq(rowptr, colidx, vals, B, C0, alpha, beta)
    whole = np.diff(rowptr) <= whole_row_limit(algo, rowptr, B.shape[0], B.shape[1])
    assert np.array_equal(C[whole].view(np.uint32), F[whole].view(np.uint32)), \
        f"{algo} {what}: short rows differ from the fp32 restatement"


def run_nl(algo, rowptr, colidx, vals, B, dev):
    """(C, rows the call panelized, None without panels)."""
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(dev)  # noqa: E731
    M, N = rowptr.size - 1, B.shape[1]
    dC = torch.full((M, N), float("nan"), device=dev)
    nl = capi.panelized_rows(algo, t(rowptr), t(colidx), t(vals), t(B), dC)
    return dC.cpu().numpy(), nl


def panel_bytes(algo, M, K, N, nnz):
    lib = capi.hip()
    a = capi.ALGO[algo]
    return lib.csrspmm_workspace_bytes(a, M, N, nnz), lib.csrspmm_workspace_bytes_ex(a, M, K, N, nnz, -1)


@pytest.mark.parametrize("N", [64, 128, 256])
@pytest.mark.parametrize("algo", list(ALGORITHMS) + ["Auto"])
def test_panels_mixed_rows(algo, N, gpu):
    # B of 64 / 64 / 128 MiB: 32 panels or more, and at N = 256 64-column
    # bands of 32 MiB, too wide for column slices to take over
    K = {64: 262144, 128: 131072, 256: 131072}[N]
    lens = np.minimum(mixed_lengths(7 + N), K)
    narrow = {int(np.nonzero(lens == 4096)[0][0]): (K // 3, K // 3 + 5000)}  # one panel-ish band
    rowptr, colidx, vals = csr_from_lengths(lens, K, seed=N, narrow=narrow)
    B = gen.dense(11, gen.TAG_B, K, N)
    print(f"[panels] mixed {algo} N={N} M={lens.size} nnz={colidx.size}", flush=True)
    base, full = panel_bytes(algo, lens.size, K, N, colidx.size)
    if expects_panels(algo, N, lens.size, K, colidx.size):
        assert full > base, "a 64 MiB B reserves the panel tables"
    else:
        assert full == base
    C = run(algo, rowptr, colidx, vals, B, gpu)
    check(algo, C, rowptr, colidx, vals, B, what=f"mixed N={N}")
    # repeated calls are bit-identical (no atomics in the float path)
    C2, nl = run_nl(algo, rowptr, colidx, vals, B, gpu)
    assert np.array_equal(C.view(np.uint32), C2.view(np.uint32))
    if full > base:
        # columns uniform apart from one row: every row of >= 1024 nonzeros
        # (sorted, fewer than the nnz / 4096 cap) is panelized
        assert nl == np.count_nonzero(lens >= 1024)


@pytest.mark.parametrize("algo", PANEL_ALGOS)
def test_panels_more_rows_than_the_cap(algo, gpu):
    # 400 rows of 1024..1299 nonzeros: more than the nnz / 4096 rows a call
    # panelizes, so the first ones (in row order) take pieces and the rest
    # segments, in the same call
    K, N = 131072, 128
    rng = np.random.default_rng(61)
    lens = rng.integers(0, 20, size=2400)
    lens[rng.choice(lens.size, 400, replace=False)] = rng.integers(1024, 1300, size=400)
    rowptr, colidx, vals = csr_from_lengths(lens, K, seed=61)
    assert np.count_nonzero(lens >= 1024) > -(-colidx.size // 4096)
    B = gen.dense(61, gen.TAG_B, K, N)
    print(f"[panels] cap {algo} M={lens.size} nnz={colidx.size}", flush=True)
    C = run(algo, rowptr, colidx, vals, B, gpu)
    check(algo, C, rowptr, colidx, vals, B, what="rows beyond the panel cap")
    C2, nl = run_nl(algo, rowptr, colidx, vals, B, gpu)
    assert np.array_equal(C.view(np.uint32), C2.view(np.uint32))
    assert nl == -(-colidx.size // 4096), "the first nnz / 4096 long rows are panelized"


@pytest.mark.parametrize("algo", PANEL_ALGOS)
def test_panels_epilogue_and_strided_b(algo, gpu):
    K, N = 131072, 128
    lens = mixed_lengths(21, M=1500)
    rowptr, colidx, vals = csr_from_lengths(lens, K, seed=21)
    Bw = gen.dense(12, gen.TAG_B, K, N + 4)
    B = Bw[:, :N]  # leading dimension N + 4 (padded rows)
    C0 = gen.dense(12, gen.TAG_C0, lens.size, N)
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(gpu)  # noqa: E731
    dBw = t(Bw)
    dB = dBw[:, :N]
    dC = t(C0)
    capi.spmm(algo, t(rowptr), t(colidx), t(vals), dB, dC, 0.75, -1.25)
    torch.cuda.synchronize()
    check(algo, dC.cpu().numpy(), rowptr, colidx, vals, np.ascontiguousarray(B), C0, 0.75, -1.25,
          what="beta != 0, ldb = N + 4")


@pytest.mark.parametrize("algo", PANEL_ALGOS)
def test_panels_unsorted_row_falls_back(algo, gpu):
    K, N = 131072, 128
    lens = mixed_lengths(33)
    r_uns = int(np.nonzero(lens == 5000)[0][0])
    rowptr, colidx, vals = csr_from_lengths(lens, K, seed=33, unsorted_rows={r_uns})
    B = gen.dense(13, gen.TAG_B, K, N)
    C, nl = run_nl(algo, rowptr, colidx, vals, B, gpu)
    check(algo, C, rowptr, colidx, vals, B, what="one unsorted long row")
    assert nl == np.count_nonzero(lens >= 1024) - 1, "all long rows but the unsorted one"


@pytest.mark.parametrize("algo", PANEL_ALGOS)
def test_panels_skewed_loads_fall_back(algo, gpu):
    # every long row gathers from the first 1/32 of the columns: one of the
    # 32 panels carries all the load, so the call keeps the rows on segments
    K, N = 131072, 128  # 32 panels of 4096 columns
    rng = np.random.default_rng(44)
    lens = rng.integers(0, 40, size=3000)
    lens[rng.choice(3000, size=12, replace=False)] = [2048, 2049, 2500, 3000, 3500, 4000] * 2
    narrow = {r: (0, 4096) for r in np.nonzero(lens >= 2048)[0].tolist()}
    rowptr, colidx, vals = csr_from_lengths(lens, K, seed=44, narrow=narrow)
    B = gen.dense(14, gen.TAG_B, K, N)
    C, nl = run_nl(algo, rowptr, colidx, vals, B, gpu)
    check(algo, C, rowptr, colidx, vals, B, what="skewed panel loads")
    assert nl == 0, "skewed panel loads keep every row on segments"


@pytest.mark.parametrize("algo", PANEL_ALGOS)
def test_panels_base_workspace_runs_without_panels(algo, gpu):
    K, N = 131072, 128
    lens = mixed_lengths(55)
    rowptr, colidx, vals = csr_from_lengths(lens, K, seed=55)
    B = gen.dense(15, gen.TAG_B, K, N)
    base, full = panel_bytes(algo, lens.size, K, N, colidx.size)
    assert full > base
    C_base = run(algo, rowptr, colidx, vals, B, gpu, workspace_bytes=base)
    check(algo, C_base, rowptr, colidx, vals, B, what="base-size workspace")
    C_full = run(algo, rowptr, colidx, vals, B, gpu, workspace_bytes=full)
    check(algo, C_full, rowptr, colidx, vals, B, what="panel-size workspace")
    # rows summed whole agree bit for bit whichever way the long rows went
    whole = np.diff(rowptr) <= whole_row_max(int(rowptr[-1]))
    assert np.array_equal(C_base[whole].view(np.uint32), C_full[whole].view(np.uint32))



@pytest.mark.parametrize("algo", PANEL_ALGOS)
@pytest.mark.parametrize("K", [150000, 98765])
def test_panels_odd_k(algo, K, gpu):
    # K not a power of two: the panel width is ceil(K / P) rounded up to a
    # power of two, so fewer panels than panel_count cover the columns and
    # the last one is partial
    N = 128 if K == 150000 else 256  # B of 73 / 101 MiB: 32 panels
    lens = np.minimum(mixed_lengths(K % 97), K)
    rowptr, colidx, vals = csr_from_lengths(lens, K, seed=K)
    B = gen.dense(16, gen.TAG_B, K, N)
    base, full = panel_bytes(algo, lens.size, K, N, colidx.size)
    if expects_panels(algo, N, lens.size, K, colidx.size):
        assert full > base
    C = run(algo, rowptr, colidx, vals, B, gpu)
    check(algo, C, rowptr, colidx, vals, B, what=f"K={K}")
