"""Pins the CPU oracle (oracle/) before it is trusted as the checker.

Each oracle function is checked against something it did not compute itself:
the scipy-built golden fixtures, numpy brute force on tiny inputs, closed
forms (identity, permutation, empty rows, integer exactness) and the
reference harness's known answer.  The cases are chosen so that a dropped
beta term, a wrong sign, a transposed operand or an off-by-one row bound
fails at least one of them (see test_planted_mistakes_are_caught).
"""
import numpy as np
import pytest

import oracle
from golden_cases import load, names


@pytest.mark.parametrize("name", names())
def test_f64_matches_scipy_golden(name):
    g = load(name)
    R, S = oracle.spmm_f64(g["rowptr"], g["colidx"], g["vals"], g["B"], g["C0"], g["alpha"],
                           g["beta"])
    assert R.shape == g["R"].shape
    scale = np.maximum(np.abs(g["R"]), g["S"]) + 1e-300
    assert np.max(np.abs(R - g["R"]) / scale) < 1e-12
    np.testing.assert_allclose(S, g["S"], rtol=1e-12, atol=1e-300)


@pytest.mark.parametrize("name", names())
def test_f32_restatement_within_tolerance_of_golden(name):
    g = load(name)
    C = oracle.spmm_f32_seq(g["rowptr"], g["colidx"], g["vals"], g["B"], g["C0"], g["alpha"],
                            g["beta"])
    bad, ratio, _, _ = oracle.check(C, g["R"], g["S"], 1e-5)
    assert bad == 0, ratio
    if name.startswith("integer"):
        assert np.array_equal(C.astype(np.float64), g["R"])  # exact in fp32


def _dense(rowptr, colidx, vals, K):
    M = rowptr.size - 1
    A = np.zeros((M, K), dtype=np.float64)
    for i in range(M):
        for p in range(rowptr[i], rowptr[i + 1]):
            A[i, colidx[p]] += vals[p]
    return A


def test_f64_brute_force_tiny():
    rng = np.random.default_rng(7)
    for M, K, N in [(1, 1, 1), (3, 5, 2), (6, 4, 7), (5, 9, 3)]:
        dens = (rng.random((M, K)) < 0.5) * rng.uniform(-1, 1, (M, K))
        rowptr = np.concatenate([[0], np.cumsum((dens != 0).sum(1))]).astype(np.int32)
        colidx = np.nonzero(dens)[1].astype(np.int32)
        vals = dens[dens != 0].astype(np.float32)
        B = rng.uniform(-1, 1, (K, N)).astype(np.float32)
        C0 = rng.uniform(-1, 1, (M, N)).astype(np.float32)
        for alpha, beta in [(1.0, 0.0), (-2.0, 0.5), (0.0, 3.0)]:
            want = np.zeros((M, N))
            A = _dense(rowptr, colidx, vals, K)
            for i in range(M):
                for j in range(N):
                    s = sum(A[i, k] * float(B[k, j]) for k in range(K))
                    want[i, j] = alpha * s + (beta * float(C0[i, j]) if beta != 0 else 0.0)
            R, _ = oracle.spmm_f64(rowptr, colidx, vals, B, C0, alpha, beta)
            np.testing.assert_allclose(R, want, rtol=1e-12, atol=1e-12)


def test_closed_forms():
    rng = np.random.default_rng(11)
    M = K = 37
    N = 13
    B = rng.uniform(-1, 1, (K, N)).astype(np.float32)
    C0 = rng.uniform(-1, 1, (M, N)).astype(np.float32)
    # identity: C = alpha*B + beta*C0
    rowptr = np.arange(M + 1, dtype=np.int32)
    eye_c = np.arange(M, dtype=np.int32)
    ones = np.ones(M, dtype=np.float32)
    R, _ = oracle.spmm_f64(rowptr, eye_c, ones, B, C0, 1.5, -0.25)
    np.testing.assert_allclose(R, 1.5 * B.astype(np.float64) - 0.25 * C0, rtol=1e-14)
    # permutation: row gather of B
    perm = rng.permutation(K).astype(np.int32)
    R, _ = oracle.spmm_f64(rowptr, perm, ones, B, None, 1.0, 0.0)
    assert np.array_equal(R, B[perm].astype(np.float64))
    C = oracle.spmm_f32_seq(rowptr, perm, ones, B, None, 1.0, 0.0)
    assert np.array_equal(C, B[perm])
    # all-empty A: beta*C0; beta == 0 gives exact zeros even with NaN in C0
    empty = np.zeros(M + 1, dtype=np.int32)
    z = np.zeros(0, dtype=np.int32)
    zf = np.zeros(0, dtype=np.float32)
    R, _ = oracle.spmm_f64(empty, z, zf, B, C0, 2.0, 0.5)
    np.testing.assert_array_equal(R, 0.5 * C0.astype(np.float64))
    nanC = np.full((M, N), np.nan, dtype=np.float32)
    R, _ = oracle.spmm_f64(empty, z, zf, B, nanC, 2.0, 0.0)
    assert np.all(R == 0.0)
    C = oracle.spmm_f32_seq(empty, z, zf, B, nanC, 2.0, 0.0)
    assert np.all(C == 0.0)
    # c0_zero: beta multiplies an implicit zero C, NaN beta still propagates
    R, _ = oracle.spmm_f64(rowptr, eye_c, ones, B, None, 1.0, 0.5, c0_zero=True)
    np.testing.assert_array_equal(R, B.astype(np.float64))
    C = oracle.spmm_f32_seq(rowptr, eye_c, ones, B, None, 1.0, float("nan"), c0_zero=True)
    assert np.all(np.isnan(C))
    # one full row: a dot product
    rp = np.array([0, K], dtype=np.int32)
    cols = np.arange(K, dtype=np.int32)
    v = rng.uniform(-1, 1, K).astype(np.float32)
    R, _ = oracle.spmm_f64(rp, cols, v, B, None, 1.0, 0.0)
    np.testing.assert_allclose(R[0], v.astype(np.float64) @ B.astype(np.float64), rtol=1e-12)


def test_f32_restatement_is_sequential_fma():
    # Ordering is observable: 1e8 + 1 - 1e8 in fp32 depends on the order.
    rp = np.array([0, 3], dtype=np.int32)
    cols = np.array([0, 1, 2], dtype=np.int32)
    vals = np.array([1.0, 1.0, -1.0], dtype=np.float32)
    B = np.array([[1e8], [1.0], [1e8]], dtype=np.float32)
    C = oracle.spmm_f32_seq(rp, cols, vals, B)
    s = np.float32(0)
    for a, b in zip(vals, B[:, 0]):
        s = np.float32(np.float64(a) * np.float64(b) + np.float64(s))  # exact product then one rounding
    assert C[0, 0] == s == np.float32(0.0)
    # fma keeps the low bits a separate multiply would round away
    a = np.float32(1.0 + 2.0 ** -12)
    rp1 = np.array([0, 2], dtype=np.int32)
    c1 = np.array([0, 1], dtype=np.int32)
    v1 = np.array([a, -1.0], dtype=np.float32)
    B1 = np.array([[a], [np.float32(np.float64(a) * np.float64(a))]], dtype=np.float32)
    C1 = oracle.spmm_f32_seq(rp1, c1, v1, B1)
    # fma(a, a, 0) rounds a*a once; then fma(-1, fl(a*a), acc) = 0 exactly.
    assert C1[0, 0] == 0.0


def test_row_subset_matches_full():
    rng = np.random.default_rng(3)
    g = load("ragged_64x96x33")
    rows = np.array([5, 0, 63, 3, 17], dtype=np.int32)
    Rf, Sf = oracle.spmm_f64(g["rowptr"], g["colidx"], g["vals"], g["B"], g["C0"], g["alpha"],
                             g["beta"])
    Rs, Ss = oracle.spmm_f64(g["rowptr"], g["colidx"], g["vals"], g["B"], g["C0"], g["alpha"],
                             g["beta"], rows=rows)
    np.testing.assert_array_equal(Rs, Rf[rows])
    np.testing.assert_array_equal(Ss, Sf[rows])
    Cf = oracle.spmm_f32_seq(g["rowptr"], g["colidx"], g["vals"], g["B"], g["C0"], g["alpha"],
                             g["beta"])
    Cs = oracle.spmm_f32_seq(g["rowptr"], g["colidx"], g["vals"], g["B"], g["C0"], g["alpha"],
                             g["beta"], rows=rows)
    np.testing.assert_array_equal(Cs, Cf[rows])
    del rng


def test_planted_mistakes_are_caught():
    """Each plausible oracle mistake, planted in a numpy copy of the fp64
    definition, fails the golden comparison this file relies on."""
    g = load("ragged_64x96x33")
    A = _dense(g["rowptr"], g["colidx"], g["vals"], g["K"])
    B = g["B"].astype(np.float64)
    C0 = g["C0"].astype(np.float64)
    al, be = g["alpha"], g["beta"]
    mistakes = {
        "dropped beta term": al * (A @ B),
        "wrong beta sign": al * (A @ B) - be * C0,
        "alpha on C0": al * (A @ B + be * C0),
        "off-by-one row bound": al * (np.roll(A, 1, axis=0) @ B) + be * C0,
        "column index off by one": al * (np.roll(A, 1, axis=1) @ B) + be * C0,
        "values of the wrong row": al * (A[::-1] @ B) + be * C0,
    }
    for what, R in mistakes.items():
        bad, _, _, _ = oracle.check(R.astype(np.float32), g["R"], g["S"], 1e-5)
        assert bad > 0, what
    # and the checker itself flags a single 2e-5 relative perturbation
    C = g["R"].astype(np.float32).copy()
    i = np.unravel_index(np.argmax(np.abs(g["R"])), C.shape)
    C[i] = np.float32(g["R"][i] * (1 + 2e-5))
    bad, ratio, _, worst = oracle.check(C, g["R"], g["S"], 1e-5)
    assert bad == 1 and worst == np.ravel_multi_index(i, C.shape)


def test_check_nonfinite_classes():
    R = np.array([[np.nan, np.inf, -np.inf, 1.0]])
    S = np.abs(R)
    ok = np.array([[np.nan, np.inf, -np.inf, 1.0]], dtype=np.float32)
    assert oracle.check(ok, R, S)[0] == 0
    wrong = np.array([[1.0, -np.inf, np.inf, np.nan]], dtype=np.float32)
    assert oracle.check(wrong, R, S)[0] == 4


def test_dense2csr_bit_exact_and_drops_zero_and_nan():
    rng = np.random.default_rng(5)
    D = rng.uniform(-1, 1, (50, 70)).astype(np.float32)
    D[rng.random(D.shape) < 0.6] = 0.0
    D[0, 3] = -0.0
    D[2, 5] = np.nan
    D[4, 0] = np.inf
    D[7, 9] = 1e-3
    for tol in (0.0, 0.5):
        rowptr, colidx, vals, mx = oracle.dense2csr(D, tol)
        with np.errstate(invalid="ignore"):
            keep = np.abs(D) > tol  # NaN compares false, as fabs(v) > tol does in C
        exp_rows, exp_cols = np.nonzero(keep)
        assert np.array_equal(colidx, exp_cols.astype(np.int32))
        assert np.array_equal(vals.view(np.uint32), D[keep].view(np.uint32))
        counts = keep.sum(1)
        assert np.array_equal(rowptr, np.concatenate([[0], np.cumsum(counts)]).astype(np.int32))
        assert mx == counts.max()
        assert not np.any(np.isnan(vals))
    # round trip through csr2dense (NaN and -0 come back as +0)
    rowptr, colidx, vals, _ = oracle.dense2csr(D, 0.0)
    back = oracle.csr2dense(rowptr, colidx, vals, 50, 70)
    with np.errstate(invalid="ignore"):
        expect = np.where(np.abs(D) > 0, D, np.float32(0))
    assert np.array_equal(back.view(np.uint32), expect.view(np.uint32))


def test_dense_gemm_cpu_integer_exact():
    rng = np.random.default_rng(9)
    A = rng.integers(-5, 6, (12, 20)).astype(np.float32)
    B = rng.integers(-5, 6, (20, 7)).astype(np.float32)
    C = rng.integers(-5, 6, (12, 7)).astype(np.float32)
    out = oracle.dense_gemm_cpu(A, B, C, 2.0, -3.0)
    np.testing.assert_array_equal(out, 2.0 * (A.astype(np.float64) @ B) - 3.0 * C)


def test_reference_harness_known_answer():
    """The reference's dense_init_random resets rand_r's seed to 1234 inside its
    loop (src/host/dense_utils.cpp:54-64), so every element is the same draw:
    r = 0.737751..., value -5.729746... for the range [-10, 10] (-5 as an
    integer).  Its default test run (tests/test_csrspmm.cu:15-21,73-108:
    M=N=K=1024, sparsity 0.7, integers, alpha=1, beta=0.5) therefore has a
    dense A and C = 25 * 1024 - 2.5 = 25597.5 everywhere."""
    A = oracle.dense_init_random_ref(4, 5, -10.0, 10.0, 0.0, False)
    assert np.all(A == A[0, 0]) and abs(A[0, 0] - (-5.729746)) < 1e-5
    Ai = oracle.dense_init_random_ref(1024, 1024, -10.0, 10.0, 0.7, True)
    assert np.all(Ai == -5.0)
    assert np.all(oracle.dense_init_random_ref(3, 3, -10.0, 10.0, 0.7377, True) == -5.0)
    assert np.all(oracle.dense_init_random_ref(3, 3, -10.0, 10.0, 0.7378, True) == 0.0)
    rowptr, colidx, vals, mx = oracle.dense2csr(Ai, 0.0)
    assert rowptr[-1] == 1024 * 1024 and mx == 1024
    B = np.full((1024, 64), -5.0, dtype=np.float32)  # first 64 columns are enough
    C0 = np.full((1024, 64), -5.0, dtype=np.float32)
    R, _ = oracle.spmm_f64(rowptr, colidx, vals, B, C0, 1.0, 0.5, rows=np.arange(8))
    assert np.all(R == 25597.5)
    C = oracle.spmm_f32_seq(rowptr, colidx, vals, B, C0, 1.0, 0.5, rows=np.arange(8))
    assert np.all(C == np.float32(25597.5))
    G = oracle.dense_gemm_cpu(Ai[:4], np.full((1024, 3), -5.0, np.float32),
                              np.full((4, 3), -5.0, np.float32), 1.0, 0.5)
    assert np.all(G == np.float32(25597.5))


def test_cpu_baseline_agrees_with_oracle():
    g = load("longrow_48x1200x20")
    C = np.array(g["C0"], copy=True)
    oracle.cpu_spmm_f32(g["rowptr"], g["colidx"], g["vals"], g["B"], C, g["alpha"], g["beta"])
    bad, ratio, _, _ = oracle.check(C, g["R"], g["S"], 1e-5)
    assert bad == 0, ratio
    assert oracle.cpu().cpu_spmm_max_threads() >= 1
