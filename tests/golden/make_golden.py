"""Writes the golden SpMM fixtures under tests/golden/ (run from the repo root:
``python tests/golden/make_golden.py``).

The reference ships no golden vectors or fixtures (its tests compute their
oracle on the fly), so these are built here from first principles,
independently of both the product and oracle/: inputs from numpy's PCG64 with
fixed seeds, expected outputs from scipy.sparse in float64
(``csr_matrix((vals, colidx, rowptr)) @ B``, which sums duplicate entries, as
the reference kernels do) and the epilogue C = alpha*AB + beta*C0 with C0
unread when beta == 0 (reference src/device/csrspmm_naive.cu:38).  Each case
is one .npz (no pickles) holding the inputs, alpha/beta, R (fp64 result) and
S (condition magnitude |alpha| sum |a b| + |beta c0|).
"""
from __future__ import annotations

import json
import os

import numpy as np
import scipy.sparse as sp

HERE = os.path.dirname(os.path.abspath(__file__))


def csr_from_lengths(rng, M, K, lengths, *, sorted_cols=True, allow_dup=False, integer=False):
    rowptr = np.zeros(M + 1, dtype=np.int32)
    rowptr[1:] = np.cumsum(lengths)
    cols = []
    for L in lengths:
        if allow_dup:
            c = rng.integers(0, K, size=L)
        else:
            c = rng.choice(K, size=L, replace=False)
        if sorted_cols:
            c = np.sort(c)
        cols.append(c)
    colidx = (np.concatenate(cols) if cols else np.zeros(0)).astype(np.int32)
    nnz = int(rowptr[-1])
    if integer:
        vals = rng.integers(-8, 9, size=nnz).astype(np.float32)
    else:
        vals = rng.uniform(-1, 1, size=nnz).astype(np.float32)
    return rowptr, colidx, vals


def expected(rowptr, colidx, vals, K, B, C0, alpha, beta):
    M = rowptr.size - 1
    A = sp.csr_matrix((vals.astype(np.float64), colidx, rowptr), shape=(M, K))
    Aabs = sp.csr_matrix((np.abs(vals.astype(np.float64)), colidx, rowptr), shape=(M, K))
    AB = A @ B.astype(np.float64)
    S = abs(alpha) * (Aabs @ np.abs(B.astype(np.float64)))
    R = alpha * AB
    if beta != 0.0:
        R = R + beta * C0.astype(np.float64)
        S = S + np.abs(beta * C0.astype(np.float64))
    return np.asarray(R), np.asarray(S)


def case(name, rng, M, K, N, lengths, alpha, beta, **kw):
    integer = kw.get("integer", False)
    rowptr, colidx, vals = csr_from_lengths(rng, M, K, lengths, **kw)
    if integer:
        B = rng.integers(-8, 9, size=(K, N)).astype(np.float32)
        C0 = rng.integers(-8, 9, size=(M, N)).astype(np.float32)
    else:
        B = rng.uniform(-1, 1, size=(K, N)).astype(np.float32)
        C0 = rng.uniform(-1, 1, size=(M, N)).astype(np.float32)
    R, S = expected(rowptr, colidx, vals, K, B, C0, alpha, beta)
    np.savez(os.path.join(HERE, f"{name}.npz"), rowptr=rowptr, colidx=colidx, vals=vals, B=B,
             C0=C0, alpha=np.float64(alpha), beta=np.float64(beta), K=np.int64(K), R=R, S=S)
    return dict(name=name, M=M, K=K, N=N, nnz=int(rowptr[-1]), alpha=alpha, beta=beta)


def main():
    rng = np.random.default_rng(20261201)
    cases = []
    # The reference's own test sizes (tests/test_pytorch.py:97-98): [4x4]x[4x8], [8x8]x[8x16].
    cases.append(case("tiny_4x4x8", rng, 4, 4, 8, [2, 0, 4, 1], 1.0, 1.0))
    cases.append(case("small_8x8x16", rng, 8, 8, 16, [3, 8, 0, 5, 1, 2, 7, 4], 1.0, 0.0))
    # Non-square, N % 4 != 0, empty and ragged rows, beta != 0 with a nonzero C0.
    lens = rng.integers(0, 40, size=64)
    lens[[3, 17, 40]] = 0
    cases.append(case("ragged_64x96x33", rng, 64, 96, 33, lens, 1.25, -0.5))
    # One row far past the 256-nonzero split length among short rows.
    lens = rng.integers(0, 6, size=48)
    lens[11] = 1000
    lens[30] = 257
    cases.append(case("longrow_48x1200x20", rng, 48, 1200, 20, lens, -0.75, 0.0))
    # Unsorted and duplicate column indices (accepted by the reference, summed in CSR order).
    lens = rng.integers(1, 12, size=32)
    cases.append(case("dup_unsorted_32x16x8", rng, 32, 16, 8, lens, 1.0, 2.0, sorted_cols=False,
                      allow_dup=True))
    # Integer-valued inputs: every summation order gives the exact same fp32 result.
    lens = rng.integers(0, 300, size=40)
    cases.append(case("integer_40x512x64", rng, 40, 512, 64, lens, 2.0, 3.0, integer=True))
    # N = 1 and a wide N that needs more than one column panel.
    cases.append(case("n1_16x16x1", rng, 16, 16, 1, rng.integers(0, 16, size=16), 1.0, 0.0))
    cases.append(case("wide_8x64x1100", rng, 8, 64, 1100, rng.integers(0, 64, size=8), 0.5, 0.25))
    with open(os.path.join(HERE, "cases.json"), "w") as f:
        json.dump(cases, f, indent=1)
    print(f"wrote {len(cases)} cases")


if __name__ == "__main__":
    main()
