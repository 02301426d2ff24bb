"""GPU parity of split rows summed in the main launch (Problem::seg_fuse).

A per-call product with a plan and no column panels or XCD shares sums its
split rows (two segments or more) in the main launch: every segment stores
its partial row past the L2 and counts itself in a per-row counter that
plan_kernel zeroes, and the last segment's group (over every column slice)
adds the row's partials in the order of the combine kernel, which a stored
plan still launches.  So per call and through a stored plan the split rows
must agree bit for bit, and both must meet the oracle's bar.

The shapes keep every row under 1024 nonzeros (a stored plan cuts longer rows
into column panels, summed in another order) and every matrix under 2^20
nonzeros (no XCD shares); with fewer than 4096 segments' worth of nonzeros
the segment shrinks (to 32 at the smallest), so rows of a few hundred
nonzeros split into many segments.  Cases: unsliced float4 and scalar
columns, XCD slices (16384 x 128), column slices launched one by one (K =
65536, N = 256: a row's segments count over four slices), the alpha/beta
epilogue, N = 1 (the combine's 8-lane groups, eight strided sums) and
N = 600 (64-lane groups, one sum over every partial), and two calls in a row
(the counters start from zero each call).

Bar: 1e-5 against the fp64 oracle on every element; split rows bit for bit
between the per-call and the stored-plan products.
"""
import numpy as np
import pytest
import torch

import oracle
from csrspmm_amd import capi, gen
from csr_cases import csr_from_lengths

pytestmark = pytest.mark.gpu

TOL = 1e-5
VARIANTS = ["WarpPerRow", "WarpPerRowFp4", "WarpPerRowSmem", "WarpPerRowSmemFp4", "Auto"]


def t(x, dev):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


def lengths(M, seed):
    """Short rows with one in five split: 33 to 1000 nonzeros."""
    rng = np.random.default_rng(seed)
    lens = rng.integers(0, 24, size=M)
    split = rng.choice(M, size=M // 5, replace=False)
    lens[split] = rng.integers(33, 1001, size=split.size)
    lens[0], lens[-1] = 1000, 777  # the first and the last row split
    return lens


def per_call(algo, rp, ci, va, B, dev, C0, alpha, beta):
    dC = t(C0, dev)
    capi.spmm(algo, t(rp, dev), t(ci, dev), t(va, dev), t(B, dev), dC, alpha, beta)
    torch.cuda.synchronize()
    return dC.cpu().numpy()


@pytest.mark.parametrize("M,K,N", [(4000, 4096, 64), (3000, 16384, 128), (2500, 65536, 256),
                                   (3000, 8192, 36), (3000, 4096, 1), (1500, 4096, 600)])
@pytest.mark.parametrize("algo", VARIANTS)
def test_fused_split_rows(algo, M, K, N, gpu):
    lens = lengths(M, seed=K + N)
    rp, ci, va = csr_from_lengths(lens, K, seed=N)
    assert int(rp[-1]) < (1 << 20)
    B = gen.dense(N, gen.TAG_B, K, N)
    C0 = gen.dense(N, gen.TAG_C0, M, N)
    alpha, beta = (0.5, -1.5) if N % 2 == 0 else (1.0, 0.0)
    assert not capi.call_shares(algo, M, K, N, int(rp[-1]))
    print(f"[fused] {algo} M={M} K={K} N={N} nnz={int(rp[-1])}", flush=True)
    C = per_call(algo, rp, ci, va, B, gpu, C0, alpha, beta)
    R, S = oracle.spmm_f64(rp, ci, va, B, C0 if beta != 0.0 else None, alpha, beta)
    bad, ratio, _, _ = oracle.check(C, R, S, TOL)
    assert bad == 0, f"{algo}: {bad} elements off (max ratio {ratio:.3g})"
    # again: the counters start from zero on every call
    C2 = per_call(algo, rp, ci, va, B, gpu, C0, alpha, beta)
    assert np.array_equal(C.view(np.uint32), C2.view(np.uint32)), "two calls differ"
    # the stored plan sums its split rows in the combine launch
    plan = capi.Plan(algo, t(rp, gpu), t(ci, gpu), t(va, gpu), K, n_hint=N)
    assert plan.panelized_rows == 0
    dC = t(C0, gpu)
    plan.spmm(t(B, gpu), dC, alpha, beta)
    torch.cuda.synchronize()
    Cp = dC.cpu().numpy()
    plan.close()
    assert np.array_equal(C.view(np.uint32), Cp.view(np.uint32)), \
        f"{algo}: per-call and stored-plan products differ " \
        f"({int((C.view(np.uint32) != Cp.view(np.uint32)).any(axis=1).sum())} rows)"
