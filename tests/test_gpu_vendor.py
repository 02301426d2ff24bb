"""The rocSPARSE comparison shim (csrspmm_amd/csrc/vendor/rocsparse_spmm_bench.cpp,
the ROCm counterpart of the reference's cusparseSpMM loop,
benchmarks/bench_cusparse.cu:182-194) against the oracle, for every rocSPARSE
algorithm the vendor bench times: C = alpha*A*B + beta*C0 with beta != 0 and
N % 4 != 0, one compute call (no warmup, so C0 is scaled once).  The
vendor numbers in profiles/vendor_comparison.md are only worth comparing if
the vendor path computes the same product."""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from csrspmm_amd import gen
from csrspmm_amd.vendor_bench import ROCSPARSE_ALGS, load_vendor

pytestmark = pytest.mark.gpu

CASES = [
    # (M, K, N, min_len, max_len, alpha, beta, seed): rows short enough that
    # any fp32 summation order stays inside the 1e-5 condition-scaled bound
    (300, 200, 13, 0, 60, 1.5, -0.75, 41),
    (2000, 5000, 37, 0, 90, 0.5, 2.0, 42),
]


@pytest.mark.parametrize("case", CASES, ids=["300x200x13", "2000x5000x37"])
@pytest.mark.parametrize("alg", sorted(ROCSPARSE_ALGS))
def test_rocsparse_shim_against_oracle(case, alg, gpu):
    M, K, N, lo, hi, alpha, beta, seed = case
    a = gen.ragged(M, K, lo, hi, seed=seed)
    B = gen.dense(seed, gen.TAG_B, K, N)
    C0 = gen.dense(seed, gen.TAG_C0, M, N)
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(gpu)  # noqa: E731
    rp, ci, va, dB, dC = t(a.rowptr), t(a.colidx), t(a.vals), t(B), t(C0)
    vendor = load_vendor()
    ms_c, ms_p = ctypes.c_double(0.0), ctypes.c_double(0.0)
    st = vendor.vendor_rocsparse_spmm(M, K, N, a.nnz, rp.data_ptr(), ci.data_ptr(), va.data_ptr(),
                                      dB.data_ptr(), dC.data_ptr(), alpha, beta,
                                      ROCSPARSE_ALGS[alg], 0, 1,
                                      ctypes.c_void_p(torch.cuda.current_stream().cuda_stream),
                                      ctypes.byref(ms_c), ctypes.byref(ms_p))
    torch.cuda.synchronize()
    assert st == 0, f"rocsparse {alg}: status {st}"
    R, S = oracle.spmm_f64(a.rowptr, a.colidx, a.vals, B, C0, alpha, beta)
    bad, ratio, _, _ = oracle.check(dC.cpu().numpy(), R, S, 1e-5)
    assert bad == 0, f"rocsparse {alg}: {bad} elements off, max ratio {ratio}"
