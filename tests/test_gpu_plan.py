"""Stored plans (csrspmm_plan_*) and CSRSPMM_ALGO_AUTO on the GPU, against
the oracle: every config, repeated calls, epilogues, N larger than the
hint, and the panelized very long rows of the XL matrix."""
import numpy as np
import pytest
import torch

import oracle
from csrspmm_amd import capi, configs, gen
from test_gpu_parity import assert_parity, config_data, dev_t, sample_rows

pytestmark = pytest.mark.gpu


def plan_run(plan, B, dev, M, N, C0=None, alpha=1.0, beta=0.0, flags=0):
    dB = dev_t(B, dev)
    dC = dev_t(C0, dev) if C0 is not None else torch.full((M, N), float("nan"), device=dev)
    plan.spmm(dB, dC, alpha, beta, flags)
    torch.cuda.synchronize()
    return dC.cpu().numpy()


@pytest.mark.parametrize("algo", ["Auto", "WarpPerRowFp4", "WarpPerRowSmem", "Naive"])
@pytest.mark.parametrize("cfg_name", ["host", "medium", "large", "xl", "rmat", "rmat512"])
def test_plan_configs(cfg_name, algo, gpu):
    cfg, a, B = config_data(cfg_name)
    print(f"[plan] {cfg_name} {algo}", flush=True)
    rp, ci, va = dev_t(a.rowptr, gpu), dev_t(a.colidx, gpu), dev_t(a.vals, gpu)
    plan = capi.Plan(algo, rp, ci, va, a.K, n_hint=cfg.N)
    if algo == "Auto":
        ex = capi.hip().csrspmm_resolve_algorithm_ex(capi.ALGO["Auto"], a.M, a.K, cfg.N, a.nnz,
                                                     int(np.diff(a.rowptr).max()))
        assert plan.algorithm == capi.hip().csrspmm_algorithm_name(ex).decode()
        assert plan.algorithm in ("WarpPerRowFp4", "WarpPerRowSmemFp4", "WarpPerRowSmem")
    rows = sample_rows(a, cfg_name in ("host", "medium"))
    concrete = plan.algorithm
    shares = plan.shares(cfg.N)
    # a plan splits long rows by XCD where the per-call path would, with its
    # true longest row as the hint (R-MAT at N = 64 and 512, scalar columns)
    assert shares == capi.call_shares(concrete, a.M, a.K, cfg.N, a.nnz, int(np.diff(a.rowptr).max()))
    if cfg_name in ("rmat", "rmat512") and concrete == "WarpPerRowSmem":
        assert shares
    C1 = plan_run(plan, B, gpu, a.M, cfg.N)
    assert not np.isnan(C1).any()
    assert_parity(concrete, C1, a.rowptr, a.colidx, a.vals, B, None, 1.0, 0.0, rows=rows,
                  what=f"plan {cfg_name}", shares=shares)
    C2 = plan_run(plan, B, gpu, a.M, cfg.N)
    assert np.array_equal(C1.view(np.uint32), C2.view(np.uint32))  # deterministic, reusable
    if shares:
        # the same tables as a per-call product with the hint: the same bits
        from test_gpu_parity import run_spmm
        Cc = run_spmm(concrete, a.rowptr, a.colidx, a.vals, B, gpu,
                      hint=int(np.diff(a.rowptr).max()))
        assert np.array_equal(C1.view(np.uint32), Cc.view(np.uint32)), "plan and per-call differ"
    if cfg_name == "xl":
        # at N = 128 the warp-per-row forms, float4 and scalar, panelize XL's
        # 1501 rows of >= 1024 nonzeros; Naive has no plan to panelize
        long_rows = int(np.count_nonzero(np.diff(a.rowptr) >= 1024))
        assert plan.panelized_rows == (long_rows if concrete.startswith("WarpPerRow") else 0)
    if cfg_name == "rmat":
        assert plan.panelized_rows == 0  # skewed columns: panels would not pay
    plan.close()


def test_plan_epilogues_and_growth(gpu):
    a = gen.powerlaw(40000, 60000, 1.5, 0.7, 16000, seed=21)
    rp, ci, va = dev_t(a.rowptr, gpu), dev_t(a.colidx, gpu), dev_t(a.vals, gpu)
    plan = capi.Plan("WarpPerRowSmemFp4", rp, ci, va, a.K, n_hint=96)
    for N in (96, 32, 200, 256):  # 200: scalar fallback of the Fp4 form; 256: buffers grow
        B = gen.dense(N, gen.TAG_B, a.K, N)
        C0 = gen.dense(N, gen.TAG_C0, a.M, N)
        rows = sample_rows(a, False)
        C = plan_run(plan, B, gpu, a.M, N, C0=C0, alpha=0.5, beta=-2.0)
        assert_parity(plan.algorithm, C, a.rowptr, a.colidx, a.vals, B, C0, 0.5, -2.0, rows=rows,
                      what=f"plan beta N={N}", shares=plan.shares(N))
        C = plan_run(plan, B, gpu, a.M, N, alpha=1.5, beta=0.25, flags=capi.FLAG_C_IS_ZERO)
        assert_parity(plan.algorithm, C, a.rowptr, a.colidx, a.vals, B, None, 1.5, 0.25,
                      rows=rows, c0_zero=True, what=f"plan c_is_zero N={N}", shares=plan.shares(N))
    plan.close()


def test_plan_unsorted_long_rows_and_small_matrix(gpu):
    rng = np.random.default_rng(4)
    K = 300000
    lens = np.array([5000, 3, 0, 70000, 2100, 0, 1], dtype=np.int64)
    rowptr = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    cols = [rng.integers(0, K, L) for L in lens]
    cols[0] = np.sort(cols[0])
    cols[4] = np.sort(cols[4])          # sorted: panelized
    colidx = np.concatenate(cols).astype(np.int32)  # rows 3 unsorted: segments
    vals = rng.uniform(-1, 1, colidx.size).astype(np.float32)
    B = rng.uniform(-1, 1, (K, 64)).astype(np.float32)
    plan = capi.Plan("WarpPerRowFp4", dev_t(rowptr, gpu), dev_t(colidx, gpu), dev_t(vals, gpu), K,
                     n_hint=64)
    assert plan.panelized_rows == 2
    C = plan_run(plan, B, gpu, lens.size, 64)
    assert_parity("WarpPerRowFp4", C, rowptr, colidx, vals, B, None, 1.0, 0.0, what="unsorted", shares=False)
    plan.close()
    # tiny matrix: no stored structures, still correct
    b = gen.ragged(50, 40, 0, 20, seed=2)
    Bs = gen.dense(2, gen.TAG_B, 40, 8)
    plan = capi.Plan("Auto", dev_t(b.rowptr, gpu), dev_t(b.colidx, gpu), dev_t(b.vals, gpu), 40,
                     n_hint=8)
    C = plan_run(plan, Bs, gpu, 50, 8)
    assert_parity(plan.algorithm, C, b.rowptr, b.colidx, b.vals, Bs, None, 1.0, 0.0, what="tiny", shares=False)
    plan.close()


def test_plan_rejects_malformed_rowptr(gpu):
    rp = dev_t(np.array([0, 5, 3, 8], dtype=np.int32), gpu)
    ci = dev_t(np.zeros(8, dtype=np.int32), gpu)
    va = dev_t(np.ones(8, dtype=np.float32), gpu)
    with pytest.raises(capi.CsrspmmError) as e:
        capi.Plan("Auto", rp, ci, va, 4)
    assert e.value.status == -4


@pytest.mark.parametrize("cfg_name", ["xl", "rmat"])
def test_auto_per_call(cfg_name, gpu):
    cfg, a, B = config_data(cfg_name)
    from test_gpu_parity import run_spmm
    C = run_spmm("Auto", a.rowptr, a.colidx, a.vals, B, gpu)
    algo = capi.hip().csrspmm_algorithm_name(capi.hip().csrspmm_resolve_algorithm(6, cfg.N)).decode()
    assert_parity(algo, C, a.rowptr, a.colidx, a.vals, B, None, 1.0, 0.0, rows=sample_rows(a, False),
                  what="auto")


def test_auto_takes_scalar_lds_on_l2_sized_long_rows(gpu):
    """At N = 128 a B of at most 4 MiB with rows of 160 nonzeros or more on
    average (M >= 4096) resolves Auto to WarpPerRowSmem, per call and in a
    stored plan: bit-identical to that variant and within the oracle's bar."""
    from csrspmm_amd import gen
    M, K, N = 4096, 4096, 128
    a = gen.uniform(M, K, 200, 21)
    B = gen.dense(21, gen.TAG_B, K, N)
    ex = capi.hip().csrspmm_resolve_algorithm_ex(capi.ALGO["Auto"], M, K, N, a.nnz, -1)
    assert capi.hip().csrspmm_algorithm_name(ex).decode() == "WarpPerRowSmem"
    from test_gpu_parity import run_spmm
    C_auto = run_spmm("Auto", a.rowptr, a.colidx, a.vals, B, gpu)
    C_smem = run_spmm("WarpPerRowSmem", a.rowptr, a.colidx, a.vals, B, gpu)
    assert np.array_equal(C_auto, C_smem)
    assert_parity("WarpPerRowSmem", C_auto, a.rowptr, a.colidx, a.vals, B, None, 1.0, 0.0,
                  rows=np.arange(0, M, 7), what="auto shape rule")
    rp, ci, va = dev_t(a.rowptr, gpu), dev_t(a.colidx, gpu), dev_t(a.vals, gpu)
    plan = capi.Plan("Auto", rp, ci, va, K, n_hint=N)
    assert plan.algorithm == "WarpPerRowSmem"
    C_plan = plan_run(plan, B, gpu, M, N)
    plan.close()
    assert_parity("WarpPerRowSmem", C_plan, a.rowptr, a.colidx, a.vals, B, None, 1.0, 0.0,
                  rows=np.arange(0, M, 7), what="auto shape rule, plan", shares=False)
