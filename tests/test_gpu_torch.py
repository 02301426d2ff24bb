"""GPU tests of the torch_csrspmm drop-in: the reference's own test cases
(tests/test_pytorch.py:94-105: [4x4]x[4x8], [8x8]x[8x16], random power-of-two
shapes, keep-mask density 0.3, alpha = beta = 1) checked against the oracle,
the beta semantics of its forwards (C allocated with zeros(), so beta scales
zero), argument checks, streams, and the XL config through the torch path."""
import numpy as np
import pytest
import torch

import torch_csrspmm as tc
import oracle
from csrspmm_amd import configs

pytestmark = pytest.mark.gpu

NAMES = ["csrspmm_naive", "csrspmm_warp_per_row", "csrspmm_warp_per_row_smem",
         "csrspmm_warp_per_row_fp4", "csrspmm_warp_per_row_smem_fp4"]


def call(name, rp, ci, va, mx, B, alpha, beta):
    fn = getattr(tc, name)
    if "smem" in name:
        return fn(rp, ci, va, mx, B, alpha, beta)
    return fn(rp, ci, va, B, alpha, beta)


def random_csr(M, K, density, rng):
    dense = rng.random((M, K)).astype(np.float32) * (rng.random((M, K)) > 1 - density)
    rp, ci, va, mx = oracle.dense2csr(dense, 0.0)
    return rp, ci, va, mx


def check(name, C, rp, ci, va, B, alpha, beta):
    R, S = oracle.spmm_f64(rp, ci, va, B, None, alpha, beta, c0_zero=True)
    bad, ratio, _, _ = oracle.check(C.cpu().numpy(), R, S, 1e-5)
    assert bad == 0, f"{name}: max ratio {ratio}"


@pytest.mark.parametrize("name", NAMES)
def test_reference_cases(name, gpu):
    rng = np.random.default_rng(2026)
    shapes = [(4, 4, 8), (8, 8, 16)] + [tuple(2 ** rng.integers(2, 11, 3)) for _ in range(5)]
    for M, K, N in shapes:
        rp, ci, va, mx = random_csr(int(M), int(K), 0.3, rng)
        B = rng.standard_normal((int(K), int(N))).astype(np.float32)
        t = lambda x: torch.from_numpy(x).to(gpu)  # noqa: E731
        C = call(name, t(rp), t(ci), t(va), mx, t(B), 1, 1)
        assert C.shape == (M, N) and C.dtype == torch.float32 and C.device == gpu
        check(name, C, rp, ci, va, B, 1.0, 1.0)


@pytest.mark.parametrize("name", NAMES)
def test_beta_scales_zero_and_nan_beta_propagates(name, gpu):
    rng = np.random.default_rng(5)
    rp, ci, va, mx = random_csr(40, 30, 0.5, rng)
    B = rng.standard_normal((30, 12)).astype(np.float32)
    t = lambda x: torch.from_numpy(x).to(gpu)  # noqa: E731
    C = call(name, t(rp), t(ci), t(va), mx, t(B), 1.5, 0.5)
    check(name, C, rp, ci, va, B, 1.5, 0.5)  # beta * 0: result is alpha*A*B
    C0 = call(name, t(rp), t(ci), t(va), mx, t(B), 1.5, 0.0)
    assert torch.equal(C, C0) or torch.allclose(C, C0, rtol=0, atol=0)
    Cn = call(name, t(rp), t(ci), t(va), mx, t(B), 1.0, float("nan"))
    assert torch.isnan(Cn).all()


@pytest.mark.parametrize("name", NAMES)
def test_argument_checks(name, gpu):
    rp = torch.tensor([0, 1, 2], dtype=torch.int32, device=gpu)
    ci = torch.tensor([0, 1], dtype=torch.int32, device=gpu)
    va = torch.ones(2, device=gpu)
    B = torch.ones(2, 4, device=gpu)
    with pytest.raises(RuntimeError, match="A_row_ptr must be int32"):
        call(name, rp.long(), ci, va, 1, B, 1.0, 0.0)
    with pytest.raises(RuntimeError, match="A_col_idx must be int32"):
        call(name, rp, ci.long(), va, 1, B, 1.0, 0.0)
    with pytest.raises(RuntimeError, match="A_values must be float32"):
        call(name, rp, ci, va.double(), 1, B, 1.0, 0.0)
    with pytest.raises(RuntimeError, match="B must be float32"):
        call(name, rp, ci, va, 1, B.half(), 1.0, 0.0)
    with pytest.raises(RuntimeError, match="row-major"):
        call(name, rp, ci, va, 1, torch.ones(4, 2, device=gpu).t(), 1.0, 0.0)
    with pytest.raises(RuntimeError, match="nnz entries"):
        call(name, rp, ci[:1], va, 1, B, 1.0, 0.0)
    # a row-major view with padding (ldb > N) is accepted
    Bp = torch.arange(2 * 8, dtype=torch.float32, device=gpu).reshape(2, 8)[:, :4]
    C = call(name, rp, ci, va, 1, Bp, 1.0, 0.0)
    assert torch.equal(C, Bp)


@pytest.mark.parametrize("name", NAMES)
def test_side_stream(name, gpu):
    rng = np.random.default_rng(3)
    rp, ci, va, mx = random_csr(300, 200, 0.2, rng)
    B = rng.standard_normal((200, 64)).astype(np.float32)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        t = lambda x: torch.from_numpy(x).to(gpu, non_blocking=False)  # noqa: E731
        C = call(name, t(rp), t(ci), t(va), mx, t(B), 1.0, 0.0)
    s.synchronize()
    check(name, C, rp, ci, va, B, 1.0, 0.0)


def test_xl_through_torch(gpu):
    cfg = configs.CONFIGS["xl"]
    a = cfg.csr()
    B = cfg.B(a.K)
    t = lambda x: torch.from_numpy(x).to(gpu)  # noqa: E731
    C = tc.csrspmm_warp_per_row_smem_fp4(t(a.rowptr), t(a.colidx), t(a.vals), a.max_row_nnz,
                                         t(B), 1.0, 0.0)
    rows = np.unique(np.concatenate([np.argsort(np.diff(a.rowptr))[-32:],
                                     np.arange(0, a.M, 97)])).astype(np.int32)
    R, S = oracle.spmm_f64(a.rowptr, a.colidx, a.vals, B, rows=rows)
    bad, ratio, _, _ = oracle.check(C.cpu().numpy()[rows], R, S, 1e-5)
    assert bad == 0, ratio


def test_auto_and_spmm_out_take_the_row_hint(gpu):
    """max_row_nnz is a scheduling hint only: given (true, or too low) or not,
    csrspmm_auto and csrspmm_spmm_out agree with the oracle, and with a hint
    of at most 256 on a mid-sized matrix (one launch, rows summed whole) bit
    for bit with the fp32 CSR-order restatement."""
    from csr_cases import csr_from_lengths
    rng = np.random.default_rng(12)
    lens = rng.integers(0, 90, 6000)
    lens[17] = 400  # longer than the too-low hint below
    rp, ci, va = csr_from_lengths(lens, 5000, seed=12)
    t = lambda x: torch.from_numpy(x).to(gpu)  # noqa: E731
    B = rng.standard_normal((5000, 128)).astype(np.float32)
    C0 = rng.standard_normal((6000, 128)).astype(np.float32)
    for mx in (-1, 400, 100):
        C = tc.csrspmm_auto(t(rp), t(ci), t(va), t(B), 1.0, 0.0, max_row_nnz=mx)
        R, S = oracle.spmm_f64(rp, ci, va, B, None, 1.0, 0.0)
        bad, ratio, _, _ = oracle.check(C.cpu().numpy(), R, S, 1e-5)
        assert bad == 0, f"auto max_row_nnz={mx}: {ratio}"
        dC = t(C0)
        tc.csrspmm_spmm_out(t(rp), t(ci), t(va), t(B), dC, 0.5, -1.25, max_row_nnz=mx)
        R, S = oracle.spmm_f64(rp, ci, va, B, C0, 0.5, -1.25)
        bad, ratio, _, _ = oracle.check(dC.cpu().numpy(), R, S, 1e-5)
        assert bad == 0, f"spmm_out max_row_nnz={mx}: {ratio}"
        if mx == 100:  # at most 256: one launch, every row summed whole
            F = oracle.spmm_f32_seq(rp, ci, va, B, None, 1.0, 0.0)
            assert np.array_equal(C.cpu().numpy().view(np.uint32), F.view(np.uint32))


def test_auto_and_spmm_out(gpu):
    rng = np.random.default_rng(11)
    rp, ci, va, mx = random_csr(500, 300, 0.1, rng)
    t = lambda x: torch.from_numpy(x).to(gpu)  # noqa: E731
    for N in (8, 64, 200, 256):
        B = rng.standard_normal((300, N)).astype(np.float32)
        C = tc.csrspmm_auto(t(rp), t(ci), t(va), t(B), 0.75, 3.0)
        check("auto", C, rp, ci, va, B, 0.75, 3.0)
        C0 = rng.standard_normal((500, N)).astype(np.float32)
        for algo in ("Auto", "Naive", "WarpPerRowFp4", "WarpPerRowSmem"):
            dC = t(C0)
            out = tc.csrspmm_spmm_out(t(rp), t(ci), t(va), t(B), dC, 0.5, -1.25, algo=algo)
            assert out.data_ptr() == dC.data_ptr()
            R, S = oracle.spmm_f64(rp, ci, va, B, C0, 0.5, -1.25)
            bad, ratio, _, _ = oracle.check(dC.cpu().numpy(), R, S, 1e-5)
            assert bad == 0, f"spmm_out {algo} N={N}: {ratio}"
    B = t(rng.standard_normal((300, 16)).astype(np.float32))
    with pytest.raises(RuntimeError, match=r"C must be \[M, N\]"):
        tc.csrspmm_spmm_out(t(rp), t(ci), t(va), B, torch.zeros(499, 16, device=gpu), 1.0, 0.0)
    with pytest.raises(RuntimeError, match="unknown algorithm"):
        tc.csrspmm_spmm_out(t(rp), t(ci), t(va), B, torch.zeros(500, 16, device=gpu), 1.0, 0.0,
                            algo="Fastest")


def test_plan_class(gpu):
    cfg = configs.CONFIGS["xl"]
    a = cfg.csr()
    B = cfg.B(a.K)
    t = lambda x: torch.from_numpy(x).to(gpu)  # noqa: E731
    plan = tc.CsrSpmmPlan(t(a.rowptr), t(a.colidx), t(a.vals), a.K, n_hint=cfg.N)
    assert plan.algorithm == "WarpPerRowFp4" and plan.panelized_rows > 0
    assert plan.device_bytes > 0
    rows = np.unique(np.concatenate([np.argsort(np.diff(a.rowptr))[-32:],
                                     np.arange(0, a.M, 97)])).astype(np.int32)
    dB = t(B)
    C = plan.spmm(dB, 1.0, 0.0)
    R, S = oracle.spmm_f64(a.rowptr, a.colidx, a.vals, B, rows=rows)
    bad, ratio, _, _ = oracle.check(C.cpu().numpy()[rows], R, S, 1e-5)
    assert bad == 0, ratio
    C2 = plan.spmm(dB, 1.0, 5.0)  # beta scales a zero C, as the forwards
    assert torch.equal(C, C2)
    plan.spmm_out(dB, C2, 1.0, -1.0)  # C - A*B: exactly zero per element
    assert float(C2.abs().max()) == 0.0
    with pytest.raises(RuntimeError, match=r"B must be \[K, N\]"):
        plan.spmm(dB[:-1], 1.0, 0.0)
