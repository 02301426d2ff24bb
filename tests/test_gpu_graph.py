"""HIP graph capture of the per-call path.

A call enqueues kernels only (no memset, copy, allocation or synchronisation
once its workspace exists), so torch.cuda.CUDAGraph can record it: the torch
forwards and csrspmm_spmm_out, a stored plan's spmm_out, and the C entry
points with a caller workspace or the static no-allocation scratch.  Each
graph is recorded once and replayed three times with new B values (and, for
the in-place forms, new C values) written eagerly between the replays, every
replay checked bit for bit against an eager call on the same inputs and the
last one against the fp64 oracle at the 1e-5 bar.  The shapes take every
launch of the per-call path: the plan, the column-panel schedule (a 64 MiB
B with rows of thousands of nonzeros), the main launch and the combine, and
split rows summed in the main launch (their counters zeroed by plan_kernel
in every replay)."""
import numpy as np
import pytest
import torch

import oracle
import torch_csrspmm as tc
from csrspmm_amd import capi, gen
from csr_cases import csr_from_lengths, mixed_lengths

pytestmark = pytest.mark.gpu

TOL = 1e-5


def cases():
    # (name, rowptr, colidx, vals, K, N): long rows with column panels, and
    # short uniform rows on an L2-sized B (the plan without panels)
    K = 131072
    lens = np.minimum(mixed_lengths(91), K)
    rp, ci, va = csr_from_lengths(lens, K, seed=91)
    yield "panels", rp, ci, va, K, 128
    rng = np.random.default_rng(92)
    lens = rng.integers(0, 40, size=20000)
    rp, ci, va = csr_from_lengths(lens, 4096, seed=92)
    yield "short", rp, ci, va, 4096, 96
    # rows split into segments on a B without panels or XCD shares: summed in
    # the main launch, their counters zeroed by plan_kernel on every replay
    lens = rng.integers(0, 30, size=6000)
    lens[rng.choice(6000, 600, replace=False)] = rng.integers(300, 1000, size=600)
    rp, ci, va = csr_from_lengths(lens, 4096, seed=93)
    yield "split", rp, ci, va, 4096, 64


CASES = list(cases())


def dev(x, d):
    return torch.from_numpy(np.ascontiguousarray(x)).to(d)


def new_b(seed, K, N, d):
    return dev(gen.dense(seed, gen.TAG_B, K, N), d)


def check_oracle(C, rp, ci, va, B, C0, alpha, beta, what):
    R, S = oracle.spmm_f64(rp, ci, va, B, C0, alpha, beta)
    bad, ratio, _, _ = oracle.check(C, R, S, TOL)
    assert bad == 0, f"{what}: {bad} elements off (max ratio {ratio:.3g})"


def replay_and_check(graph, run_eager, B_static, C_static, K, N, d, what, C0_static=None,
                     oracle_check=None):
    """Three replays; before each, new B (and C0) values go into the captured
    tensors eagerly.  Each replay equals an eager call on the same inputs."""
    for rep in range(3):
        B_static.copy_(new_b(300 + rep, K, N, d))
        if C0_static is not None:
            C0_static.copy_(dev(gen.dense(400 + rep, gen.TAG_C0, C_static.shape[0], N), d))
            C0 = C0_static.clone()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = C_static.clone()
        if C0_static is not None:
            C_static.copy_(C0)
        want = run_eager()
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int32), want.view(torch.int32)), \
            f"{what}: replay {rep} differs from the eager call"
        if oracle_check is not None and rep == 2:
            oracle_check(got.cpu().numpy(), B_static.cpu().numpy(),
                         None if C0_static is None else C0.cpu().numpy())


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
@pytest.mark.parametrize("name", ["csrspmm_auto", "csrspmm_warp_per_row_fp4", "csrspmm_warp_per_row_smem"])
def test_torch_forward_in_a_graph(name, case, gpu):
    cname, rp, ci, va, K, N = case
    print(f"[graph] torch {name} {cname} M={rp.size - 1} nnz={ci.size} N={N}", flush=True)
    drp, dci, dva = dev(rp, gpu), dev(ci, gpu), dev(va, gpu)
    mx = int(np.diff(rp).max())
    fn = getattr(tc, name)
    args = (lambda B: fn(drp, dci, dva, mx, B, 1.25, 0.0)) if "smem" in name else \
           (lambda B: fn(drp, dci, dva, B, 1.25, 0.0))
    B_static = new_b(299, K, N, gpu)
    args(B_static)  # the library's first-call set-up, outside the capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        C_static = args(B_static)
    replay_and_check(g, lambda: args(B_static), B_static, C_static, K, N, gpu, f"{name} {cname}",
                     oracle_check=lambda C, B, C0: check_oracle(C, rp, ci, va, B, None, 1.25, 0.0,
                                                                f"{name} {cname}"))


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_spmm_out_and_plan_in_graphs(case, gpu):
    cname, rp, ci, va, K, N = case
    print(f"[graph] spmm_out / plan {cname} M={rp.size - 1} nnz={ci.size} N={N}", flush=True)
    M = rp.size - 1
    drp, dci, dva = dev(rp, gpu), dev(ci, gpu), dev(va, gpu)
    B_static = new_b(299, K, N, gpu)
    C_static = torch.zeros(M, N, device=gpu)
    # csrspmm_spmm_out: in place, C = 0.5 A B - 0.75 C
    tc.csrspmm_spmm_out(drp, dci, dva, B_static, C_static, 0.5, -0.75)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        tc.csrspmm_spmm_out(drp, dci, dva, B_static, C_static, 0.5, -0.75)

    def eager_out():
        C = C_static.clone()
        tc.csrspmm_spmm_out(drp, dci, dva, B_static, C, 0.5, -0.75)
        return C

    replay_and_check(g, eager_out, B_static, C_static, K, N, gpu, f"spmm_out {cname}", C0_static=C_static,
                     oracle_check=lambda C, B, C0: check_oracle(C, rp, ci, va, B, C0, 0.5, -0.75,
                                                                f"spmm_out {cname}"))
    # a stored plan: its first call for this N builds the tables, outside the capture
    plan = tc.CsrSpmmPlan(drp, dci, dva, K, n_hint=N)
    P_static = torch.zeros(M, N, device=gpu)
    plan.spmm_out(B_static, P_static, 2.0, 0.5)
    torch.cuda.synchronize()
    gp = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gp):
        plan.spmm_out(B_static, P_static, 2.0, 0.5)

    def eager_plan():
        C = P_static.clone()
        plan.spmm_out(B_static, C, 2.0, 0.5)
        return C

    replay_and_check(gp, eager_plan, B_static, P_static, K, N, gpu, f"plan {cname}", C0_static=P_static,
                     oracle_check=lambda C, B, C0: check_oracle(C, rp, ci, va, B, C0, 2.0, 0.5,
                                                                f"plan {cname}"))


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
@pytest.mark.parametrize("entry", ["ex", "noalloc"])
def test_c_entry_points_in_a_graph(entry, case, gpu):
    cname, rp, ci, va, K, N = case
    print(f"[graph] C ABI {entry} {cname} M={rp.size - 1} nnz={ci.size} N={N}", flush=True)
    M = rp.size - 1
    drp, dci, dva = dev(rp, gpu), dev(ci, gpu), dev(va, gpu)
    B_static = new_b(299, K, N, gpu)
    C_static = torch.empty(M, N, device=gpu)
    lib = capi.hip()
    need = lib.csrspmm_workspace_bytes_ex(capi.ALGO["Auto"], M, K, N, ci.size, -1)
    # the static scratch holds CSRSPMM_NOALLOC_SCRATCH_BYTES (128 MiB)
    assert lib.csrspmm_workspace_bytes(capi.ALGO["Auto"], M, N, ci.size) <= 128 << 20
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device=gpu)
    kw = dict(noalloc=True) if entry == "noalloc" else dict(workspace=ws)

    def run(C):
        capi.spmm("Auto", drp, dci, dva, B_static, C, 1.0, 0.0, **kw)
        return C

    run(C_static)  # first call on the device (the scratch address), outside the capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        run(C_static)
    replay_and_check(g, lambda: run(torch.empty_like(C_static)), B_static, C_static, K, N, gpu,
                     f"{entry} {cname}",
                     oracle_check=lambda C, B, C0: check_oracle(C, rp, ci, va, B, None, 1.0, 0.0,
                                                                f"{entry} {cname}"))
