"""The library-owned workspaces of csrspmm_spmm_f32: released on request
(the device memory comes back and the next call still matches the oracle),
capped at 16 per process with least-recently-used eviction, and kept apart
per host thread for hipStreamPerThread, whose handle names a different stream
in every thread."""
import threading

import numpy as np
import pytest
import torch

import oracle
from csrspmm_amd import capi, gen

pytestmark = pytest.mark.gpu

HIP_STREAM_PER_THREAD = 2  # the handle value of hipStreamPerThread


def problem(M, K, per_row, N, seed):
    a = gen.uniform(M, K, per_row, seed)
    B = gen.dense(seed, gen.TAG_B, K, N)
    return a, B


def oracle_rows(a, B, C, rows):
    R, S = oracle.spmm_f64(a.rowptr, a.colidx, a.vals, B, rows=rows)
    bad, ratio, _, _ = oracle.check(C[rows], R, S, 1e-5)
    return bad, ratio


def test_release_returns_memory_and_next_call_is_exact(gpu):
    # one long row per 2048 keeps segments and partials in the workspace
    a, B = problem(8192, 4096, 300, 512, 7)
    t = lambda x: torch.from_numpy(x).to(gpu)  # noqa: E731
    rp, ci, va, dB = t(a.rowptr), t(a.colidx), t(a.vals), t(B)
    rows = np.arange(0, a.M, 37, dtype=np.int32)
    capi.release_all_workspaces()
    assert capi.owned_workspaces() == (0, 0)
    C = torch.empty(a.M, 512, device=gpu)
    capi.spmm("WarpPerRowSmemFp4", rp, ci, va, dB, C, 1.0, 0.0, owned_workspace=True)
    torch.cuda.synchronize()
    n, held = capi.owned_workspaces()
    assert n == 1 and held >= 16 << 20, (n, held)
    free_before, _ = torch.cuda.mem_get_info()
    capi.release_workspace()
    free_after, _ = torch.cuda.mem_get_info()
    assert capi.owned_workspaces() == (0, 0)
    assert free_after - free_before >= held * 0.9, (free_before, free_after, held)
    C.fill_(float("nan"))
    capi.spmm("WarpPerRowSmemFp4", rp, ci, va, dB, C, 1.0, 0.0, owned_workspace=True)
    torch.cuda.synchronize()
    bad, ratio = oracle_rows(a, B, C.cpu().numpy(), rows)
    assert bad == 0, ratio
    capi.release_workspace()  # releasing twice is a no-op
    capi.release_workspace()
    assert capi.owned_workspaces()[0] == 0


def test_cap_evicts_least_recently_used(gpu):
    a, B = problem(4096, 2048, 40, 64, 9)
    t = lambda x: torch.from_numpy(x).to(gpu)  # noqa: E731
    rp, ci, va, dB = t(a.rowptr), t(a.colidx), t(a.vals), t(B)
    rows = np.arange(0, a.M, 13, dtype=np.int32)
    capi.release_all_workspaces()
    streams = [torch.cuda.Stream() for _ in range(20)]
    outs = []
    for s in streams:
        C = torch.full((a.M, 64), float("nan"), device=gpu)
        capi.spmm("WarpPerRowSmem", rp, ci, va, dB, C, 1.0, 0.0, owned_workspace=True,
                  stream=s.cuda_stream)
        outs.append(C)
    torch.cuda.synchronize()
    assert capi.owned_workspaces()[0] == 16
    for C in outs:
        bad, ratio = oracle_rows(a, B, C.cpu().numpy(), rows)
        assert bad == 0, ratio
    capi.release_all_workspaces()
    assert capi.owned_workspaces() == (0, 0)


def test_per_thread_stream_workspaces_are_per_thread(gpu):
    """Two host threads, each on its own hipStreamPerThread, each running a
    planned product with the library-owned workspace; both exact."""
    probs = [problem(6000, 3000, 90, 128, s) for s in (21, 22)]
    t = lambda x: torch.from_numpy(x).to(gpu)  # noqa: E731
    dev = [(t(a.rowptr), t(a.colidx), t(a.vals), t(B)) for a, B in probs]
    outs = [torch.full((a.M, 128), float("nan"), device=gpu) for a, _ in probs]
    torch.cuda.synchronize()
    capi.release_all_workspaces()
    errors = []

    def run(i):
        try:
            torch.cuda.set_device(gpu)
            for _ in range(5):
                capi.spmm("Auto", *dev[i][:3], dev[i][3], outs[i], 1.0, 0.0,
                          owned_workspace=True, stream=HIP_STREAM_PER_THREAD)
            capi.check(capi.hip().csrspmm_stream_synchronize(HIP_STREAM_PER_THREAD))
        except Exception as e:  # pragma: no cover - reported below
            errors.append(e)

    th = [threading.Thread(target=run, args=(i,)) for i in range(2)]
    for x in th:
        x.start()
    for x in th:
        x.join()
    assert not errors, errors
    torch.cuda.synchronize()
    assert capi.owned_workspaces()[0] == 2
    for (a, B), C in zip(probs, outs):
        bad, ratio = oracle_rows(a, B, C.cpu().numpy(), np.arange(0, a.M, 7, dtype=np.int32))
        assert bad == 0, ratio
    capi.release_all_workspaces()
