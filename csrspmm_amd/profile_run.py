"""Profiling target for rocprofv3: a fixed number of SpMM calls of one variant
on one config, and optionally a plain device copy of known size whose
FETCH_SIZE / WRITE_SIZE readings calibrate the counters.

    rocprofv3 --kernel-trace --stats -d OUT -- python3 -m csrspmm_amd.profile_run \
        --config xl --algo WarpPerRowFp4 --calls 20
    rocprofv3 --pmc FETCH_SIZE -d OUT -- python3 -m csrspmm_amd.profile_run \
        --config xl --algo WarpPerRowFp4 --calls 3 --copy-mib 1024
    rocprofv3 --kernel-trace --stats -d OUT -- python3 -m csrspmm_amd.profile_run \
        --config xl --algo Auto --plan --calls 20

With --plan the calls go through one stored plan (csrspmm_plan_*) built
before the first call.  With --no-panels each call gets a workspace of
csrspmm_workspace_bytes (the base size), which runs without per-call column
panels: the counters of the two runs show what the panels change.
"""
from __future__ import annotations

import argparse
import sys
import time


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--config", default="xl")
    ap.add_argument("--algo", default="WarpPerRowFp4")
    ap.add_argument("--calls", type=int, default=20)
    ap.add_argument("--plan", action="store_true", help="call through a stored plan")
    ap.add_argument("--no-panels", action="store_true",
                    help="pass a base-size workspace, so the call runs without column panels")
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="also run one device-to-device copy of this many MiB")
    args = ap.parse_args(argv)

    import torch

    from csrspmm_amd import capi, configs, kernel_source_digest

    dev = torch.device("cuda:0")
    cfg = configs.CONFIGS[args.config]
    a = cfg.csr()
    B = cfg.B(a.K)
    t = lambda x: torch.from_numpy(x).to(dev)  # noqa: E731
    rp, ci, va, dB = t(a.rowptr), t(a.colidx), t(a.vals), t(B)
    C = torch.empty((a.M, cfg.N), dtype=torch.float32, device=dev)
    U = configs.distinct_columns(a.colidx, a.K)
    print(f"[profile_run] {cfg.name} {args.algo} M={a.M} nnz={a.nnz} N={cfg.N} "
          f"bytes_alg={configs.bytes_alg(a.M, a.nnz, cfg.N)} "
          f"bytes_min={configs.bytes_min(a.M, a.nnz, cfg.N, U)} U={U} "
          f"sources={kernel_source_digest()}", flush=True)
    if args.copy_mib:
        n = args.copy_mib * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        print(f"[profile_run] copy of {args.copy_mib} MiB done", flush=True)
        del src, dst
    plan = None
    if args.plan:
        plan = capi.Plan(args.algo, rp, ci, va, a.K, n_hint=cfg.N)
        torch.cuda.synchronize()
        print(f"[profile_run] plan {plan.algorithm}: {plan.panelized_rows} panelized rows, "
              f"{plan.device_bytes} device bytes", flush=True)
    ws = None
    if args.no_panels:
        algo = capi.ALGO[args.algo]
        ws = torch.empty(max(capi.hip().csrspmm_workspace_bytes(algo, a.M, cfg.N, a.nnz), 1),
                         dtype=torch.uint8, device=dev)
        print(f"[profile_run] base workspace of {ws.numel()} bytes: no column panels", flush=True)
    t0 = time.perf_counter()
    for i in range(args.calls):
        if plan is not None:
            plan.spmm(dB, C, 1.0, 0.0)
        else:
            capi.spmm(args.algo, rp, ci, va, dB, C, 1.0, 0.0, workspace=ws)
    torch.cuda.synchronize()
    print(f"[profile_run] {args.calls} calls in {time.perf_counter() - t0:.3f}s", flush=True)
    if plan is not None:
        plan.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
