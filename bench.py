"""Benchmark: CSR SpMM on one MI355X, C = A*B (alpha=1, beta=0).

    python bench.py [--steps K] [--warmup W] [--config xl] [--algo Auto]

A step is one SpMM call (all its launches) over the named config with every
input already resident in HBM.  W untimed steps, then K timed steps between
two torch.cuda.synchronize() calls, timed with HIP events on the launch
stream.  Prints ONE JSON line:
  value      GFLOPS = 2*nnz*N / (ms_per_step) for the headline variant
             (Auto by default: the variant the library picks from N)
  roofline   achieved gather-model GB/s of one SpMM call on the GPU (a HIP
             event pair around all of the call's launches, recorded by the
             library on the launch stream, csrspmm_timing_*) against 8 TB/s;
             traffic = measured HBM bytes per call from profiles/traffic.json
  modes      per-call median and mean of the headline variant timed alone:
             warm (back to back), api (host clock with a device sync, as the
             reference's spmm() pays) and cold (after a 512 MiB scratch write
             that flushes L2 and the MALL)
  variants   the same figures for every variant on the same config
  plan       the same figures for a stored plan (csrspmm_plan_*, Auto by
             default) built once outside the timed region, with its build
             time; the headline stays the per-call path, which needs no
             preprocessing of A
  cpu_baseline  the fp32 CSR restatement (oracle/cpu_spmm.c) on the host
             cores, full matrix, median of a bounded number of reps
The default config is the XL power-law matrix the north-star target is
stated on.  --gpus N > 1 exits: this build runs on one GPU.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)

HBM_PEAK_GBS = 8000.0
METRIC = "SpMM GFLOPS (2·nnz·N/t) + achieved HBM GB/s vs ~8 TB/s peak, per kernel"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default="xl")
    ap.add_argument("--algo", default="Auto")
    ap.add_argument("--variants", default="all", help="'all', 'none' or comma list")
    ap.add_argument("--variant-steps", type=int, default=20)
    ap.add_argument("--plan-algo", default="Auto", help="stored-plan leg ('none' disables it)")
    ap.add_argument("--mode-calls", type=int, default=30,
                    help="calls per timing mode (warm / api / cold) of the headline variant")
    ap.add_argument("--cpu-seconds", type=float, default=12.0,
                    help="time budget of the CPU baseline leg (0 disables it)")
    ap.add_argument("--traffic-file", default=os.path.join(HERE, "profiles", "traffic.json"))
    return ap.parse_args()


def time_variant(capi, torch, algo, d, steps, warmup):
    """(ms per call, main-kernel ms per call)."""
    stream = torch.cuda.current_stream()
    for _ in range(warmup):
        capi.spmm(algo, d["rowptr"], d["colidx"], d["vals"], d["B"], d["C"], 1.0, 0.0,
                  workspace=d["ws"])
    torch.cuda.synchronize()
    capi.timing_read()  # drop warmup recordings
    capi.timing_enable(True)
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record(stream)
    for _ in range(steps):
        capi.spmm(algo, d["rowptr"], d["colidx"], d["vals"], d["B"], d["C"], 1.0, 0.0,
                  workspace=d["ws"])
    stop.record(stream)
    torch.cuda.synchronize()
    capi.timing_enable(False)
    main_ms, calls = capi.timing_read()
    total_ms = start.elapsed_time(stop)
    return total_ms / steps, main_ms / max(calls, 1)


def time_modes(capi, torch, algo, d, calls, scratch_mib):
    """Per-call times of the headline variant in three modes (ms, median and
    mean over `calls` calls, each timed alone):
      warm  HIP events around one call, back to back with the previous one;
      api   host wall clock around one call plus a device synchronize, what
            the reference's spmm() (src/csrspmm.cpp:73-74) and its bench pay;
      cold  HIP events around one call after a scratch_mib MiB device write
            that evicts B, A and C from L2 and the MALL."""
    stream = torch.cuda.current_stream()

    def call():
        capi.spmm(algo, d["rowptr"], d["colidx"], d["vals"], d["B"], d["C"], 1.0, 0.0,
                  workspace=d["ws"])

    scratch = torch.empty(scratch_mib << 18, dtype=torch.float32, device=d["B"].device)
    out = {}
    for mode in ("warm", "api", "cold"):
        call()
        torch.cuda.synchronize()
        times = []
        for _ in range(calls):
            if mode == "cold":
                scratch.fill_(1.0)
            if mode == "api":
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                call()
                torch.cuda.synchronize()
                times.append((time.perf_counter() - t0) * 1e3)
            else:
                a = torch.cuda.Event(enable_timing=True)
                b = torch.cuda.Event(enable_timing=True)
                a.record(stream)
                call()
                b.record(stream)
                b.synchronize()
                times.append(a.elapsed_time(b))
        out[mode] = {"median_ms": round(statistics.median(times), 5),
                     "mean_ms": round(statistics.fmean(times), 5)}
    del scratch
    return out


def time_plan(capi, torch, algo, d, K, N, steps, warmup):
    """(plan object, build ms, ms per call, main-kernel ms per call)."""
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    plan = capi.Plan(algo, d["rowptr"], d["colidx"], d["vals"], K, n_hint=N)
    torch.cuda.synchronize()
    build_ms = (time.perf_counter() - t0) * 1e3
    for _ in range(warmup):
        plan.spmm(d["B"], d["C"], 1.0, 0.0)
    torch.cuda.synchronize()
    capi.timing_read()
    capi.timing_enable(True)
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    stream = torch.cuda.current_stream()
    start.record(stream)
    for _ in range(steps):
        plan.spmm(d["B"], d["C"], 1.0, 0.0)
    stop.record(stream)
    torch.cuda.synchronize()
    capi.timing_enable(False)
    main_ms, calls = capi.timing_read()
    return plan, build_ms, start.elapsed_time(stop) / steps, main_ms / max(calls, 1)


def cpu_baseline(a, B, budget_s):
    import numpy as np

    import oracle  # CPU baseline leg only

    C = np.empty((a.M, B.shape[1]), dtype=np.float32)
    threads = oracle.cpu().cpu_spmm_max_threads()
    oracle.cpu_spmm_f32(a.rowptr, a.colidx, a.vals, B, C, 1.0, 0.0, threads)  # warmup
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < 3 or (time.perf_counter() < t_end and len(times) < 25):
        t0 = time.perf_counter()
        oracle.cpu_spmm_f32(a.rowptr, a.colidx, a.vals, B, C, 1.0, 0.0, threads)
        times.append(time.perf_counter() - t0)
        if time.perf_counter() > t_end + 30:
            break
    t = statistics.median(times)
    return {
        "value": round(2.0 * a.nnz * B.shape[1] / t / 1e9, 3),
        "unit": "GFLOPS",
        "cores": threads,
        "kind": "port",
        "sample": f"full matrix, N={B.shape[1]}, median of {len(times)} reps "
                  f"({t * 1e3:.1f} ms/rep), fp32 CSR-order fma restatement, OpenMP "
                  f"schedule(dynamic,64), -O3 -ffast-math",
    }


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(the multi-GPU row/column split is design-only)", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    from csrspmm_amd import ALGORITHMS, capi, configs

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    cfg = configs.CONFIGS[args.config]
    t0 = time.perf_counter()
    a = cfg.csr()
    B = cfg.B(a.K)
    gen_s = time.perf_counter() - t0
    print(f"[bench] {cfg.name}: M={a.M} nnz={a.nnz} N={cfg.N} max_row={a.max_row_nnz} "
          f"(generated in {gen_s:.1f}s)", file=sys.stderr, flush=True)
    N = cfg.N
    d = {
        "rowptr": torch.from_numpy(a.rowptr).to(dev),
        "colidx": torch.from_numpy(a.colidx).to(dev),
        "vals": torch.from_numpy(a.vals).to(dev),
        "B": torch.from_numpy(B).to(dev),
        "C": torch.empty((a.M, N), dtype=torch.float32, device=dev),
    }
    need = max(capi.hip().csrspmm_workspace_bytes_ex(capi.ALGO[x], a.M, a.K, N, a.nnz, -1)
               for x in ALGORITHMS)
    d["ws"] = torch.empty(max(need, 1), dtype=torch.uint8, device=dev)
    torch.cuda.synchronize()

    flops = configs.flops(a.nnz, N)
    balg = configs.bytes_alg(a.M, a.nnz, N, False)

    def figures(ms, main_ms):
        return {
            "ms": round(ms, 5),
            "main_kernel_ms": round(main_ms, 5),
            "gflops": round(flops / (ms * 1e-3) / 1e9, 2),
            "gbs_alg": round(balg / (main_ms * 1e-3) / 1e9, 1),
            "frac": round(balg / (main_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        }

    lib = capi.hip()
    resolved = lib.csrspmm_algorithm_name(
        lib.csrspmm_resolve_algorithm(capi.ALGO[args.algo], N)).decode()
    ms, main_ms = time_variant(capi, torch, args.algo, d, args.steps, args.warmup)
    print(f"[bench] {args.algo} ({resolved}): {ms:.4f} ms/call, main kernel {main_ms:.4f} ms",
          file=sys.stderr, flush=True)

    variants = {}
    if args.variants != "none":
        names = ALGORITHMS if args.variants == "all" else args.variants.split(",")
        for name in names:
            if name == resolved:
                variants[name] = figures(ms, main_ms)
                continue
            vms, vmain = time_variant(capi, torch, name, d, args.variant_steps, 3)
            variants[name] = figures(vms, vmain)
            print(f"[bench] {name}: {vms:.4f} ms/call", file=sys.stderr, flush=True)

    modes = None
    if args.mode_calls > 0:
        modes = time_modes(capi, torch, args.algo, d, args.mode_calls, 512)
        print(f"[bench] modes: {modes}", file=sys.stderr, flush=True)

    plan_fig = None
    if args.plan_algo != "none":
        plan, build_ms, pms, pmain = time_plan(capi, torch, args.plan_algo, d, a.K, N,
                                               args.variant_steps, 3)
        plan_fig = {"algo": args.plan_algo, "resolved": plan.algorithm, **figures(pms, pmain),
                    "build_ms": round(build_ms, 2), "device_bytes": plan.device_bytes,
                    "panelized_rows": plan.panelized_rows}
        plan.close()
        print(f"[bench] plan {plan_fig['resolved']}: {pms:.4f} ms/call, main {pmain:.4f} ms, "
              f"built in {build_ms:.1f} ms", file=sys.stderr, flush=True)

    traffic = None
    if os.path.exists(args.traffic_file):
        with open(args.traffic_file) as f:
            tr = json.load(f)
        key = f"{cfg.name}/{args.algo}"
        if key in tr:
            traffic = tr[key]["bytes_per_call"]

    cpu = None
    if args.cpu_seconds > 0:
        print("[bench] cpu baseline...", file=sys.stderr, flush=True)
        cpu = cpu_baseline(a, B, args.cpu_seconds)

    achieved = balg / (main_ms * 1e-3) / 1e9
    out = {
        "metric": METRIC,
        "value": round(flops / (ms * 1e-3) / 1e9, 2),
        "unit": "GFLOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded generator, csrspmm_amd/configs.py)",
        "config": {"workload": cfg.name, "description": cfg.description, "algo": args.algo,
                   "resolved_algo": resolved,
                   "M": a.M, "K": a.K, "N": N, "nnz": a.nnz, "max_row_nnz": a.max_row_nnz,
                   "alpha": 1.0, "beta": 0.0, "bytes_alg": balg},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic, "kernel": f"{resolved}: all launches of one call",
                     "kernel_ms": round(main_ms, 5)},
        "cpu_baseline": cpu,
        "modes": modes,
        "variants": variants,
        "plan": plan_fig,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
