"""Benchmark: CSR SpMM on one MI355X, C = A*B (alpha=1, beta=0).

    python bench.py [--steps K] [--warmup W] [--config xl] [--algo Auto]

A step is one SpMM call (all its launches) over the named config with every
input already resident in HBM.  W untimed steps, then K timed steps between
two torch.cuda.synchronize() calls, timed with HIP events on the launch
stream.  Prints ONE JSON line:
  value      GFLOPS = 2*nnz*N / (ms_per_step) for the headline variant
             (Auto by default: the variant the library picks from N)
  roofline   measured HBM bytes of one SpMM call (rocprofv3 FETCH_SIZE and
             WRITE_SIZE, calibrated on a device copy: profiles/traffic.json)
             over the GPU time of that call (a HIP event pair around all of
             the call's launches, recorded by the library on the launch
             stream, csrspmm_timing_*, on every TIMING_EVERY-th call of the
             timed loop), against 8 TB/s.  Beside it, never in
             its place: the compulsory fraction (each distinct B row read
             once) and the gather-model figure (a full B row per nonzero,
             above 1 when B is served from L2 or the MALL).  traffic.json
             records the kernel-source digest it was measured on; a
             mismatch with the sources being benched is flagged.  Also from
             traffic.json: the L2 (TCC) busy fraction of the main kernel and
             of the whole call (TCC_BUSY_avr over GRBM_GUI_ACTIVE per XCD),
             the bound these gather kernels run against
  modes      per-call median and mean of the headline variant timed alone:
             warm (back to back), api (host clock with a device sync, as the
             reference's spmm() pays) and cold (after a 512 MiB scratch write
             that flushes L2 and the MALL)
  variants   the same figures for every variant on the same config
  configs    per-variant ms, GFLOPS and (where profiles/traffic.json holds
             the key) measured HBM fraction of Auto and every variant on the
             other BASELINE configs (medium, large, rmat, rmat512 by default)
  plan       the same figures for a stored plan (csrspmm_plan_*, Auto by
             default) built once outside the timed region, with its build
             time; the headline stays the per-call path, which needs no
             preprocessing of A
  cpu_baseline  the fp32 CSR restatement (oracle/cpu_spmm.c) on the host
             cores, full matrix, median of a bounded number of reps, on all
             threads and on one; the CPU model; and the reference's own dense
             CPU GEMM (src/host/dense_utils.cpp:109-126) on the host config
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
    ap.add_argument("--configs", default="medium,large,rmat,rmat512",
                    help="per-config leg: comma list of other configs ('none' disables it)")
    ap.add_argument("--plan-algo", default="Auto", help="stored-plan leg ('none' disables it)")
    ap.add_argument("--mode-calls", type=int, default=30,
                    help="calls per timing mode (warm / api / cold) of the headline variant")
    ap.add_argument("--cpu-seconds", type=float, default=12.0,
                    help="time budget of the CPU baseline leg (0 disables it)")
    ap.add_argument("--traffic-file", default=os.path.join(HERE, "profiles", "traffic.json"))
    return ap.parse_args()


def load_config(capi, torch, cfg, dev, algos):
    """(csr, B on the host, device inputs + a workspace for every algo)."""
    a = cfg.csr()
    B = cfg.B(a.K)
    N = cfg.N
    d = {
        "rowptr": torch.from_numpy(a.rowptr).to(dev),
        "colidx": torch.from_numpy(a.colidx).to(dev),
        "vals": torch.from_numpy(a.vals).to(dev),
        "B": torch.from_numpy(B).to(dev),
        "C": torch.empty((a.M, N), dtype=torch.float32, device=dev),
    }
    need = max(capi.hip().csrspmm_workspace_bytes_ex(capi.ALGO[x], a.M, a.K, N, a.nnz, -1)
               for x in algos)
    d["ws"] = torch.empty(max(need, 1), dtype=torch.uint8, device=dev)
    torch.cuda.synchronize()
    return a, B, d


def figures(cfg, a, ms, main_ms, traffic_file, key=None, bmin=None, balg=None):
    """GFLOPS and HBM fractions of one timed variant on one config."""
    from csrspmm_amd import configs

    flops = configs.flops(a.nnz, cfg.N)
    f = {
        "ms": round(ms, 5),
        "main_kernel_ms": round(main_ms, 5),
        "gflops": round(flops / (ms * 1e-3) / 1e9, 2),
    }
    if bmin is not None:
        f["compulsory_frac"] = round(bmin / (main_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)
    if balg is not None:
        f["gather_model_gbs"] = round(balg / (main_ms * 1e-3) / 1e9, 1)
    if key is not None:
        e, fresh = traffic_entry(traffic_file, key)
        if e is not None:
            gbs = e["bytes_per_call"] / (main_ms * 1e-3) / 1e9
            f["measured_gbs"] = round(gbs, 1)
            f["measured_frac"] = round(gbs / HBM_PEAK_GBS, 4)
            f["traffic_current"] = fresh
            if e.get("l2_busy_main") is not None:
                f["l2_busy_main"] = e["l2_busy_main"]
    return f


def config_leg(capi, torch, name, dev, args):
    """Auto and every variant on one more config: {algo: figures}."""
    from csrspmm_amd import ALGORITHMS, configs

    cfg = configs.CONFIGS[name]
    t0 = time.perf_counter()
    a, _, d = load_config(capi, torch, cfg, dev, ALGORITHMS)
    lib = capi.hip()
    resolved = lib.csrspmm_algorithm_name(
        lib.csrspmm_resolve_algorithm_ex(capi.ALGO["Auto"], a.M, a.K, cfg.N, a.nnz, -1)).decode()
    out = {"M": a.M, "K": a.K, "N": cfg.N, "nnz": a.nnz, "resolved_auto": resolved, "algos": {}}
    for algo in ("Auto",) + tuple(ALGORITHMS):
        ms, main_ms = time_variant(capi, torch, algo, d, args.variant_steps, 3)
        out["algos"][algo] = figures(cfg, a, ms, main_ms, args.traffic_file, f"{name}/{algo}")
    del d
    torch.cuda.empty_cache()
    out["seconds"] = round(time.perf_counter() - t0, 1)
    print(f"[bench] config {name}: Auto ({resolved}) {out['algos']['Auto']['ms']:.4f} ms/call, "
          f"leg {out['seconds']} s", file=sys.stderr, flush=True)
    return out


# The library's span events are recorded on one call in TIMING_EVERY of a
# timed loop: each recording adds two marker packets to the stream, which cost
# about 8 us of GPU time per call on medium (48.4 against 40.6 us per call
# back to back), so recording every call inflated the per-call times of the
# short configs.
TIMING_EVERY = 8


def time_variant(capi, torch, algo, d, steps, warmup):
    """(ms per call, main-kernel ms per call)."""
    stream = torch.cuda.current_stream()
    for _ in range(warmup):
        capi.spmm(algo, d["rowptr"], d["colidx"], d["vals"], d["B"], d["C"], 1.0, 0.0,
                  workspace=d["ws"])
    torch.cuda.synchronize()
    capi.timing_read()  # drop warmup recordings
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record(stream)
    for i in range(steps):
        capi.timing_enable(i % TIMING_EVERY == 0)
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
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    stream = torch.cuda.current_stream()
    start.record(stream)
    for i in range(steps):
        capi.timing_enable(i % TIMING_EVERY == 0)
        plan.spmm(d["B"], d["C"], 1.0, 0.0)
    stop.record(stream)
    torch.cuda.synchronize()
    capi.timing_enable(False)
    main_ms, calls = capi.timing_read()
    return plan, build_ms, start.elapsed_time(stop) / steps, main_ms / max(calls, 1)


def _median_reps(fn, budget_s, min_reps=3, max_reps=25):
    """Median seconds of fn() after one warmup: at least min_reps, more while
    the budget lasts (at most max_reps)."""
    fn()
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < min_reps or (time.perf_counter() < t_end and len(times) < max_reps):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times), len(times)


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(a, B, budget_s):
    """The fp32 CSR restatement of the reference kernels on the host cores
    (all threads the OpenMP runtime grants, and one), plus the reference's
    dense CPU GEMM on the host config."""
    import numpy as np

    import oracle  # CPU baseline leg only

    from csrspmm_amd import configs, gen

    N = B.shape[1]
    C = np.empty((a.M, N), dtype=np.float32)
    threads = oracle.cpu().cpu_spmm_max_threads()
    spmm = lambda nt: oracle.cpu_spmm_f32(a.rowptr, a.colidx, a.vals, B, C, 1.0, 0.0, nt)  # noqa: E731
    t_all, n_all = _median_reps(lambda: spmm(threads), budget_s * 0.6)
    t_one, n_one = _median_reps(lambda: spmm(1), budget_s * 0.4, min_reps=3, max_reps=5)
    # the reference's only CPU product: dense O(M*K*N) GEMM, host config
    host = configs.CONFIGS["host"]
    ha = host.csr()
    Ad = np.zeros((ha.M, ha.K), dtype=np.float32)
    rows = np.repeat(np.arange(ha.M), np.diff(ha.rowptr))
    Ad[rows, ha.colidx] = ha.vals
    Bh = gen.dense(host.seed, gen.TAG_B, ha.K, host.N)
    Ch = np.zeros((ha.M, host.N), dtype=np.float32)
    t_gemm, n_gemm = _median_reps(lambda: oracle.cpu_dense_gemm(Ad, Bh, Ch, 1.0, 0.0), 1.0,
                                  min_reps=5, max_reps=20)
    gf = lambda t: round(2.0 * a.nnz * N / t / 1e9, 3)  # noqa: E731
    return {
        "value": gf(t_all),
        "unit": "GFLOPS",
        "cores": threads,
        "kind": "port",
        "sample": f"full matrix, N={N}, median of {n_all} reps ({t_all * 1e3:.1f} ms/rep) on "
                  f"{threads} threads; fp32 CSR-order fma restatement of the reference kernels, "
                  f"OpenMP schedule(dynamic,64), -O3 -ffast-math -march=x86-64-v3",
        "cpu_model": cpu_model(),
        "one_thread": {"value": gf(t_one), "unit": "GFLOPS", "ms": round(t_one * 1e3, 2),
                       "reps": n_one},
        "reference_dense_gemm_host": {
            "what": "the reference's dense_gemm_cpu (src/host/dense_utils.cpp:109-126), 1 thread, "
                    "on the host config: dense A 1024x1024 (its 10,240 nonzeros and zeros), "
                    "B 1024x32",
            "ms": round(t_gemm * 1e3, 3), "reps": n_gemm,
            "dense_gflops": round(2.0 * ha.M * ha.K * host.N / t_gemm / 1e9, 3),
            "sparse_equivalent_gflops": round(2.0 * ha.nnz * host.N / t_gemm / 1e9, 4)},
    }


def traffic_entry(path, key):
    """(entry of profiles/traffic.json for key or None, digest matches?)."""
    from csrspmm_amd import kernel_source_digest

    if not os.path.exists(path):
        return None, False
    with open(path) as f:
        tr = json.load(f)
    e = tr.get(key)
    if e is None:
        return None, False
    return e, e.get("source_digest") == kernel_source_digest()


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
    a, B, d = load_config(capi, torch, cfg, dev, ALGORITHMS)
    gen_s = time.perf_counter() - t0
    print(f"[bench] {cfg.name}: M={a.M} nnz={a.nnz} N={cfg.N} max_row={a.max_row_nnz} "
          f"(generated and uploaded in {gen_s:.1f}s)", file=sys.stderr, flush=True)
    N = cfg.N

    flops = configs.flops(a.nnz, N)
    balg = configs.bytes_alg(a.M, a.nnz, N, False)
    U = configs.distinct_columns(a.colidx, a.K)
    bmin = configs.bytes_min(a.M, a.nnz, N, U, False)

    def fig(ms, main_ms, key=None):
        return figures(cfg, a, ms, main_ms, args.traffic_file, key, bmin, balg)

    lib = capi.hip()
    resolved = lib.csrspmm_algorithm_name(
        lib.csrspmm_resolve_algorithm_ex(capi.ALGO[args.algo], a.M, a.K, N, a.nnz, -1)).decode()
    ms, main_ms = time_variant(capi, torch, args.algo, d, args.steps, args.warmup)
    print(f"[bench] {args.algo} ({resolved}): {ms:.4f} ms/call, main kernel {main_ms:.4f} ms",
          file=sys.stderr, flush=True)

    variants = {}
    if args.variants != "none":
        names = ALGORITHMS if args.variants == "all" else args.variants.split(",")
        for name in names:
            if name == resolved:
                variants[name] = fig(ms, main_ms, f"{cfg.name}/{args.algo}")
                continue
            vms, vmain = time_variant(capi, torch, name, d, args.variant_steps, 3)
            variants[name] = fig(vms, vmain, f"{cfg.name}/{name}")
            print(f"[bench] {name}: {vms:.4f} ms/call", file=sys.stderr, flush=True)

    modes = None
    if args.mode_calls > 0:
        modes = time_modes(capi, torch, args.algo, d, args.mode_calls, 512)
        print(f"[bench] modes: {modes}", file=sys.stderr, flush=True)

    plan_fig = None
    if args.plan_algo != "none":
        plan, build_ms, pms, pmain = time_plan(capi, torch, args.plan_algo, d, a.K, N,
                                               args.variant_steps, 3)
        plan_fig = {"algo": args.plan_algo, "resolved": plan.algorithm,
                    **fig(pms, pmain, f"{cfg.name}/plan{args.plan_algo}"),
                    "build_ms": round(build_ms, 2), "device_bytes": plan.device_bytes,
                    "panelized_rows": plan.panelized_rows}
        plan.close()
        print(f"[bench] plan {plan_fig['resolved']}: {pms:.4f} ms/call, main {pmain:.4f} ms, "
              f"built in {build_ms:.1f} ms", file=sys.stderr, flush=True)

    per_config = {}
    if args.configs != "none":
        del d  # the headline config's device inputs
        torch.cuda.empty_cache()
        for name in args.configs.split(","):
            if name and name != cfg.name:
                per_config[name] = config_leg(capi, torch, name, dev, args)

    from csrspmm_amd import kernel_source_digest

    tr, tr_fresh = traffic_entry(args.traffic_file, f"{cfg.name}/{args.algo}")
    traffic = tr["bytes_per_call"] if tr is not None else None

    cpu = None
    if args.cpu_seconds > 0:
        print("[bench] cpu baseline...", file=sys.stderr, flush=True)
        cpu = cpu_baseline(a, B, args.cpu_seconds)

    t_s = main_ms * 1e-3
    if traffic is not None:
        # measured HBM-side bytes of one call over its GPU time
        achieved, basis = traffic / t_s / 1e9, "measured traffic (rocprofv3 FETCH_SIZE + WRITE_SIZE)"
    else:
        achieved, basis = bmin / t_s / 1e9, "compulsory bytes (no traffic measurement for this key)"
    roofline = {
        "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic, "frac_basis": basis,
        "traffic_source_digest": tr.get("source_digest") if tr else None,
        "kernel_source_digest": kernel_source_digest(),
        "traffic_current": bool(tr_fresh),
        "compulsory_bytes": bmin, "distinct_columns": U,
        "compulsory_frac": round(bmin / t_s / 1e9 / HBM_PEAK_GBS, 4),
        "gather_model_bytes": balg,
        "gather_model_gbs": round(balg / t_s / 1e9, 1),
        "kernel": f"{resolved}: all launches of one call", "kernel_ms": round(main_ms, 5),
        # the bound the counters show: the main kernel's L2 (TCC) busy fraction
        "l2_busy_main": tr.get("l2_busy_main") if tr else None,
        "l2_busy_main_kernel": tr.get("l2_busy_main_kernel") if tr else None,
        "l2_busy_call": tr.get("l2_busy_call") if tr else None}
    if traffic is not None and not tr_fresh:
        print("[bench] WARNING: profiles/traffic.json was measured on other kernel sources "
              f"({roofline['traffic_source_digest']} vs {roofline['kernel_source_digest']})",
              file=sys.stderr, flush=True)

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
                   "alpha": 1.0, "beta": 0.0},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "modes": modes,
        "variants": variants,
        "plan": plan_fig,
        "configs": per_config,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
