"""The reference's own headline benchmarks, rerun on this GPU through this
library's drop-in surfaces.

* C++ sweep -- reference benchmarks/csrspmm_vs_cusparse.sh: the rebuilt
  bench_csrspmm driver (csrspmm::spmm, a device synchronisation per call,
  wall-clock timed, 200 warmup + 1000 calls) over the script's 4 shapes x 5
  densities for the five variants, GFLOPS = 2 nnz K / t
  (benchmarks/bench_csrspmm.cu:121).  Shapes read as the script passes them:
  A is M x N sparse, B is N x K.  The reference's own table is the mean over
  the 20 shapes (README.md:80-88).
* torch sweep -- reference torch_csrspmm/torch_benchmarks.py: the five torch
  forwards of torch_csrspmm, plus torch.sparse.mm / addmm, over
  its 4 shapes x 5 densities (A is M x K with a Bernoulli(density) mask, B is
  K x N), alpha 1.1, beta 0.5, each call host-timed with a synchronisation,
  mean of 100 after 20 warmups, GFLOPS = 2 nnz N / t (torch_benchmarks.py:
  31-63, 91-128; README.md:91-100 for the means).

The published means (NVIDIA GeForce RTX 4070) are printed beside ours.  The
reference's generator re-seeds per element (src/host/dense_utils.cpp:54-64),
which makes A empty or dense; its published numbers show real densities, and
this library's dense_init_random draws independent values, so the sweep runs
at the nominal densities.  rocSPARSE's SpMM (default algorithm, HIP-event
timed, no per-call synchronisation) is reported beside the C++ sweep as the
counterpart of the reference's cuSPARSE column.

    python -m csrspmm_amd.reference_sweep --out sweep_out --md profiles/reference_sweep.md
"""
from __future__ import annotations

import argparse
import csv
import ctypes
import json
import os
import re
import subprocess
import sys
import time

# (name, M, N, K) of benchmarks/csrspmm_vs_cusparse.sh:8-13 and
# torch_csrspmm/torch_benchmarks.py:15-20; densities of both.
SHAPES = [("small", 512, 1024, 64), ("medium", 1024, 2048, 128), ("large", 4096, 4096, 128),
          ("XL", 8192, 4096, 256)]
DENSITIES = [0.01, 0.05, 0.10, 0.20, 0.30]
VARIANTS = ["Naive", "WarpPerRow", "WarpPerRowSmem", "WarpPerRowFp4", "WarpPerRowSmemFp4"]

# Published means on an RTX 4070 (README.md:82-88 and 93-100).
PUBLISHED_CPP = {"WarpPerRowFp4": 727, "WarpPerRowSmemFp4": 595, "Naive": 531, "WarpPerRowSmem": 520,
                 "WarpPerRow": 444, "cuSPARSE": 488}
PUBLISHED_TORCH = {"WarpPerRowSmemFp4": 479, "WarpPerRowFp4": 466, "torch.sparse.addmm": 347,
                   "WarpPerRowSmem": 324, "Naive": 310, "WarpPerRow": 275, "torch.sparse.mm": 241}

_GFLOPS = re.compile(r"performance: \(\s*([0-9.]+)\) GFLOPS")


def cpp_sweep(lib_dir, algos, out_rows, vendor_ctx):
    exe = os.path.join(lib_dir, "bench_csrspmm")
    if not os.path.exists(exe):
        raise OSError(f"{exe} is missing: build it with `python -m csrspmm_amd.build`")
    for name, M, N, K in SHAPES:
        for dens in DENSITIES:
            spars = round(1.0 - dens, 2)
            for algo in algos:
                r = subprocess.run([exe, "-M", str(M), "-N", str(N), "-K", str(K), "-s", str(spars),
                                    "-algo", algo], capture_output=True, text=True, timeout=300)
                if r.returncode != 0:
                    raise RuntimeError(f"bench_csrspmm {name} {dens} {algo}: {r.stderr.strip()}")
                m = _GFLOPS.search(r.stdout)
                g = float(m.group(1))
                out_rows.append({"sweep": "cpp", "case": name, "M": M, "N": N, "K": K, "density": dens,
                                 "algo": algo, "gflops": g})
                print(f"[cpp] {name} d={dens} {algo}: {g:.1f} GFLOPS", flush=True)
            if vendor_ctx is not None:
                g = vendor_ctx(M, N, K, dens)
                out_rows.append({"sweep": "cpp", "case": name, "M": M, "N": N, "K": K, "density": dens,
                                 "algo": "rocSPARSE", "gflops": g})
                print(f"[cpp] {name} d={dens} rocSPARSE: {g:.1f} GFLOPS", flush=True)


def make_vendor_ctx(torch):
    """rocSPARSE default-algorithm SpMM on a matrix of the same shape and
    density (A M x N, B N x K, alpha 1, beta 0.5), GFLOPS = 2 nnz K / t."""
    from csrspmm_amd.vendor_bench import load_vendor

    vendor = load_vendor()
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)

    def run(M, N, K, dens):
        gen.manual_seed(M * 7 + N * 3 + K + int(dens * 1000))
        A = (torch.rand(M, N, device=dev, generator=gen) < dens).float() * \
            (torch.rand(M, N, device=dev, generator=gen) * 20 - 10)
        S = A.to_sparse_csr()
        rp = S.crow_indices().to(torch.int32)
        ci = S.col_indices().to(torch.int32)
        va = S.values().contiguous()
        B = torch.rand(N, K, device=dev, generator=gen) * 20 - 10
        C = torch.rand(M, K, device=dev, generator=gen) * 20 - 10
        nnz = va.numel()
        ms_c, ms_p = ctypes.c_double(0.0), ctypes.c_double(0.0)
        st = vendor.vendor_rocsparse_spmm(M, N, K, nnz, rp.data_ptr(), ci.data_ptr(), va.data_ptr(),
                                          B.data_ptr(), C.data_ptr(), 1.0, 0.5, 0, 20, 200,
                                          ctypes.c_void_p(torch.cuda.current_stream().cuda_stream),
                                          ctypes.byref(ms_c), ctypes.byref(ms_p))
        if st != 0:
            raise RuntimeError(f"rocSPARSE status {st}")
        return 2.0 * nnz * K / (ms_c.value * 1e-3) / 1e9

    return run


def torch_sweep(torch, out_rows):
    import torch_csrspmm as tc

    dev = torch.device("cuda:0")
    torch.manual_seed(0)
    alpha, beta = 1.1, 0.5

    def time_fn(fn, n_warmup=20, iters=100):
        for _ in range(n_warmup):
            fn()
            torch.cuda.synchronize()
        ts = []
        for _ in range(iters):
            t0 = time.time()
            fn()
            torch.cuda.synchronize()
            ts.append(time.time() - t0)
        return sum(ts) / len(ts)

    for name, M, N, K in SHAPES:
        for dens in DENSITIES:
            A = (torch.rand(M, K, device=dev) < dens).float() * torch.rand(M, K, device=dev)
            B = torch.rand(K, N, device=dev)
            C = torch.zeros(M, N, device=dev)
            A_csr = A.to_sparse_csr()
            nnz = A_csr.values().numel()
            row = A_csr.crow_indices().to(torch.int32)
            col = A_csr.col_indices().to(torch.int32)
            val = A_csr.values()
            mr = int((row[1:] - row[:-1]).max().item())
            fns = {
                "torch.sparse.mm": lambda: alpha * torch.sparse.mm(A_csr, B) + beta * C,
                "torch.sparse.addmm": lambda: torch.sparse.addmm(C, A_csr, B, beta=beta, alpha=alpha),
                "Naive": lambda: tc.csrspmm_naive(row, col, val, B, alpha, beta),
                "WarpPerRow": lambda: tc.csrspmm_warp_per_row(row, col, val, B, alpha, beta),
                "WarpPerRowSmem": lambda: tc.csrspmm_warp_per_row_smem(row, col, val, mr, B, alpha, beta),
                "WarpPerRowFp4": lambda: tc.csrspmm_warp_per_row_fp4(row, col, val, B, alpha, beta),
                "WarpPerRowSmemFp4": lambda: tc.csrspmm_warp_per_row_smem_fp4(row, col, val, mr, B, alpha,
                                                                             beta),
            }
            ref = (alpha * (A @ B)).float()
            for algo, fn in fns.items():
                out = fn()
                if algo not in ("torch.sparse.mm", "torch.sparse.addmm"):
                    err = float((out - ref).abs().max()) / max(float(ref.abs().max()), 1e-30)
                    if not err < 1e-4:  # the torch forwards compute alpha*A*B (beta scales zeros)
                        raise RuntimeError(f"{algo} {name} {dens}: max rel diff {err:.3g}")
                t = time_fn(fn)
                g = 2.0 * nnz * N / t / 1e9
                out_rows.append({"sweep": "torch", "case": name, "M": M, "N": N, "K": K, "density": dens,
                                 "algo": algo, "gflops": g})
                print(f"[torch] {name} d={dens} {algo}: {g:.1f} GFLOPS", flush=True)


def means(rows, sweep):
    acc = {}
    for r in rows:
        if r["sweep"] == sweep:
            acc.setdefault(r["algo"], []).append(r["gflops"])
    return {k: sum(v) / len(v) for k, v in acc.items()}


def markdown(rows, gpu_name, cmd):
    out = ["# The reference's headline sweeps on MI355X", "",
           "Command (repository root on the MI355X box):", "```", cmd, "```", "",
           f"GPU: {gpu_name}. Published numbers: the reference's README (NVIDIA GeForce RTX 4070).", ""]
    mc = means(rows, "cpp")
    if mc:
        out += ["## C++ API (reference benchmarks/csrspmm_vs_cusparse.sh, README \"Kernel-Level Performance\")",
                "", "`csrspmm::spmm` through the rebuilt `bench_csrspmm`: a device synchronisation per call, "
                "wall-clock timed over 1000 calls after 200 warmups; mean GFLOPS (2·nnz·K/t) over the 20 "
                "shapes. rocSPARSE (default algorithm) is HIP-event timed without the per-call "
                "synchronisation, which favours it.", "",
                "| variant | mean GFLOPS here | published (RTX 4070) | ratio |", "|---|---|---|---|"]
        for k in sorted(mc, key=lambda x: -mc[x]):
            pub = PUBLISHED_CPP.get(k, PUBLISHED_CPP["cuSPARSE"] if k == "rocSPARSE" else None)
            label = k if k != "rocSPARSE" else "rocSPARSE (vs the published cuSPARSE)"
            ratio = f"{mc[k] / pub:.2f}×" if pub else "—"
            out.append(f"| {label} | {mc[k]:.0f} | {pub if pub else '—'} | {ratio} |")
        out.append("")
    mt = means(rows, "torch")
    if mt:
        out += ["## Python API (reference torch_csrspmm/torch_benchmarks.py, README \"Python API Performance\")",
                "", "The five `torch_csrspmm` forwards and `torch.sparse` (on ROCm), host-timed "
                "with a synchronisation per call, mean of 100 after 20 warmups; mean GFLOPS (2·nnz·N/t) "
                "over the 20 shapes.", "",
                "| function | mean GFLOPS here | published (RTX 4070) | ratio |", "|---|---|---|---|"]
        for k in sorted(mt, key=lambda x: -mt[x]):
            pub = PUBLISHED_TORCH.get(k)
            ratio = f"{mt[k] / pub:.2f}×" if pub else "—"
            out.append(f"| {k} | {mt[k]:.0f} | {pub if pub else '—'} | {ratio} |")
        out.append("")
    out += ["## Per shape (GFLOPS)", "", "| sweep | case | density | " + " | ".join(
        sorted({r['algo'] for r in rows})) + " |", "|---|---|---|" + "---|" * len({r['algo'] for r in rows})]
    algos = sorted({r["algo"] for r in rows})
    keyed = {}
    for r in rows:
        keyed.setdefault((r["sweep"], r["case"], r["density"]), {})[r["algo"]] = r["gflops"]
    for (sw, case, dens), d in keyed.items():
        out.append(f"| {sw} | {case} | {dens} | " + " | ".join(
            f"{d[a]:.0f}" if a in d else "" for a in algos) + " |")
    return "\n".join(out) + "\n"


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--out", default="sweep_out", help="directory for the CSV and JSON")
    ap.add_argument("--md", default=None, help="also write the summary here")
    ap.add_argument("--skip-cpp", action="store_true")
    ap.add_argument("--skip-torch", action="store_true")
    ap.add_argument("--no-vendor", action="store_true", help="leave rocSPARSE out of the C++ sweep")
    args = ap.parse_args(argv)

    import torch

    from csrspmm_amd import LIB_DIR

    if not torch.cuda.is_available():
        print("reference_sweep needs a GPU", file=sys.stderr)
        return 2
    os.makedirs(args.out, exist_ok=True)
    rows = []
    if not args.skip_cpp:
        ctx = None if args.no_vendor else make_vendor_ctx(torch)
        cpp_sweep(LIB_DIR, VARIANTS + ["Auto"], rows, ctx)
    if not args.skip_torch:
        torch_sweep(torch, rows)
    with open(os.path.join(args.out, "sweep.csv"), "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["sweep", "case", "M", "N", "K", "density", "algo", "gflops"])
        w.writeheader()
        w.writerows(rows)
    summary = {"cpp_means": means(rows, "cpp"), "torch_means": means(rows, "torch"),
               "published_cpp": PUBLISHED_CPP, "published_torch": PUBLISHED_TORCH}
    with open(os.path.join(args.out, "summary.json"), "w") as f:
        json.dump(summary, f, indent=1)
    print(json.dumps(summary), flush=True)
    if args.md:
        cmd = "python -m csrspmm_amd.reference_sweep" + "".join(
            f" {a}" for a in (argv if argv is not None else sys.argv[1:]))
        with open(args.md, "w") as f:
            f.write(markdown(rows, torch.cuda.get_device_name(0), cmd))
    return 0


if __name__ == "__main__":
    sys.exit(main())
