"""Vendor comparison bench: this library against rocSPARSE and torch.sparse on
the same seeded configs, one MI355X.

    python -m csrspmm_amd.vendor_bench [--configs medium,large,xl,rmat,rmat512]
                                       [--reps 20] [--json out.json]

The ROCm counterparts of the reference's comparison benches:
benchmarks/bench_cusparse.cu (cusparseSpMM on a CSR A, row-major B and C)
becomes rocsparse_spmm through csrspmm_amd/lib/libcsrspmm_vendor.so, and
torch_csrspmm/torch_benchmarks.py:70-74 (torch.sparse.mm) runs as is on
PyTorch-ROCm.  Every timing is C = A*B (alpha 1, beta 0) with all operands
resident on the GPU, mean over `reps` calls after warmup, HIP events on the
current stream.  rocSPARSE's preprocess stage is timed apart and excluded,
like this library's stored-plan build.  Every result, this library's and the
vendors', is compared on sampled rows (4096 spread over the matrix plus the
64 longest) with an fp64 product computed here with numpy:
max_rel_diff = max |C - R| / max |R|, and bound_frac = the largest
|C - R| / (1e-5 * max(|R|, S)) (S = sum of |a*b| per element; at most 1 passes
the library's own parity bar).  tests/test_gpu_vendor.py checks the rocSPARSE
shim against the test oracle on small cases.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))

ROCSPARSE_ALGS = {"default": 0, "csr": 1, "csr_row_split": 4, "csr_nnz_split": 5,
                  "csr_merge_path": 9}


def load_vendor():
    from csrspmm_amd import LIB_DIR

    lib = ctypes.CDLL(os.path.join(LIB_DIR, "libcsrspmm_vendor.so"))
    lib.vendor_rocsparse_version.restype = ctypes.c_int
    lib.vendor_rocsparse_spmm.restype = ctypes.c_int
    lib.vendor_rocsparse_spmm.argtypes = (
        [ctypes.c_int] * 4 + [ctypes.c_void_p] * 5 + [ctypes.c_float, ctypes.c_float] +
        [ctypes.c_int] * 3 + [ctypes.c_void_p, ctypes.POINTER(ctypes.c_double),
                              ctypes.POINTER(ctypes.c_double)])
    return lib


def sampled_rows(a, n=4096, seed=0):
    import numpy as np

    rng = np.random.default_rng(seed)
    longest = np.argsort(np.diff(a.rowptr))[-64:]
    rows = rng.choice(a.M, size=min(n, a.M), replace=False)
    return np.unique(np.concatenate([rows, longest])).astype(np.int64)


def fp64_rows(a, B, rows):
    """(R, S): the fp64 product and the per-element sum of |a*b| on `rows`."""
    import numpy as np

    R = np.zeros((rows.size, B.shape[1]))
    S = np.zeros_like(R)
    for i, r in enumerate(rows):
        lo, hi = a.rowptr[r], a.rowptr[r + 1]
        v = a.vals[lo:hi].astype(np.float64)
        Br = B[a.colidx[lo:hi]].astype(np.float64)
        R[i] = v @ Br
        S[i] = np.abs(v) @ np.abs(Br)
    return R, S


def timed(torch, fn, reps, warmup=3):
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--configs", default="medium,large,xl,rmat,rmat512")
    ap.add_argument("--reps", type=int, default=20)
    ap.add_argument("--json", default=None)
    args = ap.parse_args(argv)

    import torch  # before the vendor shim: one HIP runtime and rocSPARSE per process

    from csrspmm_amd import capi, configs

    dev = torch.device("cuda:0")
    vendor = load_vendor()
    rs_ver = vendor.vendor_rocsparse_version()
    print(f"[vendor_bench] rocSPARSE {rs_ver // 100000}.{rs_ver // 100 % 1000}.{rs_ver % 100}, "
          f"torch {torch.__version__}", flush=True)
    rows = []
    for cname in args.configs.split(","):
        cfg = configs.CONFIGS[cname]
        a = cfg.csr()
        B = cfg.B(a.K)
        N = cfg.N
        t = lambda x: torch.from_numpy(x).to(dev)  # noqa: E731
        rp, ci, va, dB = t(a.rowptr), t(a.colidx), t(a.vals), t(B)
        flops = configs.flops(a.nnz, N)
        balg = configs.bytes_alg(a.M, a.nnz, N, False)
        rows_s = sampled_rows(a)
        R, S = fp64_rows(a, B, rows_s)
        rows_d = torch.from_numpy(rows_s).to(dev)

        def row(impl, ms, C, extra=None):
            r = {"config": cname, "impl": impl, "ms": round(ms, 5),
                 "gflops": round(flops / (ms * 1e-3) / 1e9, 1),
                 "gbs_alg": round(balg / (ms * 1e-3) / 1e9, 1)}
            if C is not None:
                import numpy as np

                got = C.index_select(0, rows_d).double().cpu().numpy()
                err = np.abs(got - R)
                r["max_rel_diff"] = float(err.max() / (np.abs(R).max() or 1.0))
                r["bound_frac"] = float((err / (1e-5 * np.maximum(np.maximum(np.abs(R), S), 1e-300))).max())
            if extra:
                r.update(extra)
            rows.append(r)
            print(json.dumps(r), flush=True)

        ours_C = torch.empty((a.M, N), device=dev)
        ws = torch.empty(max(capi.hip().csrspmm_workspace_bytes_ex(capi.ALGO["Auto"], a.M, a.K, N, a.nnz, -1),
                             1), dtype=torch.uint8, device=dev)
        ms = timed(torch, lambda: capi.spmm("Auto", rp, ci, va, dB, ours_C, 1.0, 0.0, workspace=ws),
                   args.reps)
        row("csrspmm Auto (per call)", ms, ours_C)
        # with max_row_nnz, which a reference CSRMatrix carries (csrspmm::spmm passes it)
        mr = int((a.rowptr[1:] - a.rowptr[:-1]).max()) if a.M else 0
        ws_h = torch.empty(max(capi.hip().csrspmm_workspace_bytes_ex(capi.ALGO["Auto"], a.M, a.K, N, a.nnz, mr),
                               1), dtype=torch.uint8, device=dev)
        Ch = torch.empty_like(ours_C)
        ms = timed(torch, lambda: capi.spmm("Auto", rp, ci, va, dB, Ch, 1.0, 0.0, workspace=ws_h, hint=mr),
                   args.reps)
        row("csrspmm Auto (per call, max_row_nnz given)", ms, Ch)
        del Ch, ws_h
        plan = capi.Plan("Auto", rp, ci, va, a.K, n_hint=N)
        Cp = torch.empty_like(ours_C)
        ms = timed(torch, lambda: plan.spmm(dB, Cp, 1.0, 0.0), args.reps)
        row("csrspmm Auto (stored plan)", ms, Cp)
        plan.close()
        del Cp

        stream = torch.cuda.current_stream().cuda_stream
        for name, alg in ROCSPARSE_ALGS.items():
            Cv = torch.zeros_like(ours_C)
            ms_c = ctypes.c_double(0.0)
            ms_p = ctypes.c_double(0.0)
            st = vendor.vendor_rocsparse_spmm(a.M, a.K, N, a.nnz, rp.data_ptr(), ci.data_ptr(),
                                              va.data_ptr(), dB.data_ptr(), Cv.data_ptr(), 1.0, 0.0,
                                              alg, 3, args.reps, ctypes.c_void_p(stream),
                                              ctypes.byref(ms_c), ctypes.byref(ms_p))
            torch.cuda.synchronize()
            if st != 0:
                print(json.dumps({"config": cname, "impl": f"rocsparse {name}", "status": st}),
                      flush=True)
                continue
            row(f"rocsparse {name}", ms_c.value, Cv, {"preprocess_ms": round(ms_p.value, 3)})
            del Cv

        try:
            At = torch.sparse_csr_tensor(rp.long(), ci.long(), va, (a.M, a.K))
            Ct = torch.sparse.mm(At, dB)
            ms = timed(torch, lambda: torch.sparse.mm(At, dB), args.reps)
            row("torch.sparse.mm", ms, Ct)
            del At, Ct
        except RuntimeError as exc:  # an unsupported path is reported, not fatal
            print(json.dumps({"config": cname, "impl": "torch.sparse.mm", "error": str(exc)[:200]}),
                  flush=True)
        del rp, ci, va, dB, ours_C, ws
        torch.cuda.empty_cache()
    if args.json:
        with open(args.json, "w") as f:
            json.dump({"rocsparse_version": rs_ver, "torch": torch.__version__, "rows": rows}, f,
                      indent=1)
    return 0


if __name__ == "__main__":
    sys.exit(main())
