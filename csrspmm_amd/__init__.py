"""csrspmm_amd: CSR sparse x dense matrix multiplication for AMD Instinct
MI355X (gfx950), C = alpha * A * B + beta * C with A in CSR (int32 indices,
fp32 values) and row-major fp32 B and C.

Surfaces:
  include/csrspmm_c.h         C ABI (libcsrspmm_hip.so: kernels + launch)
  include/csrspmm/*.h         drop-in C++ API of the reference (libcsrspmm.so)
  torch_csrspmm (top level)   drop-in torch entry points (torch_csrspmm/_C)
  csrspmm_amd.capi            ctypes view of the C ABI (tests, benchmarks)
  csrspmm_amd.gen / configs   seeded synthetic inputs and the benchmark configs
"""
import os

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.join(PKG_DIR, "lib")

ALGORITHMS = ("Naive", "NaiveSmem", "WarpPerRow", "WarpPerRowFp4", "WarpPerRowSmem",
              "WarpPerRowSmemFp4")
# The five variants the reference's torch package exposes (torch_csrspmm/__init__.py:10-23).
TORCH_ALGORITHMS = ("Naive", "WarpPerRow", "WarpPerRowSmem", "WarpPerRowFp4", "WarpPerRowSmemFp4")

__version__ = "0.2.0"


def kernel_source_digest() -> str:
    """SHA-256 (first 16 hex digits) of the HIP sources and headers the
    kernels are built from (csrc/device/ and include/csrspmm_c.h).  Measured
    counter figures (profiles/traffic.json) carry the digest of the sources
    they were measured on, so that bench.py can tell when they are stale."""
    import hashlib

    h = hashlib.sha256()
    dev = os.path.join(PKG_DIR, "csrc", "device")
    files = sorted(os.path.join(dev, f) for f in os.listdir(dev)
                   if f.endswith((".hip", ".h", ".hpp")))
    files.append(os.path.join(os.path.dirname(PKG_DIR), "include", "csrspmm_c.h"))
    for path in files:
        h.update(os.path.relpath(path, os.path.dirname(PKG_DIR)).encode())
        with open(path, "rb") as f:
            h.update(f.read())
    return h.hexdigest()[:16]
