"""Build recipe for the in-tree libraries (no cmake; plain compiler lines).

    python -m csrspmm_amd.build            # all targets
    python -m csrspmm_amd.build hip host   # selected targets

Targets (outputs under csrspmm_amd/lib/ and the top-level torch_csrspmm/):
  hip    libcsrspmm_hip.so   hipcc --offload-arch=gfx950: the kernels + C ABI
  host   libcsrspmm.so       g++: C++ API (include/csrspmm/*), generators
  torch  torch_csrspmm/_C.so g++: PyTorch-ROCm extension over the C ABI (the same
                             module setup.py's CppExtension builds)
  apps   test_csrspmm, bench_csrspmm   g++: C++ drivers over libcsrspmm.so
         test_kernels_h                 hipcc: launches the kernels of <csrspmm/kernels.h>
  vendor libcsrspmm_vendor.so g++: rocSPARSE SpMM timing shim (comparison bench only)
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
LIB = os.path.join(PKG, "lib")
INC = os.path.join(ROOT, "include")

HIP_SOURCES = ["device/capi.hip", "device/rowgroup.hip", "device/naive.hip", "device/plan.hip",
               "device/panels.hip", "device/csr_tools.hip", "device/kernels_direct.hip"]
HOST_SOURCES = ["host/csrspmm.cpp", "host/spmm_launcher.cpp", "host/csr_utils.cpp",
                "host/dense_utils.cpp", "host/gen.cpp"]

# Packed-FP32 VALU ops are switched off for every HIP object.
HIPCC_FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
               "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
GXX_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function"]


def _run(cmd: list[str]) -> None:
    print("+", " ".join(cmd), flush=True)
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # hipcc's host pass reports the packed-fp32 feature as unknown: harmless.
    out = "\n".join(l for l in proc.stdout.splitlines() if "packed-fp32-ops" not in l)
    if out.strip():
        print(out, flush=True)
    if proc.returncode != 0:
        raise RuntimeError(f"build step failed ({proc.returncode}): {cmd[0]}")


def _hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found")


def build_hip() -> str:
    os.makedirs(LIB, exist_ok=True)
    objdir = os.path.join(PKG, "_build", "hip")
    os.makedirs(objdir, exist_ok=True)
    hipcc = _hipcc()
    objs = []

    def compile_one(src: str) -> str:
        obj = os.path.join(objdir, os.path.basename(src) + ".o")
        _run([hipcc, *HIPCC_FLAGS, "-I", INC, "-c", os.path.join(CSRC, src), "-o", obj])
        return obj

    with ThreadPoolExecutor(max_workers=len(HIP_SOURCES)) as ex:
        objs = list(ex.map(compile_one, HIP_SOURCES))
    out = os.path.join(LIB, "libcsrspmm_hip.so")
    _run([hipcc, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", out + ".tmp"])
    os.replace(out + ".tmp", out)
    return out


def build_host() -> str:
    os.makedirs(LIB, exist_ok=True)
    out = os.path.join(LIB, "libcsrspmm.so")
    srcs = [os.path.join(CSRC, s) for s in HOST_SOURCES]
    _run(["g++", *GXX_FLAGS, "-fopenmp", "-shared", "-I", INC, *srcs,
          "-L", LIB, "-lcsrspmm_hip", "-Wl,-rpath,$ORIGIN", "-o", out + ".tmp"])
    os.replace(out + ".tmp", out)
    return out


def build_torch() -> str:
    import torch
    from torch.utils import cpp_extension

    outdir = os.path.join(ROOT, "torch_csrspmm")
    out = os.path.join(outdir, "_C" + sysconfig.get_config_var("EXT_SUFFIX"))
    incs = cpp_extension.include_paths(device_type="cuda") + [sysconfig.get_paths()["include"], INC]
    libdirs = cpp_extension.library_paths(device_type="cuda")
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-shared",
           "-DTORCH_EXTENSION_NAME=_C", "-DTORCH_API_INCLUDE_EXTENSION_H",
           f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
           "-Wno-deprecated-declarations"]
    for i in incs:
        cmd += ["-isystem", i] if i != INC else ["-I", i]
    cmd += [os.path.join(CSRC, "torch", "torch_csrspmm.cpp")]
    for d in libdirs:
        cmd += ["-L", d]
    cmd += ["-L", LIB, "-lcsrspmm_hip", "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu",
            "-ltorch_hip", "-ltorch_python",
            "-Wl,-rpath,$ORIGIN/../csrspmm_amd/lib", "-o", out + ".tmp"]
    _run(cmd)
    os.replace(out + ".tmp", out)
    return out


def build_apps() -> list[str]:
    outs = []
    for name in ("test_csrspmm", "bench_csrspmm"):
        out = os.path.join(LIB, name)
        _run(["g++", *GXX_FLAGS, "-I", INC, os.path.join(CSRC, "apps", name + ".cpp"),
              "-L", LIB, "-lcsrspmm", "-lcsrspmm_hip", "-Wl,-rpath,$ORIGIN", "-o", out + ".tmp"])
        os.replace(out + ".tmp", out)
        outs.append(out)
    # HIP code that includes <csrspmm/kernels.h> and launches the kernels itself
    out = os.path.join(LIB, "test_kernels_h")
    _run([_hipcc(), *HIPCC_FLAGS, "-I", INC, os.path.join(CSRC, "apps", "test_kernels_h.hip"),
          "-L", LIB, "-lcsrspmm_hip", "-Wl,-rpath,$ORIGIN", "-o", out + ".tmp"])
    os.replace(out + ".tmp", out)
    outs.append(out)
    return outs


def build_vendor() -> str:
    out = os.path.join(LIB, "libcsrspmm_vendor.so")
    _run(["g++", *GXX_FLAGS, "-shared", "-D__HIP_PLATFORM_AMD__=1", "-isystem", "/opt/rocm/include",
          os.path.join(CSRC, "vendor", "rocsparse_spmm_bench.cpp"), "-L", "/opt/rocm/lib",
          "-lrocsparse", "-lamdhip64", "-Wl,-rpath,/opt/rocm/lib", "-o", out + ".tmp"])
    os.replace(out + ".tmp", out)
    return out


TARGETS = {"hip": build_hip, "host": build_host, "torch": build_torch, "apps": build_apps,
           "vendor": build_vendor}


def build(targets: list[str] | None = None) -> None:
    for t in targets or list(TARGETS):
        TARGETS[t]()


if __name__ == "__main__":
    build(sys.argv[1:] or None)
