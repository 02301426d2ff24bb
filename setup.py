"""Builds the torch extension torch_csrspmm._C, the module the reference's
setup.py builds (reference setup.py:79-86), as a CppExtension for
PyTorch-ROCm: plain C++ over the C ABI of the in-tree gfx950 kernel library.

    python -m csrspmm_amd.build hip          # the kernels: csrspmm_amd/lib/libcsrspmm_hip.so
    python setup.py build_ext --inplace      # torch_csrspmm/_C*.so, linked against it

(`python -m csrspmm_amd.build` builds everything, this module included, with
the same flags.)  No CUDAExtension and no hipify: the kernels are HIP code
built by hipcc for gfx950, and this extension only calls their C ABI.
"""
import os

from setuptools import setup

ROOT = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(ROOT, "csrspmm_amd", "lib")


def ext_modules():
    from torch.utils import cpp_extension

    return [cpp_extension.CppExtension(
        name="torch_csrspmm._C",
        sources=[os.path.join("csrspmm_amd", "csrc", "torch", "torch_csrspmm.cpp")],
        include_dirs=[os.path.join(ROOT, "include")] + cpp_extension.include_paths(device_type="cuda"),
        library_dirs=[LIB] + cpp_extension.library_paths(device_type="cuda"),
        libraries=["csrspmm_hip", "c10_hip", "torch_hip"],
        define_macros=[("__HIP_PLATFORM_AMD__", "1"), ("USE_ROCM", "1")],
        extra_compile_args=["-O2", "-std=c++17", "-Wno-deprecated-declarations"],
        extra_link_args=["-Wl,-rpath,$ORIGIN/../csrspmm_amd/lib"],
    )]


if __name__ == "__main__":
    from torch.utils.cpp_extension import BuildExtension

    if not os.path.exists(os.path.join(LIB, "libcsrspmm_hip.so")):
        raise SystemExit("build the kernels first: python -m csrspmm_amd.build hip")
    setup(
        name="torch_csrspmm",
        version="0.2.0",
        packages=["torch_csrspmm"],
        ext_modules=ext_modules(),
        cmdclass={"build_ext": BuildExtension.with_options(use_ninja=False)},
    )
