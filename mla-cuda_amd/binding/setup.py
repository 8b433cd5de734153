"""setup.py for the `mla_custom_cuda` PyTorch-ROCm extension (the reference's module name,
setup.py:19-31 there).  Plain g++ over one C++ file: no device code and no hipify here --
the kernels live in libmla_amd.so, which this module links (rpath $ORIGIN).

Built in-tree by mla-cuda_amd/build.py (run from the package directory)."""

import os

from setuptools import setup
from torch.utils.cpp_extension import BuildExtension, CppExtension

PKG = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ROOT = os.path.dirname(PKG)

setup(
    name="mla_custom_cuda",
    ext_modules=[
        CppExtension(
            name="mla_custom_cuda",
            sources=[os.path.join(PKG, "binding", "mla_custom_cuda.cpp")],
            include_dirs=[os.path.join(ROOT, "include"), "/opt/rocm/include"],
            define_macros=[("__HIP_PLATFORM_AMD__", "1"), ("USE_ROCM", "1")],
            library_dirs=[PKG],
            libraries=["mla_amd", "c10_hip"],
            runtime_library_dirs=["$ORIGIN"],
            extra_compile_args=["-O2", "-Wall", "-Wno-unused-function"],
        )
    ],
    cmdclass={"build_ext": BuildExtension},
)
