"""Build the two in-tree artefacts of the package, for gfx950 only:

1. ``libmla_amd.so``  -- the HIP kernels and the C ABI of include/mla/mla.h, compiled with
   hipcc --offload-arch=gfx950 (no hipify, no CUDA sources).
2. ``mla_custom_cuda*.so`` -- the PyTorch extension with the reference's operator surface,
   a g++-compiled binding that calls the C ABI.

Usage:  python mla-cuda_amd/build.py [--lib-only]
"""

from __future__ import annotations

import glob
import os
import shutil
import subprocess
import sys
import sysconfig

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
LIB = os.path.join(PKG, "libmla_amd.so")

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-fvisibility=hidden",
    # packed fp32 VALU ops (v_pk_*_f32) are disabled in all device code: some of their
    # forms have given silently wrong results on this platform
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


def hipcc() -> str:
    for c in ("/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if c and os.path.exists(c):
            return c
    raise RuntimeError("hipcc not found")


def build_lib(verbose: bool = False) -> str:
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    tmp = LIB + ".tmp"
    cmd = [hipcc(), *HIPCC_FLAGS, "-I", os.path.join(ROOT, "include"), *srcs, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature: harmless
    noise = "'-packed-fp32-ops' is not a recognized feature"
    err = "\n".join(l for l in r.stderr.splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed ({r.returncode}):\n{err}")
    if err.strip() and verbose:
        print(err)
    os.replace(tmp, LIB)
    return LIB


def build_binding(verbose: bool = False) -> str:
    env = dict(os.environ)
    env.setdefault("MAX_JOBS", "8")
    cmd = [sys.executable, os.path.join(PKG, "binding", "setup.py"), "build_ext", "--inplace"]
    r = subprocess.run(cmd, cwd=PKG, capture_output=True, text=True, env=env)
    if r.returncode != 0:
        raise RuntimeError(f"binding build failed:\n{r.stdout[-4000:]}\n{r.stderr[-4000:]}")
    suffix = sysconfig.get_config_var("EXT_SUFFIX")
    out = os.path.join(PKG, "mla_custom_cuda" + suffix)
    if not os.path.exists(out):
        raise RuntimeError(f"binding build produced no {out}")
    shutil.rmtree(os.path.join(PKG, "build"), ignore_errors=True)
    return out


def main(argv=None):
    argv = sys.argv[1:] if argv is None else argv
    print("built", build_lib(verbose="-v" in argv), flush=True)
    if "--lib-only" not in argv:
        print("built", build_binding(verbose="-v" in argv), flush=True)


if __name__ == "__main__":
    main()
