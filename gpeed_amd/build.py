"""Build recipe for libgpeed_iq3.so (gfx950), compiled in-tree with hipcc.

Every HIP source is compiled with packed-FP32 instruction selection disabled
(``-target-feature -packed-fp32-ops``); the host pass warns that it does not
know the feature, which is harmless.
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libgpeed_iq3.so")
HOST_LIB = os.path.join(HERE, "libgpeed_glm5.so")
ROOT = os.path.dirname(HERE)
HOST_CHECK = os.path.join(ROOT, "tests", "cpp", "host_check")
SOURCES = ["capi.hip", "iq3_dequant.hip", "iq3_gemv.hip", "iq3_moe.hip", "iq3_gemm.hip", "quant_rows.hip"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # a kernel's first six scalar arguments are preloaded into SGPRs at wave
    # launch, so its first loads wait for no kernel-argument read (the code
    # object keeps a fallback that loads them on firmware without preloading)
    "-mllvm", "-amdgpu-kernarg-preload-count=6",
]


def _run(cmd):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        sys.stderr.write(out + "\n")
        raise RuntimeError(f"build failed: {' '.join(cmd)}")
    return out


# Per-source extra flags: none at present.
EXTRA: dict = {}


def build(verbose: bool = False) -> str:
    """Compile every source to an object in csrc/_build and link the shared library."""
    bdir = os.path.join(CSRC, "_build")
    os.makedirs(bdir, exist_ok=True)
    objs = []
    for src in SOURCES:
        obj = os.path.join(bdir, src.replace(".hip", ".o"))
        out = _run([HIPCC, *FLAGS, *EXTRA.get(src, []), "-c", os.path.join(CSRC, src), "-o", obj])
        if verbose and out.strip():
            print(out)
        objs.append(obj)
    tmp = LIB + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs])
    os.replace(tmp, LIB)
    build_host()
    return LIB


def build_host() -> str:
    """C++ host layer with the reference's signatures (glm5 namespace) over the
    C ABI, and the small driver the GPU tests run it through. Plain g++: the
    host layer needs no HIP header."""
    cxx = os.environ.get("CXX", "g++")
    tmp = HOST_LIB + ".tmp"
    _run([cxx, "-std=c++17", "-O2", "-Wall", "-fPIC", "-shared", os.path.join(HERE, "host", "glm5_gpu.cpp"),
          os.path.join(HERE, "host", "gguf.cpp"), "-o", tmp, "-L" + HERE, "-lgpeed_iq3", "-Wl,-rpath,$ORIGIN"])
    os.replace(tmp, HOST_LIB)
    tmp = HOST_CHECK + ".tmp"
    _run([cxx, "-std=c++17", "-O2", "-Wall", os.path.join(ROOT, "tests", "cpp", "host_check.cpp"), "-o", tmp,
          "-L" + HERE, "-lgpeed_glm5", "-lgpeed_iq3", "-Wl,-rpath,$ORIGIN/../../gpeed_amd"])
    os.replace(tmp, HOST_CHECK)
    return HOST_LIB


if __name__ == "__main__":
    print(build(verbose=True))
