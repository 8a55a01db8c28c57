"""Builds libcircatt.so (gfx950) in-tree from csrc/ with hipcc.

Usage: python circulantattention.jl_amd/build.py   (or call build()).
The library lands next to this file; it is git-ignored but travels with the
tree to GPU machines.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libcircatt.so")
INCLUDE = os.path.join(os.path.dirname(HERE), "include")

HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
SOURCES = ["api.cpp", "unfused.hip", "apply_rb.hip", "fused.hip", "fused_fwd.hip", "fused_sim.hip",
           "fused_bwdq.hip", "fused_bwdkv.hip", "fused2d_fwd.hip", "fused2d_bwdq.hip",
           "fused2d_bwdkv.hip", "fused2h_fwd.hip", "fused2h_bwdq.hip", "fused2h_bwdkv.hip",
           "fused2h2_fwd.hip", "fused2h2_bwdq.hip", "fused2h2_bwdkv.hip", "fused1h_fwd.hip",
           "fused1h_bwdq.hip", "fused1h_bwdkv.hip", "fused1h2_fwd.hip", "fused1h2_bwdq.hip",
           "fused1h2_bwdkv.hip", "fused_wide.hip",
           "batch_ops.hip"]
FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Wall",
    # packed FP32 VALU ops are kept out of every code object
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA accumulators in VGPRs: the softmax rescale and the B-operand reuse
    # of the accumulator then need no AGPR copies
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    # the kernels' LDS atomics are issued by one lane per wave already; the
    # atomic optimizer would wrap each in a lane-iteration loop
    "-mllvm", "-amdgpu-atomic-optimizer-strategy=None",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


def _compile(src: str) -> str:
    out = os.path.join(OBJ, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC, *FLAGS, "-c", os.path.join(CSRC, src), "-o", out]
    if src.endswith(".cpp"):
        cmd[1:1] = ["-x", "hip"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{res.stdout}\n{res.stderr}")
    return out


def build(verbose: bool = False) -> str:
    """Compile every source (always) and link libcircatt.so; returns its path."""
    os.makedirs(OBJ, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=len(SOURCES)) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


def asan_runtime() -> str:
    """Path of the compiler's shared AddressSanitizer runtime (with the
    UndefinedBehaviorSanitizer handlers), which a process preloads to load a
    library from build_host_sanitized()."""
    clang = os.path.join(os.path.dirname(os.path.realpath(HIPCC)), "..", "llvm", "bin", "clang++")
    if not os.path.exists(clang):
        clang = shutil.which("amdclang++") or "/opt/rocm/llvm/bin/clang++"
    res = subprocess.run([clang, "-print-file-name=libclang_rt.asan-x86_64.so"],
                         capture_output=True, text=True, check=True)
    return res.stdout.strip()


def build_host_sanitized(out_dir: str) -> str:
    """A copy of libcircatt in out_dir whose host code (api.cpp: the C ABI's
    argument checks, workspace arithmetic and dispatch) is instrumented by
    AddressSanitizer and UndefinedBehaviorSanitizer, without recovery; the
    device code and the kernels' objects are those of build(), which must have
    run.  The copy resolves the sanitizer runtime at load time, so the loading
    process preloads asan_runtime().  Returns the library's path."""
    objs = [os.path.join(OBJ, os.path.splitext(s)[0] + ".o") for s in SOURCES if s != "api.cpp"]
    missing = [o for o in objs if not os.path.exists(o)]
    if missing:
        raise FileNotFoundError(f"in-tree objects not built: {missing[:3]}")
    os.makedirs(out_dir, exist_ok=True)
    api = os.path.join(out_dir, "api_sanitized.o")
    san = ["-g", "-Xarch_host", "-fsanitize=address,undefined",
           "-Xarch_host", "-fno-sanitize-recover=all", "-Xarch_host", "-fno-omit-frame-pointer"]
    cmd = [HIPCC, "-x", "hip", *FLAGS, *san, "-c", os.path.join(CSRC, "api.cpp"), "-o", api]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for the sanitized api.cpp:\n{res.stderr}")
    lib = os.path.join(out_dir, "libcircatt_host_sanitized.so")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", lib, api, *objs]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    return lib


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
