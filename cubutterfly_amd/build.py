"""Build libcubutterfly.so in-tree with hipcc for gfx950.

Usage: python -m cubutterfly_amd.build [-j N]
Objects go to cubutterfly_amd/_build/; the shared library is written next to
this file so it travels with the source tree. Every call recompiles.
"""
import argparse
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
SRC = HERE / "csrc"
OUT = HERE / "libcubutterfly.so"
BUILD = HERE / "_build"
ARCH = "gfx950"
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")

COMMON = [
    "-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function",
    "-fvisibility=hidden",
    f"-I{HERE.parent / 'include'}",
]
# Device code: gfx950 only; packed FP32 instructions are disabled (the host
# pass warns that it does not know the feature, which is harmless).
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-x", "hip", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc():
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found; ROCm is required to build libcubutterfly")
    return path


def sources():
    return sorted(SRC.glob("*.hip")) + sorted(SRC.glob("*.cpp"))


def compile_one(src):
    obj = BUILD / (src.name + ".o")
    host_only = ["-x", "c++", "-D__HIP_PLATFORM_AMD__", f"-I{ROCM}/include"]
    cmd = [hipcc()] + COMMON + (HIP_FLAGS if src.suffix == ".hip" else host_only) + ["-c", str(src), "-o", str(obj)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"compile failed: {src.name}\n{' '.join(cmd)}\n{result.stdout}{result.stderr}")
    return obj


def build(jobs=None, verbose=False):
    BUILD.mkdir(exist_ok=True)
    srcs = sources()
    jobs = jobs or min(8, os.cpu_count() or 1)
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(compile_one, srcs))
    tmp = OUT.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp)] + [str(o) for o in objs]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"link failed\n{' '.join(cmd)}\n{result.stdout}{result.stderr}")
    os.replace(tmp, OUT)
    if verbose:
        print(f"built {OUT}")
    return OUT


if __name__ == "__main__":
    parser = argparse.ArgumentParser()
    parser.add_argument("-j", type=int, default=None)
    args = parser.parse_args()
    try:
        build(args.j, verbose=True)
    except RuntimeError as error:
        print(error, file=sys.stderr)
        sys.exit(1)
