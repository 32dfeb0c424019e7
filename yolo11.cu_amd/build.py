"""Builds libyolo11_amd.so (gfx950) in-tree with hipcc.

    python yolo11.cu_amd/build.py          # or __graft_entry__.build()

Objects go to yolo11.cu_amd/_build/, the library to yolo11.cu_amd/libyolo11_amd.so.
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libyolo11_amd.so")
# host-only JPEG header / entropy decoding, without the HIP runtime (server front-ends)
JPEG_LIB = os.path.join(HERE, "libyolo11_jpeg.so")
JPEG_SOURCES = ("jpeg.cpp", "jpeg_abi.cpp")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

# packed-fp32 instructions are disabled for all device code (some of their forms have
# produced wrong results on this hardware pool); frame.hip and nms.hip also disable FMA
# contraction so their fp32 arithmetic rounds exactly as written.
DEV_FLAGS = [f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
HOST_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-D__HIP_PLATFORM_AMD__", "-I", "/opt/rocm/include"]
# host-only translation units go through clang++ directly (hipcc would compile them as
# HIP for a default device target); clang also provides _Float16 on x86-64
HOSTCXX = os.environ.get("HOSTCXX", "/opt/rocm/llvm/bin/clang++")
SOURCES = {
    "conv.hip": DEV_FLAGS,
    "elementwise.hip": DEV_FLAGS,
    "attention.hip": DEV_FLAGS,
    "frame.hip": DEV_FLAGS + ["-ffp-contract=off"],
    "nms.hip": DEV_FLAGS + ["-ffp-contract=off"],
    "noalloc.hip": DEV_FLAGS,
    "jpeg.hip": DEV_FLAGS,
    "jpeg.cpp": ["-O3"] + HOST_FLAGS[1:],
    "jpeg_abi.cpp": HOST_FLAGS,
    "graph.cpp": HOST_FLAGS,
    "engine.cpp": HOST_FLAGS,
    "batcher.cpp": HOST_FLAGS,
}


def _compile(src: str, flags: list[str]) -> str:
    obj = os.path.join(OUT, src + ".o")
    cc = HIPCC if src.endswith(".hip") else HOSTCXX
    cmd = [cc, *flags, "-I", CSRC, "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "not a recognized feature for this target"
    msgs = "\n".join(l for l in (r.stdout + r.stderr).splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{msgs}")
    return obj


def build(verbose: bool = True) -> str:
    os.makedirs(OUT, exist_ok=True)
    with ThreadPoolExecutor(max_workers=min(8, len(SOURCES))) as ex:
        objs = list(ex.map(lambda kv: _compile(*kv), SOURCES.items()))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}{r.stderr}")
    os.replace(tmp, LIB)
    jobjs = [os.path.join(OUT, src + ".o") for src in JPEG_SOURCES]
    tmp = JPEG_LIB + ".tmp"
    r = subprocess.run([HOSTCXX, "-shared", "-fPIC", "-pthread", "-o", tmp, *jobjs], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link of {JPEG_LIB} failed:\n{r.stdout}{r.stderr}")
    os.replace(tmp, JPEG_LIB)
    if verbose:
        print(f"built {LIB}, {JPEG_LIB}")
    return LIB


if __name__ == "__main__":
    build()
    sys.exit(0)
