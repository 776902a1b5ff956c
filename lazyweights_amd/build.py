"""Builds lazyweights_amd/liblazyweights_amd.so in-tree (HIP kernels for gfx950 + host C++ runtime).

    python -m lazyweights_amd.build

Device code: hipcc --offload-arch=gfx950, with packed-fp32 instruction selection disabled. Pure host C++ (codec,
layout, bundle writer) is compiled with g++; everything is linked into one shared library exposing the C-ABI of
include/lazyweights_amd.h (with rocBLAS for the prefill GEMMs).
"""
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
BUILD = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "liblazyweights_amd.so")
ARCH = os.environ.get("LW_OFFLOAD_ARCH", "gfx950")

HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
ROCM_LIB = os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "lib")
CXX = shutil.which("g++") or "g++"
COMMON = ["-O3", "-std=c++17", "-fPIC", "-Wall", "-I", CSRC, "-I", os.path.join(ROOT, "include")]
HIP_DEVICE = ["--offload-arch=" + ARCH, "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
              "-Wno-unused-command-line-argument"]

SOURCES = [
    ("lw_kernels.hip", "hip"),
    ("lw_runtime.cpp", "hiphost"),
    ("lw_codec.cpp", "cxx"),
    ("lw_layout.cpp", "cxx"),
    ("lw_bundle.cpp", "cxx"),
]


def _run(cmd):
    p = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(line for line in p.stdout.splitlines() if "packed-fp32-ops" not in line)
    if p.returncode != 0:
        raise RuntimeError("build failed: %s\n%s" % (" ".join(cmd), out))
    return out


def _compile(src, kind):
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    path = os.path.join(CSRC, src)
    if kind == "hip":
        cmd = [HIPCC, "-c", "-x", "hip", path, "-o", obj] + COMMON + HIP_DEVICE
    elif kind == "hiphost":
        cmd = [HIPCC, "-c", "-x", "hip", path, "-o", obj] + COMMON + HIP_DEVICE
    else:
        cmd = [CXX, "-c", path, "-o", obj, "-pthread"] + COMMON
    _run(cmd)
    return obj


def build(verbose=False):
    os.makedirs(BUILD, exist_ok=True)
    with ThreadPoolExecutor(max_workers=len(SOURCES)) as ex:
        objs = list(ex.map(lambda s: _compile(*s), SOURCES))
    tmp = LIB + ".tmp"
    _run([HIPCC, "-shared", "-fPIC", "--offload-arch=" + ARCH, "-o", tmp] + objs +
         ["-L" + ROCM_LIB, "-lrocblas", "-pthread", "-lm"])
    os.replace(tmp, LIB)
    if verbose:
        print("built", LIB)
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
