"""Builds lazyweights_amd/liblazyweights_amd.so in-tree (HIP kernels for gfx950 + host C++ runtime).

    python -m lazyweights_amd.build               # the library
    python -m lazyweights_amd.build --timeline    # the diagnostic timestamp build (lazyweights_amd.timeline)

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
TIMELINE_LIB = os.path.join(PKG, "liblazyweights_amd_timeline.so")  # diagnostic build (build_timeline)
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


OBJDUMP = os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "llvm", "bin", "llvm-objdump")


def _vregs(op):
    """VGPR numbers named by one operand (v5, v[4:7]); empty for anything else."""
    import re
    m = re.match(r"v\[(\d+):(\d+)\]$", op)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"v(\d+)$", op)
    return {int(m.group(1))} if m else set()


# wait states after a matrix-core write of a VGPR before a DPP read of it (at least the longest MFMA form's
# MFMA-to-VALU read wait: 16 passes and a few more)
MFMA_WAITS = 19


def dpp_violations(disasm):
    """DPP operations in an llvm-objdump disassembly of gfx950 code without their wait states: 2 after a VALU write
    of the DPP source (src0), 5 after a write of EXEC (an SALU write naming exec, or any v_cmpx, which writes EXEC
    implicitly), and MFMA_WAITS after a matrix-core (v_mfma) write of the DPP source (a bound above the MFMA-to-VALU
    read wait of the longest form, 16 passes). The walk goes back over the operation's basic block (branch targets
    and function starts end it); at a block start the predecessor is unknown, so 5 wait states (s_nop) must lie
    inside the block (an MFMA write before the block start is not seen: none of this build's DPP sources comes from
    the matrix cores). Returns "function at 0xaddr" strings."""
    import re
    fn, base = "?", 0
    ins, targets = [], set()
    for line in disasm.splitlines():
        m = re.match(r"([0-9a-f]+) <(.+)>:$", line)
        if m:
            fn, base = m.group(2), int(m.group(1), 16)
            ins.append(None)  # function boundary
            continue
        m = re.match(r"\s+(\S+)\s*(.*?)\s*//\s*([0-9A-F]+):", line)
        if not m:
            continue
        t = re.search(r"<(.+)\+0x([0-9a-f]+)>", line)
        if t:
            targets.add(base + int(t.group(2), 16))
        ops = [o.strip() for o in m.group(2).split(",")] if m.group(2) else []
        ins.append((int(m.group(3), 16), m.group(1), ops, fn))
    bad = []
    for i, it in enumerate(ins):
        if it is None or "_dpp" not in it[1]:
            continue
        src = _vregs(it[2][1]) if len(it[2]) > 1 else set()
        waits, j, ok = 0, i - 1, False
        while True:
            if j < 0 or ins[j] is None or ins[j + 1][0] in targets:  # the block starts at j + 1
                ok = waits >= 5
                break
            mn, ops = ins[j][1], ins[j][2]
            if mn.startswith("s_nop"):
                waits += (int(ops[0], 0) if ops else 0) + 1
            else:
                writes_src = bool(ops) and mn.startswith("v_") and bool(_vregs(ops[0]) & src)
                if ((writes_src and mn.startswith("v_mfma") and waits < MFMA_WAITS) or
                        (writes_src and waits < 2) or
                        (((ops and ops[0].startswith("exec")) or mn.startswith("v_cmpx")) and waits < 5)):
                    break
                waits += 1
            if waits >= MFMA_WAITS:
                ok = True
                break
            j -= 1
        if not ok:
            bad.append("%s at 0x%x" % (it[3], it[0]))
    return bad


def check_dpp_hazards(lib):
    """The DPP operations of the built code objects (the v_dot2c_f32_f16_dpp broadcasts, written as inline assembly,
    which the compiler's hazard recognizer does not see) must have their wait states (dpp_violations). The check
    disassembles this build's own gfx950 code objects; raises RuntimeError naming each violation."""
    import tempfile
    if not os.path.exists(OBJDUMP):
        raise RuntimeError("build: %s not found (needed to check DPP wait states)" % OBJDUMP)
    tmp = tempfile.mkdtemp(prefix="lw_dpp_")
    try:
        shutil.copy(lib, os.path.join(tmp, "l.so"))
        subprocess.run([OBJDUMP, "--offloading", "l.so"], cwd=tmp, stdout=subprocess.DEVNULL,
                       stderr=subprocess.DEVNULL, check=True)
        objs = [f for f in os.listdir(tmp) if "amdgcn" in f and ARCH in f]
        if not objs:
            raise RuntimeError("build: no %s code object found in %s" % (ARCH, lib))
        bad = []
        for obj in objs:
            out = subprocess.run([OBJDUMP, "-d", "--mcpu=" + ARCH, os.path.join(tmp, obj)], stdout=subprocess.PIPE,
                                 stderr=subprocess.DEVNULL, text=True, check=True).stdout
            bad += dpp_violations(out)
        if bad:
            raise RuntimeError("build: DPP operations without their wait states: " + ", ".join(bad[:8]))
        return len(objs)
    finally:
        shutil.rmtree(tmp, ignore_errors=True)


def build(verbose=False):
    os.makedirs(BUILD, exist_ok=True)
    with ThreadPoolExecutor(max_workers=len(SOURCES)) as ex:
        objs = list(ex.map(lambda s: _compile(*s), SOURCES))
    tmp = LIB + ".tmp"
    _run([HIPCC, "-shared", "-fPIC", "--offload-arch=" + ARCH, "-o", tmp] + objs +
         ["-L" + ROCM_LIB, "-lrocblas", "-pthread", "-lm"])
    check_dpp_hazards(tmp)
    os.replace(tmp, LIB)
    if verbose:
        print("built", LIB)
    return LIB


def build_timeline(verbose=False):
    """The diagnostic library (lazyweights_amd.timeline): the same sources, the device code compiled with
    -DLW_TIMELINE (per-wave timestamps in the whole-tile kernel), beside the product library. Builds the product's
    host objects first if they are missing."""
    os.makedirs(BUILD, exist_ok=True)
    objs = [os.path.join(BUILD, os.path.splitext(src)[0] + ".o") for src, kind in SOURCES if kind != "hip"]
    if not all(os.path.exists(o) for o in objs):
        build()
    obj = os.path.join(BUILD, "lw_kernels_timeline.o")
    _run([HIPCC, "-c", "-x", "hip", os.path.join(CSRC, "lw_kernels.hip"), "-o", obj] + COMMON + HIP_DEVICE +
         ["-DLW_TIMELINE"])
    tmp = TIMELINE_LIB + ".tmp"
    _run([HIPCC, "-shared", "-fPIC", "--offload-arch=" + ARCH, "-o", tmp, obj] + objs +
         ["-L" + ROCM_LIB, "-lrocblas", "-pthread", "-lm"])
    check_dpp_hazards(tmp)
    os.replace(tmp, TIMELINE_LIB)
    if verbose:
        print("built", TIMELINE_LIB)
    return TIMELINE_LIB


if __name__ == "__main__":
    if "--timeline" in sys.argv[1:]:
        build_timeline(verbose=True)
    else:
        build(verbose=True)
    sys.exit(0)
