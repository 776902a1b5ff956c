"""ORACLE — test infrastructure only (tests/, __graft_entry__.smoke(), bench.py's cpu_baseline leg).

ctypes front end of oracle/liblworacle.so (the plain-C restatement in lw_oracle.c, which cites the reference
file:line of every function) plus small numpy helpers. Nothing in lazyweights_amd/ imports this module.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "liblworacle.so")
_lib = None


def build():
    subprocess.run(["make", "-s", "-C", HERE, "liblworacle.so"], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            build()
        L = ctypes.CDLL(LIB)
        vp, i, ll = ctypes.c_void_p, ctypes.c_int, ctypes.c_longlong
        L.orc_decode_lockstep.argtypes = [vp, i, i, vp]
        L.orc_cpu_decode.argtypes = [vp, i, i, i, vp]
        L.orc_canon_build.argtypes = [vp, vp, vp, vp, vp]
        L.orc_canon_build.restype = None
        L.orc_canon_lookup.argtypes = [vp, vp, vp, vp, ctypes.c_uint32]
        L.orc_sub_scales.argtypes = [i, vp, ll, vp, vp]
        L.orc_dequant.argtypes = [i, vp, vp, i, i, vp]
        L.orc_unpack_symbols.argtypes = [i, vp, i, i, vp]
        L.orc_unpack_symbols.restype = None
        L.orc_gemv_f64.argtypes = [vp, vp, i, i, i, vp]
        L.orc_gemv_f64.restype = None
        L.orc_decode_gemv.argtypes = [i, vp, vp, i, i, vp, i, vp, vp]
        _lib = L
    return _lib


def _buf(b):
    a = np.frombuffer(b, np.uint8) if isinstance(b, (bytes, bytearray)) else np.ascontiguousarray(b, np.uint8)
    # 16 bytes of slack: the 64-bit window of the last symbol may read past the last payload word
    return np.concatenate([a, np.zeros(16, np.uint8)])


def decode_lockstep(blob, N, KS):
    b = _buf(blob)
    out = np.zeros((N, KS), np.uint8)
    if lib().orc_decode_lockstep(b.ctypes.data, N, KS, out.ctypes.data) != 0:
        raise ValueError("bad shape")
    return out


def cpu_decode(blob, N, KS, threads=1):
    b = _buf(blob)
    out = np.zeros((N, KS), np.uint8)
    if lib().orc_cpu_decode(b.ctypes.data, N, KS, threads, out.ctypes.data) != 0:
        raise ValueError("bad shape")
    return out


def canon_tables(lut):
    lut = np.ascontiguousarray(lut, np.uint16)
    limit = np.zeros(12, np.uint16)
    first = np.zeros(12, np.uint16)
    base = np.zeros(12, np.uint16)
    srt = np.zeros(256, np.uint8)
    lib().orc_canon_build(lut.ctypes.data, limit.ctypes.data, first.ctypes.data, base.ctypes.data, srt.ctypes.data)
    return limit, first, base, srt


def canon_lookup(tables, win):
    limit, first, base, srt = tables
    return lib().orc_canon_lookup(limit.ctypes.data, first.ctypes.data, base.ctypes.data, srt.ctypes.data, win)


def sub_scales(kqt, side_records):
    side_records = np.ascontiguousarray(side_records, np.uint8)
    n = side_records.shape[0]
    g = 16 if kqt == 3 else 8
    s = np.zeros((n, g), np.float32)
    o = np.zeros((n, g), np.float32)
    if lib().orc_sub_scales(kqt, side_records.ctypes.data, n, s.ctypes.data, o.ctypes.data) != 0:
        raise ValueError("bad kqt")
    return s, o


def dequant(kqt, codes, side):
    codes = np.ascontiguousarray(codes, np.uint8)
    side = np.ascontiguousarray(side, np.uint8)
    N, K = codes.shape
    w = np.zeros((N, K), np.float32)
    if lib().orc_dequant(kqt, codes.ctypes.data, side.ctypes.data, N, K, w.ctypes.data) != 0:
        raise ValueError("bad arguments")
    return w


def unpack_symbols(symbits, sym):
    sym = np.ascontiguousarray(sym, np.uint8)
    N, KS = sym.shape
    codes = np.zeros((N, KS * (2 if symbits == 4 else 1)), np.uint8)
    lib().orc_unpack_symbols(symbits, sym.ctypes.data, N, KS, codes.ctypes.data)
    return codes


def gemv_f64(w, x):
    """Y[m, N] = X[m, K] W[N, K]^T in fp64 (W fp32 dequantized weights)."""
    w = np.ascontiguousarray(w, np.float32)
    x = np.ascontiguousarray(np.atleast_2d(x), np.float64)
    N, K = w.shape
    y = np.zeros((x.shape[0], N), np.float64)
    lib().orc_gemv_f64(w.ctypes.data, x.ctypes.data, x.shape[0], N, K, y.ctypes.data)
    return y


def decode_gemv(kqt, blob, side, N, K, x, threads=1):
    """CPU baseline: decode the raw blob, dequantize and multiply (fp32 accumulation). Returns y [N]."""
    b = _buf(blob)
    side = np.ascontiguousarray(side, np.uint8)
    x = np.ascontiguousarray(x, np.float32)
    ks = K // 2 if kqt in (1, 4) else K
    scratch = np.zeros((N, ks), np.uint8)
    y = np.zeros(N, np.float32)
    if lib().orc_decode_gemv(kqt, b.ctypes.data, side.ctypes.data, N, K, x.ctypes.data, threads,
                             scratch.ctypes.data, y.ctypes.data) != 0:
        raise ValueError("bad arguments")
    return y


def rel_err(y, y64):
    """max |y - y64| / max |y64| (the reference's check metric, kernels/llmrt.cu:2874-2879)."""
    y = np.asarray(y, np.float64)
    y64 = np.asarray(y64, np.float64)
    return float(np.max(np.abs(y - y64)) / max(np.max(np.abs(y64)), 1e-300))
