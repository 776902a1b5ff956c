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


# ── int8 activations (the reference's act8 path) ────────────────────────────────────────────────────────────
# IQ4_XS grid (llama.cpp kvalues_iq4nl, the table the reference dequantizes with: kernels/llmrt.cu:1057-1065)
IQ4_GRID = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113], np.int32)


def quant_x8(x):
    """x [m, K] (fp32; K a multiple of 32) -> (q int8 [m, K], d fp32 [m, K / 32], sx fp32 [m, K / 32]).

    Follows k_quant_x8 (kernels/llmrt.cu:1035-1055): per block of 32, d = max|x| / 127 in fp32, q = x / d (fp32
    quotient) rounded to nearest even (__float2int_rn), 0 where d = 0, and sx = d * (sum of q) in fp32.
    """
    x = np.ascontiguousarray(np.atleast_2d(x), np.float32)
    m, K = x.shape
    if K % 32:
        raise ValueError("K must be a multiple of 32")
    b = x.reshape(m, K // 32, 32)
    d = (np.abs(b).max(axis=2) / np.float32(127)).astype(np.float32)
    safe = np.where(d > 0, d, np.float32(1))
    q = np.where(d[..., None] > 0, np.rint(b / safe[..., None]), np.float32(0)).astype(np.int32)
    sx = (d * q.sum(axis=2).astype(np.float32)).astype(np.float32)
    return q.reshape(m, K).astype(np.int8), d, sx


def grid_i8(kqt, codes):
    """The integer each code contributes to the int8 dot products (kernels/llmrt.cu:1134-1146): Q4_K / Q5_K q,
    Q6_K q - 32, IQ4_XS the grid value kv[q]."""
    c = np.asarray(codes).astype(np.int32)
    if kqt == 4:
        return IQ4_GRID[c & 15]
    if kqt == 3:
        return c - 32
    return c


def gemv_act8_f64(kqt, codes, side, q, d, sx):
    """y [m, N] that the int8-activation kernels approximate, in fp64 (kernels/llmrt.cu:1127-1160): per sub-block g
    of GW weights (32; 16 for Q6_K), y += s_ng d_b acc_ng - o_ng sx_b, with acc_ng = sum over g of grid_i8 x q
    (an exact integer), b = g's 32-block and (s, o) the sub-block scale and offset of sub_scales."""
    codes = np.ascontiguousarray(codes, np.uint8)
    N, K = codes.shape
    q = np.atleast_2d(q).astype(np.float64)
    d = np.atleast_2d(d).astype(np.float64)
    sx = np.atleast_2d(sx).astype(np.float64)
    m = q.shape[0]
    G = 16 if kqt == 3 else 8
    GW = 256 // G
    s, o = sub_scales(kqt, np.ascontiguousarray(side, np.uint8).reshape(N * (K // 256), -1))
    s = s.astype(np.float64).reshape(N, K // GW)
    o = o.astype(np.float64).reshape(N, K // GW)
    v = grid_i8(kqt, codes).astype(np.float64).reshape(N, K // GW, GW)
    acc = np.einsum("ngk,mgk->mng", v, q.reshape(m, K // GW, GW))  # integers below 2^53: exact
    blk = (np.arange(K // GW) * GW) // 32
    y = np.einsum("ng,mg,mng->mn", s, d[:, blk], acc)
    return y - np.einsum("ng,mg->mn", o, sx[:, blk])
