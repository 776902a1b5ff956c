"""Bundle directories and coded blobs, with the reference's Python names (lazyweights/bundle.py).

A bundle directory (lazyweights/bundle.py:10-21, 114-150) is `weights.bin`, every tensor starting at a 256-byte
boundary, plus `manifest.txt`: `cfg <key> <value>` lines and one `t <name> <enc> <N> <K> <scale> <zp> <offset>
<nbytes>` line per tensor. Writer drives the library's C++ bundle writer (lw_bundle_*); read_manifest parses the
manifest by the field table below. encode_huf8 produces the same blob bytes as lazyweights/bundle.py:57-85 (checked
byte for byte against fixtures written by the reference encoder), computed by the C++ codec of this library.
"""
import ctypes
import os

import numpy as np

from ._lib import last_error, load_library

TN, TK, LMAX, LANES = 64, 256, 11, 32
ALIGN = 256
KQ = {"Q4_K": 1, "Q5_K": 2, "Q6_K": 3, "IQ4_XS": 4}
KQ_NAME = {v: k for k, v in KQ.items()}
SIDE_BYTES = {1: 16, 2: 16, 3: 18, 4: 8}       # per 256-weight super-block
SYMBITS = {1: 4, 2: 8, 3: 8, 4: 4}             # 4: two codes per symbol (huf4p), 8: one (huf8)


def encode_huf8(sym):
    """uint8 symbols [N, KS] -> (blob bytes, payload bits)."""
    sym = np.ascontiguousarray(sym, np.uint8)
    N, KS = sym.shape
    lib = load_library()
    bits = ctypes.c_uint64(0)
    n = lib.lw_encode(sym.ctypes.data, N, KS, None, 0, ctypes.byref(bits))
    if n < 0:
        raise ValueError("encode_huf8: shape %s is not a whole number of 64 x 256 tiles" % (sym.shape,))
    out = np.zeros(n, np.uint8)
    lib.lw_encode(sym.ctypes.data, N, KS, out.ctypes.data, n, ctypes.byref(bits))
    return out.tobytes(), int(bits.value)


def synth_matrix(kqt, N, K, entropy, seed, threads=8):
    """Seeded synthetic K-quant matrix: (codes [N, K] uint8, side bytes [N, K / 256 * SB] uint8)."""
    codes = np.zeros((N, K), np.uint8)
    side = np.zeros((N, K // 256 * SIDE_BYTES[kqt]), np.uint8)
    if load_library().lw_synth_matrix(kqt, N, K, float(entropy), int(seed), codes.ctypes.data, side.ctypes.data,
                                      threads) != 0:
        raise ValueError("synth_matrix: bad arguments")
    return codes, side


def form_symbols(kqt, codes):
    """codes [N, K] -> symbols [N, KS] (scripts/a2_kq_bundle.py:108: pair = q[2c] | q[2c + 1] << 4)."""
    codes = np.ascontiguousarray(codes, np.uint8)
    if SYMBITS[kqt] == 8:
        return codes.copy()
    return (codes[:, 0::2] | (codes[:, 1::2] << 4)).astype(np.uint8)


class Writer:
    """Writer(path).cfg(key, value) / .add(name, enc, N, K, scale, zp, blob) / .add_kquant(...) / .close()."""

    def __init__(self, path):
        self.lib = load_library()
        self.path = str(path)
        self.h = self.lib.lw_bundle_create(self.path.encode())
        if not self.h:
            raise OSError("cannot write a bundle at %s" % self.path)

    def _check(self, rc, what):
        if rc != 0:
            raise ValueError("bundle %s: %s refused (a name, key or value with white space, or a write error)"
                             % (self.path, what))

    def cfg(self, k, v):
        self._check(self.lib.lw_bundle_cfg(self.h, str(k).encode(), str(v).encode()), "cfg " + str(k))

    def add(self, name, enc, N, K, scale, zp, blob):
        data = np.frombuffer(bytes(blob), np.uint8)
        self._check(self.lib.lw_bundle_add(self.h, name.encode(), enc.encode(), int(N), int(K), float(scale), int(zp),
                                           data.ctypes.data if data.size else None, data.size), "tensor " + name)

    def add_kquant(self, name, kqt, codes, side, packed=False):
        """A K-quant matrix as the reference bundler writes it (scripts/a2_kq_bundle.py:216-218): Huffman-coded
        (huf4p / huf8), or with packed=True the fixed-rate twin (pk4 / pk8: the symbol bytes as they are)."""
        N, K = codes.shape
        sym = form_symbols(kqt, codes)
        if packed:
            self.add(name, "pk4" if SYMBITS[kqt] == 4 else "pk8", N, K, 1.0, 0, np.ascontiguousarray(sym).tobytes())
        else:
            blob, _ = encode_huf8(sym)
            self.add(name, "huf4p" if SYMBITS[kqt] == 4 else "huf8", N, K, 1.0, 0, blob)
        self.add(name + ".kqs", "kq_" + KQ_NAME[kqt], N, side.shape[1], 1.0, 0, np.ascontiguousarray(side).tobytes())

    def close(self):
        if self.h:
            h, self.h = self.h, None
            self._check(self.lib.lw_bundle_finish(h), "finish")


# fields of a manifest `t` line after the tag, in order, with their types
T_FIELDS = (("name", str), ("enc", str), ("N", int), ("K", int), ("scale", float), ("zp", int), ("offset", int),
            ("nbytes", int))


def read_manifest(path):
    """(cfg dict of strings, list of tensor dicts with the T_FIELDS keys, in manifest order)."""
    cfg, tensors = {}, []
    with open(os.path.join(path, "manifest.txt")) as f:
        text = f.read()
    for fields in (ln.split() for ln in text.splitlines()):
        tag, rest = (fields[0], fields[1:]) if fields else ("", [])
        if tag == "t" and len(rest) == len(T_FIELDS):
            tensors.append({key: conv(v) for (key, conv), v in zip(T_FIELDS, rest)})
        elif tag == "cfg" and len(rest) >= 2:
            cfg[rest[0]] = rest[1]
    return cfg, tensors


def read_tensor(path, t):
    with open(os.path.join(path, "weights.bin"), "rb") as f:
        f.seek(t["offset"])
        return np.frombuffer(f.read(t["nbytes"]), np.uint8)


def write_packed_bundle(path, mats, threads=16):
    """The packed twin of write_synthetic_bundle's matrices (the same seeded codes and side bytes), enc pk4 / pk8."""
    w = Writer(str(path))
    for name, kqt, N, K, H, seed in mats:
        codes, side = synth_matrix(kqt, N, K, H, seed, threads)
        w.add_kquant(name, kqt, codes, side, packed=True)
    w.close()
    return path


def write_synthetic_bundle(path, mats, threads=16):
    """Fast all-C++ writer: mats = [(name, kqt, N, K, entropy, seed), ...]."""
    n = len(mats)
    names = (ctypes.c_char_p * n)(*[m[0].encode() for m in mats])
    kq = (ctypes.c_int * n)(*[m[1] for m in mats])
    Ns = (ctypes.c_int * n)(*[m[2] for m in mats])
    Ks = (ctypes.c_int * n)(*[m[3] for m in mats])
    Hs = (ctypes.c_double * n)(*[float(m[4]) for m in mats])
    seeds = (ctypes.c_uint64 * n)(*[int(m[5]) for m in mats])
    rc = load_library().lw_write_bundle(str(path).encode(), n, names, kq, Ns, Ks, Hs, seeds, threads)
    if rc != 0:
        raise RuntimeError("lw_write_bundle failed: " + last_error())
    return path
