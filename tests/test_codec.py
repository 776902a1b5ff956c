"""Encoder and Huffman tables against fixtures written by the reference's own codec (tests/golden/make_golden.py)."""
import ctypes

import numpy as np
import pytest

from conftest import GOLDEN, golden_cases, load_golden


@pytest.mark.parametrize("case", golden_cases())
def test_encoder_byte_exact(lib, case):
    from lazyweights_amd import bundle
    g = load_golden(case)
    blob, bits = bundle.encode_huf8(g["sym"])
    assert bits == int(g["total_bits"])
    assert blob == g["blob"].tobytes()


@pytest.mark.parametrize("case", golden_cases())
def test_lut_and_lengths(lib, case):
    g = load_golden(case)
    hist = np.bincount(g["sym"].ravel(), minlength=256).astype(np.int64)
    L = np.zeros(256, np.uint8)
    assert lib.lw_huffman_lengths(hist.ctypes.data, 256, 11, L.ctypes.data) == 0
    if (L > 0).sum() == 1:
        L = np.where(hist > 0, 1, 0).astype(np.uint8)
    assert np.array_equal(L, g["lengths"])
    lut = np.frombuffer(g["blob"].tobytes()[:4096], np.uint16)
    assert np.array_equal(lut, g["lut"])


def test_heap_lengths_with_ties(lib):
    z = np.load(GOLDEN + "/huffman_lengths.npz")
    for h, want, want_lim in zip(z["hist"], z["code_lengths"], z["limited"]):
        h = np.ascontiguousarray(h, np.int64)
        L = np.zeros(256, np.uint8)
        lib.lw_huffman_lengths(h.ctypes.data, 256, 0, L.ctypes.data)
        assert np.array_equal(L.astype(np.int64), want)
        lib.lw_huffman_lengths(h.ctypes.data, 256, 11, L.ctypes.data)
        assert np.array_equal(L.astype(np.int64), want_lim)


def test_kraft_and_limit_on_synthetic(lib):
    """Length-limited codes are complete prefix codes: Kraft sum 1, every length <= 11."""
    from lazyweights_amd import bundle
    for kqt, H in ((1, 2.3), (2, 3.4), (3, 4.3), (4, 2.6)):
        codes, _ = bundle.synth_matrix(kqt, 128, 1024, H, 5)
        sym = bundle.form_symbols(kqt, codes)
        hist = np.bincount(sym.ravel(), minlength=256).astype(np.int64)
        L = np.zeros(256, np.uint8)
        lib.lw_huffman_lengths(hist.ctypes.data, 256, 11, L.ctypes.data)
        used = L[hist > 0].astype(np.float64)
        assert used.max() <= 11 and abs(np.sum(2.0 ** -used) - 1.0) < 1e-12


def test_synthetic_entropy_and_determinism(lib):
    from lazyweights_amd import bundle
    a, sa = bundle.synth_matrix(1, 256, 4096, 2.3, 42, threads=1)
    b, sb = bundle.synth_matrix(1, 256, 4096, 2.3, 42, threads=7)
    assert np.array_equal(a, b) and np.array_equal(sa, sb)
    p = np.bincount(a.ravel(), minlength=16) / a.size
    H = -np.sum(p[p > 0] * np.log2(p[p > 0]))
    assert abs(H - 2.3) < 0.02
    assert a.max() <= 15
    d = sa[:, 0::16].astype(np.uint16) | (sa[:, 1::16].astype(np.uint16) << 8)
    dv = d.view(np.float16).astype(np.float32)
    assert dv.min() >= 0.0049 and dv.max() <= 0.0201


def test_encode_rejects_bad_shapes(lib):
    bits = ctypes.c_uint64(0)
    sym = np.zeros((63, 256), np.uint8)
    assert lib.lw_encode(sym.ctypes.data, 63, 256, None, 0, ctypes.byref(bits)) == -1
    sym = np.zeros((64, 200), np.uint8)
    assert lib.lw_encode(sym.ctypes.data, 64, 200, None, 0, ctypes.byref(bits)) == -1
