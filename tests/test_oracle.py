"""Pins the oracle (oracle/lw_oracle.c) before it is trusted as the checker.

- decoders: against decodes written by the reference's lazyweights/bundle.py (golden fixtures) and against the
  reference's own C++ decoder (hw/huff/tb/csim_main.cpp) compiled under oracle/_ref;
- comparator tables: against the LUT over all 2048 windows (brute force);
- sub-scale extraction: against the reference's field *packing* (scripts/kq_quant.py:204-221), restated here as
  the inverse function, and against hand-computed known answers;
- GEMV: against numpy's fp64 matmul;
- int8 activations: the quantizer against hand-built blocks (exact scale, ties to even, zero blocks, the error
  bound), and the int8 GEMV against the identity it must satisfy: the sum of s d acc - o sx over sub-blocks equals
  the fp64 product of the dequantized weights with the dequantized activations d q.
"""
import os
import subprocess

import numpy as np
import pytest

from conftest import ROOT, golden_cases, load_golden


@pytest.mark.parametrize("case", golden_cases())
def test_lockstep_decode_matches_reference(orc, case):
    g = load_golden(case)
    N, KS = g["sym"].shape
    assert np.array_equal(orc.decode_lockstep(g["blob"], N, KS), g["decoded"])


@pytest.mark.parametrize("case", golden_cases())
def test_cpu_decode_matches_reference(orc, case):
    g = load_golden(case)
    N, KS = g["sym"].shape
    for th in (1, 3):
        assert np.array_equal(orc.cpu_decode(g["blob"], N, KS, th), g["decoded"])


@pytest.mark.parametrize("case", golden_cases())
def test_comparator_equals_lut(orc, case):
    lut = load_golden(case)["lut"]
    tabs = orc.canon_tables(lut)
    for w in range(2048):
        if lut[w] >> 8:       # entries a code reaches (the single-symbol table leaves odd windows empty)
            assert orc.canon_lookup(tabs, w) == int(lut[w]), w


def pack_q4k(d, dmin, sc, m):
    """scripts/kq_quant.py:204-215 field packing of one Q4_K/Q5_K super-block (the inverse of extraction)."""
    s = np.zeros(12, np.uint8)
    for j in range(4):
        s[j] = sc[j] | ((sc[4 + j] >> 4) << 6)
        s[4 + j] = m[j] | ((m[4 + j] >> 4) << 6)
        s[8 + j] = (sc[4 + j] & 15) | ((m[4 + j] & 15) << 4)
    return np.concatenate([np.array([d], np.float16).view(np.uint8), np.array([dmin], np.float16).view(np.uint8), s])


def pack_iq4xs(d, ls):
    """scripts/kq_quant.py:218-221 (ls = stored 6-bit values)."""
    hi = 0
    for j in range(8):
        hi |= (ls[j] >> 4) << (2 * j)
    lo = [ls[j] & 15 for j in range(8)]
    b = [lo[2 * j] | (lo[2 * j + 1] << 4) for j in range(4)]
    return np.concatenate([np.array([d], np.float16).view(np.uint8), np.array([hi], np.uint16).view(np.uint8),
                           np.array(b, np.uint8)])


def test_sub_scales_invert_reference_packing(orc):
    rng = np.random.default_rng(3)
    for kqt in (1, 2):
        for _ in range(50):
            d, dmin = np.float16(rng.uniform(0.005, 0.02)), np.float16(rng.uniform(0.005, 0.02))
            sc, m = rng.integers(0, 64, 8), rng.integers(0, 64, 8)
            s, o = orc.sub_scales(kqt, pack_q4k(d, dmin, sc, m)[None])
            assert np.array_equal(s[0], np.float32(d) * sc.astype(np.float32))
            assert np.array_equal(o[0], np.float32(dmin) * m.astype(np.float32))
    for _ in range(50):
        d, ls = np.float16(rng.uniform(0.005, 0.02)), rng.integers(0, 64, 8)
        s, o = orc.sub_scales(4, pack_iq4xs(d, ls)[None])
        assert np.array_equal(s[0], np.float32(d) * (ls - 32).astype(np.float32)) and not o.any()
    for _ in range(20):
        d, sc = np.float16(rng.uniform(0.005, 0.02)), rng.integers(-128, 128, 16)
        rec = np.concatenate([sc.astype(np.int8).view(np.uint8), np.array([d], np.float16).view(np.uint8)])
        s, o = orc.sub_scales(3, rec[None])
        assert np.array_equal(s[0], np.float32(d) * sc.astype(np.float32)) and not o.any()


def test_sub_scales_known_answers(orc):
    # Q4_K: d = 1, dmin = 0.5; scale bytes chosen by hand. Sub-block 5: sc = (b[9] & 15) | (b[1] >> 6) << 4
    rec = np.zeros(16, np.uint8)
    rec[0:2] = np.array([1.0], np.float16).view(np.uint8)
    rec[2:4] = np.array([0.5], np.float16).view(np.uint8)
    rec[4 + 1] = 0b11000011   # q[1]: sc[1] = 3, high bits of sc[5] = 3
    rec[4 + 5] = 0b01000111   # q[5]: m[1] = 7, high bits of m[5] = 1
    rec[4 + 9] = 0x2A         # q[9]: sc[5] low nibble 10, m[5] low nibble 2
    s, o = orc.sub_scales(1, rec[None])
    assert s[0, 1] == 3 and o[0, 1] == 3.5            # d*3, 0.5*7
    assert s[0, 5] == 10 + 48 and o[0, 5] == 0.5 * (2 + 16)
    # IQ4_XS: ls_j = ((b[4 + j/2] >> 4 (j & 1)) & 15) | ((hi >> 2j) & 3) << 4; s = d (ls - 32)
    rec = np.zeros(8, np.uint8)
    rec[0:2] = np.array([2.0], np.float16).view(np.uint8)
    rec[2:4] = np.array([0b11 << 6], np.uint16).view(np.uint8)   # hi bits of ls_3 = 3
    rec[4 + 1] = 0x70          # ls_3 low nibble = 7 (high nibble of byte 1), ls_2 low = 0
    s, _ = orc.sub_scales(4, rec[None])
    assert s[0, 3] == 2.0 * ((7 | 48) - 32) and s[0, 2] == 2.0 * (0 - 32)


def test_dequant_known_grid(orc):
    # IQ4_XS grid (llama.cpp kvalues_iq4nl) and Q6_K centring on a 1 x 256 matrix with unit scales
    side = np.zeros((1, 8), np.uint8)
    side[0, 0:2] = np.array([1.0], np.float16).view(np.uint8)
    side[0, 2:4] = np.array([0xAAAA], np.uint16).view(np.uint8)   # ls high bits 2 -> ls = 32 + low
    side[0, 4:8] = 0x11                                           # ls low nibbles 1 -> ls = 33 -> s = 1
    codes = np.tile(np.arange(16, dtype=np.uint8), 16)[None]
    w = orc.dequant(4, codes, side)
    assert list(w[0, :16]) == [-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113]
    side6 = np.zeros((1, 18), np.uint8)
    side6[0, :16] = 1
    side6[0, 16:18] = np.array([0.5], np.float16).view(np.uint8)
    codes6 = np.arange(256, dtype=np.uint8)[None] % 64
    w6 = orc.dequant(3, codes6, side6)
    assert np.array_equal(w6[0], 0.5 * (codes6[0].astype(np.float32) - 32))


def test_dequant_known_answers_q4k_q5k(orc):
    """Q4_K / Q5_K dequant of one super-block with eight distinct sub-block scales and mins, the 12 scale bytes
    written out by hand (not by a packer) from get_scale_min_k4's field layout:
    sc = [1, 2, 3, 4, 17, 34, 51, 63], m = [5, 6, 7, 8, 20, 40, 60, 9], d = 0.5, dmin = 0.25, so w = 0.5 sc_j q - 0.25 m_j
    on sub-block j (weights 32 j .. 32 j + 31)."""
    q = [0x41, 0x82, 0xC3, 0xC4,   # sc0..3 in bits 0-5; bits 6-7: high bits of sc4..7 (1, 2, 3, 3)
         0x45, 0x86, 0xC7, 0x08,   # m0..3 in bits 0-5; bits 6-7: high bits of m4..7 (1, 2, 3, 0)
         0x41, 0x82, 0xC3, 0x9F]   # low nibble: sc4..7 low 4 bits (1, 2, 3, 15); high nibble: m4..7 low (4, 8, 12, 9)
    rec = np.concatenate([np.array([0.5, 0.25], np.float16).view(np.uint8), np.array(q, np.uint8)])[None]
    s, o = orc.sub_scales(1, rec)
    assert list(s[0]) == [0.5, 1.0, 1.5, 2.0, 8.5, 17.0, 25.5, 31.5]
    assert list(o[0]) == [1.25, 1.5, 1.75, 2.0, 5.0, 10.0, 15.0, 2.25]
    k = np.arange(256)
    for kqt, codes in ((1, (k + k // 32) % 16), (2, (k + 3 * (k // 32)) % 32)):
        w = orc.dequant(kqt, codes.astype(np.uint8)[None], rec)[0]
        # a few entries by hand
        if kqt == 1:
            assert w[0] == -1.25                    # sub-block 0, q 0: 0 - 0.25 * 5
            assert w[37] == 1.0 * 6 - 1.5           # sub-block 1, q (37 + 1) % 16 = 6
            assert w[165] == 17.0 * 10 - 10.0       # sub-block 5, q (165 + 5) % 16 = 10: 160
            assert w[255] == 31.5 * 6 - 2.25        # sub-block 7, q (255 + 7) % 16 = 6
        else:
            assert w[31] == 0.5 * 31 - 1.25         # q 31 at the end of sub-block 0
            assert w[200] == 25.5 * 26 - 15.0       # sub-block 6, q (200 + 18) % 32 = 26
            assert w[250] == 31.5 * 15 - 2.25       # sub-block 7, q (250 + 21) % 32 = 15
        sc = np.array([1, 2, 3, 4, 17, 34, 51, 63], np.float64).repeat(32)
        m = np.array([5, 6, 7, 8, 20, 40, 60, 9], np.float64).repeat(32)
        assert np.array_equal(w.astype(np.float64), 0.5 * sc * codes - 0.25 * m)


def test_gemv_f64_matches_numpy(orc):
    rng = np.random.default_rng(0)
    w = rng.standard_normal((64, 512)).astype(np.float32)
    x = rng.standard_normal((3, 512))
    assert np.allclose(orc.gemv_f64(w, x), x @ w.astype(np.float64).T, rtol=1e-13, atol=1e-12)


def test_decode_gemv_baseline_matches_dequant(orc):
    from lazyweights_amd import bundle
    rng = np.random.default_rng(1)
    for kqt in (1, 2, 3, 4):
        codes, side = bundle.synth_matrix(kqt, 128, 1024, 2.5, 11)
        blob, _ = bundle.encode_huf8(bundle.form_symbols(kqt, codes))
        x = rng.standard_normal(1024).astype(np.float32)
        y = orc.decode_gemv(kqt, blob, side, 128, 1024, x, threads=2)
        y64 = orc.gemv_f64(orc.dequant(kqt, codes, side), x.astype(np.float64))[0]
        assert orc.rel_err(y, y64) < 1e-5


CSIM = os.path.join(ROOT, "oracle", "_ref", "huff_csim")


@pytest.mark.skipif(not os.path.exists(CSIM), reason="reference C++ decoder not built (reference tree absent)")
def test_reference_cpp_decoder_reads_our_bundles(tmp_path):
    from lazyweights_amd.bundle import Writer
    w = Writer(str(tmp_path))
    names = []
    for case in ("huf4p_q4k_128x1024", "huf8_q6k_64x512", "limited_64x768"):
        g = load_golden(case)
        N, KS = g["sym"].shape
        from lazyweights_amd.bundle import encode_huf8
        blob, _ = encode_huf8(g["sym"])
        four = case.startswith("huf4p")
        w.add(case, "huf4p" if four else "huf8", N, 2 * KS if four else KS, 1.0, 0, blob)
        names.append((case, g["sym"]))
    w.close()
    for case, sym in names:
        dump = tmp_path / (case + ".bin")
        p = subprocess.run([CSIM, str(tmp_path), "--threads", "2", "--only", case, "--dump-ref", case, str(dump)],
                           stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True, timeout=300)
        assert p.returncode == 0, p.stderr
        assert '"mismatch": 0' in p.stdout and '"mismatch": 1' not in p.stdout
        assert np.array_equal(np.fromfile(dump, np.uint8).reshape(sym.shape), sym)


def test_quant_x8_known_blocks(orc):
    # block 0: max |x| = 127 -> d = 1 exactly; halves round to even (2.5 -> 2, 3.5 -> 4, -2.5 -> -2)
    b0 = np.zeros(32, np.float32)
    b0[:6] = [127, 2.5, 3.5, -2.5, 0.5, -1.49]
    b1 = np.zeros(32, np.float32)                        # all zero: d = 0, q = 0, sx = 0
    b2 = np.zeros(32, np.float32)
    b2[7] = -3.0                                         # one value: q = -127 there
    b3 = np.linspace(-1, 2, 32).astype(np.float32)       # max at the end: q = 127 there
    q, d, sx = orc.quant_x8(np.concatenate([b0, b1, b2, b3])[None])
    q = q.reshape(4, 32).astype(int)
    assert d[0, 0] == 1.0 and list(q[0, :6]) == [127, 2, 4, -2, 0, -1] and sx[0, 0] == 130.0
    assert d[0, 1] == 0 and not q[1].any() and sx[0, 1] == 0
    assert d[0, 2] == np.float32(3.0) / np.float32(127) and q[2, 7] == -127 and q[2].sum() == -127
    assert q[3, 31] == 127 and q[3, 0] == round(-1 / (2 / 127))


def test_quant_x8_bounds(orc):
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((4, 4096)) * rng.uniform(1e-3, 1e3, (4, 1))).astype(np.float32)
    q, d, sx = orc.quant_x8(x)
    qb = q.astype(np.int64).reshape(4, 128, 32)
    xb = x.astype(np.float64).reshape(4, 128, 32)
    assert np.abs(qb).max() <= 127 and (np.abs(qb).max(axis=2) == 127).all()
    assert (np.abs(xb - d[..., None] * qb) <= d[..., None] * (0.5 + 1e-5)).all()
    assert np.allclose(sx, d * qb.sum(axis=2), rtol=1e-7, atol=0)


@pytest.mark.parametrize("kqt", [1, 2, 3, 4])
def test_act8_gemv_identity(orc, kqt, monkeypatch):
    """gemv_act8_f64 (sub-block integer sums, scales applied per sub-block) == fp64 product of dequant(W) with the
    dequantized activations: pins the per-sub-block scale, the 32-block index, the offset term and the grid."""
    from lazyweights_amd import bundle
    codes, side = bundle.synth_matrix(kqt, 64, 1024, 3.0, 5)
    x = np.random.default_rng(kqt).standard_normal((3, 1024)).astype(np.float32)
    q, d, sx = orc.quant_x8(x)
    y8 = orc.gemv_act8_f64(kqt, codes, side, q, d, sx)
    xh = (q.astype(np.float64).reshape(3, 32, 32) * d[..., None]).reshape(3, 1024)
    W = orc.dequant(kqt, codes, side)
    assert orc.rel_err(y8, orc.gemv_f64(W, xh)) < 1e-7
    # the int8 result stays near the fp32-x product (quantization error only)
    assert orc.rel_err(y8, orc.gemv_f64(W, x.astype(np.float64))) < 2e-2
    # planted mistakes the identity catches: the offset term dropped, the grid off by one, the wrong 32-block
    ref = orc.gemv_f64(W, xh)
    if kqt in (1, 2):
        assert orc.rel_err(y8 - orc.gemv_act8_f64(kqt, codes, side, 0 * q, d, sx), ref) > 1e-3
    assert orc.rel_err(orc.gemv_act8_f64(kqt, codes, side, q, np.roll(d, 1, axis=1), sx), ref) > 1e-3
    if kqt in (3, 4):
        monkeypatch.setattr(orc, "grid_i8", lambda k, c: np.asarray(c).astype(np.int32))
        assert orc.rel_err(orc.gemv_act8_f64(kqt, codes, side, q, d, sx), ref) > 1e-3
