"""The device layout built at load time (lane-split interleaved words), checked on the CPU.

A numpy emulation of the kernels' chain decode (chain L of a tile: lane L % 32 from bit 0, or from its `mid` offset
for L >= 32; window = words rows r, r + 1 of the lane) must reproduce the reference decode of the golden blobs.
"""
import numpy as np
import pytest

from conftest import golden_cases, load_golden


def build_layout(lib, blob, N, KS, pre_il=0, compact=0):
    b = np.frombuffer(blob, np.uint8) if isinstance(blob, bytes) else np.ascontiguousarray(blob, np.uint8)
    T = (N // 64) * (KS // 256)
    tbase = np.zeros(T, np.uint32)
    mid = np.zeros(T * 32, np.uint16)
    rows = np.zeros(T, np.uint16)
    n = lib.lw_build_layout(b.ctypes.data, len(b), N, KS, pre_il, compact, tbase.ctypes.data, mid.ctypes.data,
                            rows.ctypes.data, None, 0)
    if n < 0:
        return None
    words = np.zeros(n, np.uint32)
    lib.lw_build_layout(b.ctypes.data, len(b), N, KS, pre_il, compact, None, None, None, words.ctypes.data, n)
    return tbase, mid.reshape(T, 32), rows, words


def emulate_decode(lut, tbase, mid, rows, words, N, KS):
    """Chain decode as the kernels do it: 64 chains per tile, window from rows r and r + 1 of the lane."""
    KT = KS // 256
    out = np.zeros((N, KS), np.uint8)
    w = words.astype(np.uint64)
    lut = lut.astype(np.uint64)
    for t in range(len(tbase)):
        tr, tc = divmod(t, KT)
        lanes = np.arange(64) % 32
        pos = np.where(np.arange(64) >= 32, mid[t][lanes], 0).astype(np.uint64)
        base = int(tbase[t]) + lanes
        assert int(rows[t]) * 32 + int(tbase[t]) <= len(words)
        for c in range(256):
            r = (pos >> np.uint64(5)).astype(np.int64)
            assert np.all(r + 1 <= int(rows[t]))    # the staged rows [0, rows] cover every window
            lo = w[base + 32 * r]
            hi = w[base + 32 * (r + 1)]
            e = lut[(((hi << np.uint64(32)) | lo) >> (pos & np.uint64(31))) & np.uint64(2047)]
            out[tr * 64 + np.arange(64), tc * 256 + c] = (e & np.uint64(255)).astype(np.uint8)
            pos += e >> np.uint64(8)
    return out


@pytest.mark.parametrize("case", golden_cases())
def test_layout_chain_decode(lib, case):
    g = load_golden(case)
    N, KS = g["sym"].shape
    lay = build_layout(lib, g["blob"], N, KS)
    assert lay is not None
    tbase, mid, rows, words = lay
    assert np.all(tbase % 32 == 0)
    got = emulate_decode(g["lut"], tbase, mid, rows, words, N, KS)
    assert np.array_equal(got, g["decoded"])


@pytest.mark.parametrize("case", ["huf4p_q4k_128x1024", "huf8_q6k_64x512"])
def test_layout_mid_is_first_row_length(lib, case):
    g = load_golden(case)
    N, KS = g["sym"].shape
    tbase, mid, rows, words = build_layout(lib, g["blob"], N, KS)
    L = g["lengths"].astype(np.int64)
    KT = KS // 256
    for t in range(len(tbase)):
        tr, tc = divmod(t, KT)
        for l in range(32):
            first = g["sym"][tr * 64 + l, tc * 256:(tc + 1) * 256]
            assert mid[t, l] == L[first].sum()
            second = g["sym"][tr * 64 + 32 + l, tc * 256:(tc + 1) * 256]
            assert rows[t] >= (L[first].sum() + L[second].sum() + 31) // 32


def test_layout_rejects_corrupt_blob(lib):
    g = load_golden("huf4p_q4k_128x1024")
    N, KS = g["sym"].shape
    b = bytearray(g["blob"].tobytes())
    st = np.frombuffer(b, np.uint32, 4, 4096).copy()
    st[1] += 3                                   # lane 1 no longer starts where lane 0 ends
    b[4096:4112] = st.tobytes()
    assert build_layout(lib, bytes(b), N, KS) is None
    assert build_layout(lib, g["blob"].tobytes()[:5000], N, KS) is None     # truncated


def interleave_reference_layout(blob, N, KS, compact):
    """The reference's pre-interleaved export layout (kernels/llmrt.cu:1206-1257 semantics), written here only to
    produce _il / _ilc test inputs: [lut][tbase T][wc T (padded even) u16][ovf T x 32 u16][words][96 zero]."""
    T = (N // 64) * (KS // 256)
    b = np.frombuffer(blob, np.uint8)
    starts = np.frombuffer(blob, np.uint32, T * 32, 4096).astype(np.int64)
    pay = np.frombuffer(blob, np.uint32, offset=4096 + T * 128).astype(np.uint64)
    pw = len(pay)
    ends = np.append(starts[1:], min(starts[-1] + 512 * 11, (pw - 2) * 32))
    wc = np.zeros(T + (T & 1), np.uint16)
    ovf = np.zeros((T, 32), np.uint16)
    tb = np.zeros(T, np.uint32)
    body = []
    off = 0

    def word(bitpos, left):
        wi = bitpos >> 5
        x = (int(pay[wi]) | (int(pay[wi + 1]) << 32 if wi + 1 < pw else 0)) >> (bitpos & 31)
        v = x & 0xFFFFFFFF
        return v & ((1 << left) - 1) if left < 32 else v

    for t in range(T):
        nb = ends[t * 32:(t + 1) * 32] - starts[t * 32:(t + 1) * 32]
        w = (nb + 31) // 32
        W = int(w.min()) if compact else int(w.max())
        ov = 0
        for l in range(32):
            ovf[t, l] = ov
            ov += max(0, int(w[l]) - W)
        tb[t] = off
        blk = np.zeros(W * 32 + ov, np.uint32)
        for l in range(32):
            for i in range(int(w[l])):
                v = word(int(starts[t * 32 + l]) + 32 * i, int(nb[l]) - 32 * i)
                blk[i * 32 + l if i < W else W * 32 + int(ovf[t, l]) + (i - W)] = v
        wc[t] = W
        body.append(blk)
        off += len(blk)
    words = np.concatenate(body + [np.zeros(96, np.uint32)])
    return b[:4096].tobytes() + tb.tobytes() + wc.tobytes() + ovf.tobytes() + words.tobytes()


@pytest.mark.parametrize("compact", [0, 1])
def test_layout_from_reference_export(lib, compact):
    g = load_golden("huf4p_q4k_128x1024")
    N, KS = g["sym"].shape
    il = interleave_reference_layout(g["blob"].tobytes(), N, KS, compact)
    lay = build_layout(lib, il, N, KS, pre_il=1, compact=compact)
    assert lay is not None
    got = emulate_decode(g["lut"], *lay, N, KS)
    assert np.array_equal(got, g["decoded"])
    raw = build_layout(lib, g["blob"], N, KS)
    for a, b in zip(lay, raw):      # same device layout either way
        assert np.array_equal(a, b)
