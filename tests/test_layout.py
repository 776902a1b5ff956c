"""The device layout built at load time (lane-split interleaved words, 2 guard bits per lane stream, ring staging
schedules), checked on the CPU.

Numpy emulations of the kernels (whole-tile: chain L of a tile = lane L % 32 from bit GUARD, or from its `mid`
offset for L >= 32, window = word rows r, r + 1 of the lane; ring: the same chains reading 2-symbol windows from a
per-front ring of staged rows filled on the tile's schedule) must reproduce the reference decode of the golden
blobs, and every window the ring kernel reads must equal the true rows.
"""
GUARD = 2
import numpy as np
import pytest

from conftest import golden_cases, load_golden


def build_layout(lib, blob, N, KS, pre_il=0, compact=0, extra=False, splits=False):
    import ctypes
    b = np.frombuffer(blob, np.uint8) if isinstance(blob, bytes) else np.ascontiguousarray(blob, np.uint8)
    T = (N // 64) * (KS // 256)
    tbase = np.zeros(T, np.uint32)
    mid = np.zeros(T * 32, np.uint16)
    split = np.zeros(T * 16 * 32, np.uint16)
    rows = np.zeros(T, np.uint16)
    sched = np.zeros(2 * T, np.uint64)
    rr = ctypes.c_int(0)
    n = lib.lw_build_layout(b.ctypes.data, len(b), N, KS, pre_il, compact, tbase.ctypes.data, mid.ctypes.data,
                            split.ctypes.data, rows.ctypes.data, sched.ctypes.data, ctypes.byref(rr), None, 0)
    if n < 0:
        return None
    words = np.zeros(n, np.uint32)
    lib.lw_build_layout(b.ctypes.data, len(b), N, KS, pre_il, compact, None, None, None, None, None, None,
                        words.ctypes.data, n)
    if splits:
        return tbase, split.reshape(T, 16, 32), rows, words
    if extra:
        return tbase, mid.reshape(T, 32), rows, words, sched, rr.value
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
        pos = np.where(np.arange(64) >= 32, mid[t][lanes], GUARD).astype(np.uint64)
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
            assert mid[t, l] == GUARD + L[first].sum()
            second = g["sym"][tr * 64 + 32 + l, tc * 256:(tc + 1) * 256]
            assert rows[t] >= (GUARD + L[first].sum() + L[second].sum() + 31) // 32


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


def emulate_ring(lut, tbase, mid, words, sched, RS, N, KS, syms):
    """The ring kernel's staging and register window (k_fused_ring), per tile and front: rows r, r + 1 of the
    window in registers A, B, row r + 2 re-read from the ring (C) after every pair, one 32-bit window per pair."""
    KT = KS // 256
    lut = lut.astype(np.uint64)
    out = np.zeros((N, KS), np.uint8)
    l = np.arange(32)
    M32 = np.uint64(0xFFFFFFFF)
    RS0 = RS
    for t in range(len(tbase)):
        tr, tc = divmod(t, KT)
        counts, meta = int(sched[2 * t]), int(sched[2 * t + 1])
        RS = RS0
        if (meta >> 32) & 3 == 3:   # exception tile with a 32-row schedule
            RS = 32
        elif (meta >> 32) & 1:      # exception tile without a ring schedule: the whole-tile kernel's
            out[tr * 64:(tr + 1) * 64, tc * 256:(tc + 1) * 256] = syms[tr * 64:(tr + 1) * 64, tc * 256:(tc + 1) * 256]
            continue
        base1, init = meta & 255, [(meta >> 8) & 255, (meta >> 16) & 255]
        for f in range(2):
            base = base1 if f else 0
            W = lambda r: words[int(tbase[t]) + 32 * (base + r) + l].astype(np.uint64)   # noqa: E731
            ring = np.zeros((RS, 32), np.uint64)

            def put(k):
                for i in range(2):
                    ring[(2 * k + i) & (RS - 1)] = W(2 * k + i)
            for k in range(init[f]):
                put(k)
            issued = init[f]
            pend = [[], []]
            P = ((mid[t].astype(np.int64) - GUARD) if f else np.zeros(32, np.int64)) - 32 * base + 64
            assert np.all(P >= 64)
            slot = (P >> 5) & (RS - 1)
            A, B, C = ring[(slot - 2) & (RS - 1), l], ring[(slot - 1) & (RS - 1), l], ring[slot, l]
            for k, v in ((2, A), (1, B), (0, C)):
                assert np.array_equal(v, W((P >> 5) - k)), (t, f, "initial window")
            col = 0
            for g in range(16):
                h = g & 1
                for k in pend[h]:
                    put(k)
                pend[h] = []
                for _ in range((counts >> (32 * f + 2 * g)) & 3):
                    pend[h].append(issued)
                    issued += 1
                for p in range(8):
                    w1 = (((B << np.uint64(32)) | A) >> (P & 31).astype(np.uint64)) & M32
                    e1 = lut[(w1 >> np.uint64(GUARD)) & np.uint64(2047)]
                    w2 = w1 >> (e1 >> np.uint64(8))                  # second symbol from the same 32 bits
                    e2 = lut[(w2 >> np.uint64(GUARD)) & np.uint64(2047)]
                    rows_out = tr * 64 + 32 * f + l
                    out[rows_out, tc * 256 + col] = (e1 & np.uint64(255)).astype(np.uint8)
                    out[rows_out, tc * 256 + col + 1] = (e2 & np.uint64(255)).astype(np.uint8)
                    col += 2
                    P = P + (e1 >> np.uint64(8)).astype(np.int64) + (e2 >> np.uint64(8)).astype(np.int64)
                    nslot = (P >> 5) & (RS - 1)
                    slide = nslot != slot
                    A, B = np.where(slide, B, A), np.where(slide, C, B)
                    slot = nslot
                    C = ring[slot, l]
                    assert np.array_equal(A, W((P >> 5) - 2)) and np.array_equal(B, W((P >> 5) - 1)), (t, f, g, p)
                    last = g == 15 and p == 7          # the final re-read is never used
                    assert last or np.array_equal(C, W(P >> 5)), (t, f, g, p)
    return out


def emulate_split(lut, tbase, split, rows, words, N, KS):
    """The low-latency kernel's decode (k_fused_split): per tile and lane 8 chains of 64 symbols from the load-time
    split offsets, each with the register window (rows r, r + 1, then r + 2 after every pair) over the staged tile
    image of rows[t] + 2 rows, asserting that every row read lies inside it."""
    KT = KS // 256
    lut = lut.astype(np.uint64)
    out = np.zeros((N, KS), np.uint8)
    l = np.arange(32)
    M32 = np.uint64(0xFFFFFFFF)
    for t in range(len(tbase)):
        tr, tc = divmod(t, KT)
        R = int(rows[t]) + 2
        img = words[int(tbase[t]):int(tbase[t]) + 32 * R].astype(np.uint64).reshape(R, 32)

        def row(r):
            assert np.all(r >= 0) and np.all(r < R), (t, "row outside the staged image")
            return img[r, l]
        for f in range(2):
            for w in range(4):
                P = split[t, 2 * (4 * f + w)].astype(np.int64) - GUARD + 64
                slot = P >> 5
                A, B, C = row(slot - 2), row(slot - 1), row(slot)
                col = 64 * w
                for p in range(32):
                    w1 = (((B << np.uint64(32)) | A) >> (P & 31).astype(np.uint64)) & M32
                    e1 = lut[(w1 >> np.uint64(GUARD)) & np.uint64(2047)]
                    w2 = w1 >> (e1 >> np.uint64(8))
                    e2 = lut[(w2 >> np.uint64(GUARD)) & np.uint64(2047)]
                    rr = tr * 64 + 32 * f + l
                    out[rr, tc * 256 + col] = (e1 & np.uint64(255)).astype(np.uint8)
                    out[rr, tc * 256 + col + 1] = (e2 & np.uint64(255)).astype(np.uint8)
                    col += 2
                    P = P + (e1 >> np.uint64(8)).astype(np.int64) + (e2 >> np.uint64(8)).astype(np.int64)
                    nslot = P >> 5
                    slide = nslot != slot
                    A, B = np.where(slide, B, A), np.where(slide, C, B)
                    slot = nslot
                    C = row(slot)
    return out


def emulate_tiles(lut, tbase, split, rows, words, N, KS):
    """The whole-tile kernel's decode (k_fused_tiles): lane l of a tile decodes row l (lane stream l % 32, front
    l / 32) as 8 chains of 32 symbols from the load-time split offsets, each with the register window (rows r, r + 1,
    then row r + 2 after every pair) over the tile image of rows[t] + 2 rows, every read asserted inside it."""
    KT = KS // 256
    lut = lut.astype(np.uint64)
    out = np.zeros((N, KS), np.uint8)
    l = np.arange(32)
    M32 = np.uint64(0xFFFFFFFF)
    for t in range(len(tbase)):
        tr, tc = divmod(t, KT)
        R = int(rows[t]) + 2
        img = words[int(tbase[t]):int(tbase[t]) + 32 * R].astype(np.uint64).reshape(R, 32)

        def row(r):
            assert np.all(r >= 0) and np.all(r < R), (t, "row outside the tile image")
            return img[r, l]
        for f in range(2):
            for j in range(8):
                P = split[t, 8 * f + j].astype(np.int64) - GUARD + 64
                slot = P >> 5
                A, B, C = row(slot - 2), row(slot - 1), row(slot)
                col = 32 * j
                for p in range(16):
                    w1 = (((B << np.uint64(32)) | A) >> (P & 31).astype(np.uint64)) & M32
                    e1 = lut[(w1 >> np.uint64(GUARD)) & np.uint64(2047)]
                    w2 = w1 >> (e1 >> np.uint64(8))
                    e2 = lut[(w2 >> np.uint64(GUARD)) & np.uint64(2047)]
                    rr = tr * 64 + 32 * f + l
                    out[rr, tc * 256 + col] = (e1 & np.uint64(255)).astype(np.uint8)
                    out[rr, tc * 256 + col + 1] = (e2 & np.uint64(255)).astype(np.uint8)
                    col += 2
                    P = P + (e1 >> np.uint64(8)).astype(np.int64) + (e2 >> np.uint64(8)).astype(np.int64)
                    nslot = P >> 5
                    slide = nslot != slot
                    A, B = np.where(slide, B, A), np.where(slide, C, B)
                    slot = nslot
                    C = row(slot)
    return out


@pytest.mark.parametrize("case", golden_cases())
def test_split_chain_emulation(lib, case):
    """The chain starts per lane reproduce the golden decode (k = 0 is the guard, k = 8 is mid)."""
    g = load_golden(case)
    N, KS = g["sym"].shape
    tbase, split, rows, words = build_layout(lib, g["blob"], N, KS, splits=True)
    _, mid, _, _ = build_layout(lib, g["blob"], N, KS)
    assert np.all(split[:, 0] == GUARD) and np.array_equal(split[:, 8], mid)
    assert np.array_equal(emulate_split(g["lut"], tbase, split, rows, words, N, KS), g["decoded"])
    assert np.array_equal(emulate_tiles(g["lut"], tbase, split, rows, words, N, KS), g["decoded"])


def test_split_chain_emulation_exception_tiles(lib):
    """Tiles without a 16-row ring schedule (one with a 32-row schedule, one with none) decode through the chains
    like any other tile."""
    from lazyweights_amd import bundle
    for codes, _ in (mild_skew_codes(), skewed_tile_codes()):
        sym = bundle.form_symbols(2, codes)
        blob, _ = bundle.encode_huf8(sym)
        tbase, split, rows, words = build_layout(lib, blob, 128, 8192, splits=True)
        lut = np.frombuffer(blob, np.uint16, 2048, 0)
        assert np.array_equal(emulate_split(lut, tbase, split, rows, words, 128, 8192), sym)
        assert np.array_equal(emulate_tiles(lut, tbase, split, rows, words, 128, 8192), sym)


def test_tile_stride(lib):
    """Tiles lie at a fixed stride of max(rows) word rows when that pads the words by at most 1/8, else back to back;
    either way tbase holds the offsets, the words end 16 zero rows past the last slot, and the chains decode the same
    symbols (a config-2-like matrix takes the stride; a matrix with one tile of twice the rows does not)."""
    from lazyweights_amd import bundle
    cases = [bundle.synth_matrix(1, 256, 2048, 2.3, 11)[0], skewed_tile_codes()[0]]
    for kqt, codes in zip((1, 2), cases):
        sym = bundle.form_symbols(kqt, codes)
        blob, _ = bundle.encode_huf8(sym)
        N, KS = sym.shape
        tbase, split, rows, words = build_layout(lib, blob, N, KS, splits=True)
        r = rows.astype(np.int64)
        T = len(r)
        fixed = T * r.max() * 32 <= r.sum() * 32 + (r.sum() * 32) // 8
        want = 32 * r.max() * np.arange(T) if fixed else np.concatenate([[0], np.cumsum(32 * r)[:-1]])
        assert np.array_equal(tbase.astype(np.int64), want)
        assert len(words) == (T * r.max() if fixed else r.sum()) * 32 + 16 * 32
        assert fixed == (kqt == 1)
        if fixed:  # the rows past a tile's own are zeros
            for t in range(T):
                assert not words[int(tbase[t]) + 32 * int(r[t]):int(tbase[t]) + 32 * int(r.max())].any()
        lut = np.frombuffer(blob, np.uint16, 2048, 0)
        assert np.array_equal(emulate_tiles(lut, tbase, split, rows, words, N, KS), sym)


@pytest.mark.parametrize("case", golden_cases())
def test_ring_schedule_emulation(lib, case):
    g = load_golden(case)
    N, KS = g["sym"].shape
    tbase, mid, rows, words, sched, RS = build_layout(lib, g["blob"], N, KS, extra=True)
    if RS == 0:
        pytest.skip("no ring schedule for this matrix (whole-tile kernel)")
    got = emulate_ring(g["lut"], tbase, mid, words, sched, RS, N, KS, g["sym"])
    assert np.array_equal(got, g["decoded"])


def test_ring_schedules_exist_for_benchmark_shapes(lib):
    """Every BASELINE format gets a ring schedule (16 rows) at realistic entropies."""
    from lazyweights_amd import bundle
    for kqt, H in ((1, 2.3), (1, 2.6), (2, 3.4), (3, 4.3), (4, 2.6)):
        codes, _ = bundle.synth_matrix(kqt, 256, 4096, H, 77)
        blob, _ = bundle.encode_huf8(bundle.form_symbols(kqt, codes))
        ks = 2048 if kqt in (1, 4) else 4096
        lay = build_layout(lib, blob, 256, ks, extra=True)
        assert lay[5] == 16, (kqt, H, lay[5])


def skewed_tile_codes(seed=3):
    """Q5_K codes [128, 8192] (64 tiles) where tile 5 has lanes alternating between the most frequent code and the
    two rarest ones: its fronts drift apart by dozens of word rows, so no ring schedule exists for that tile."""
    from lazyweights_amd import bundle
    codes, side = bundle.synth_matrix(2, 128, 8192, 3.4, seed)
    blk = codes[0:64, 5 * 256:6 * 256]
    for r in range(64):
        blk[r] = 16 if (r % 32) % 2 == 0 else np.where(np.arange(256) % 2 == 0, 0, 31)
    return codes, side


def mild_skew_codes(tiles=(5, 37), seed=3):
    """Q5_K codes [128, 8192] (64 tiles, KT = 32) where the given tiles have every odd lane of each front replace
    15 % of its codes with the two rarest ones: the fronts drift apart by more than a 16-row ring holds but fit a
    32-row ring. Tiles 5 and 37 are tile rows 0 and 1 of tile column 5, adjacent in the flat kernel's order."""
    from lazyweights_amd import bundle
    codes, side = bundle.synth_matrix(2, 128, 8192, 3.4, seed)
    rng = np.random.default_rng(1)
    for t in tiles:
        tr, tc = divmod(t, 32)
        blk = codes[tr * 64:(tr + 1) * 64, tc * 256:(tc + 1) * 256]
        for r in range(1, 64, 2):
            rare = rng.random(256) < 0.15
            blk[r] = np.where(rare, np.where(np.arange(256) % 2 == 0, 0, 31), blk[r])
    return codes, side


def test_ring_exception_tiles_with_32_row_schedule(lib):
    """Mildly skewed tiles fail the 16-row check but keep a 32-row schedule (sched bits 32 and 33), listed first
    among the exceptions; the ring emulation decodes them with 32-row rings, every window checked."""
    from lazyweights_amd import bundle
    codes, _ = mild_skew_codes()
    sym = bundle.form_symbols(2, codes)
    blob, _ = bundle.encode_huf8(sym)
    tbase, mid, rows, words, sched, RS = build_layout(lib, blob, 128, 8192, extra=True)
    assert RS == 16
    flags = {t: (int(sched[2 * t + 1]) >> 32) & 3 for t in range(len(tbase)) if (int(sched[2 * t + 1]) >> 32) & 1}
    assert flags == {5: 3, 37: 3}
    lut = np.frombuffer(blob, np.uint16, 2048, 0)
    assert np.array_equal(emulate_ring(lut, tbase, mid, words, sched, RS, 128, 8192, sym), sym)


def test_ring_exception_tiles(lib):
    """A tile without a 16-row schedule is flagged and listed as an exception; every other tile keeps the ring."""
    from lazyweights_amd import bundle
    codes, _ = skewed_tile_codes()
    sym = bundle.form_symbols(2, codes)
    blob, _ = bundle.encode_huf8(sym)
    tbase, mid, rows, words, sched, RS = build_layout(lib, blob, 128, 8192, extra=True)
    assert RS == 16
    flagged = [t for t in range(len(tbase)) if (int(sched[2 * t + 1]) >> 32) & 1]
    assert flagged == [5]
    assert (int(sched[2 * 5 + 1]) >> 33) & 1 == 0  # no 32-row schedule either
    lut = np.frombuffer(blob, np.uint16, 2048, 0)
    assert np.array_equal(emulate_ring(lut, tbase, mid, words, sched, RS, 128, 8192, sym), sym)


def _bitrev11(w):
    return int("{:011b}".format(w)[::-1], 2)


@pytest.mark.parametrize("case", golden_cases())
def test_canon_table_matches_oracle(lib, orc, case):
    """The comparator table of kernel mode 9 (lw_canon_table, built for every K-quant matrix at load time) on the
    reference encoder's decode tables: the oracle's limits, first / base per length and symbol order
    (orc_canon_build, itself pinned to the table over every window), and its own lookup of every window a code
    reaches gives the table's symbol and length."""
    lut = np.ascontiguousarray(load_golden(case)["lut"], np.uint16)
    out = np.zeros(288, np.uint32)
    assert lib.lw_canon_table(1, lut.ctypes.data, out.ctypes.data) == 0
    limit, first, base, srt = orc.canon_tables(lut)
    assert np.array_equal(out[:10], limit[1:11].astype(np.uint32))
    for l in range(1, 12):
        w = int(out[9 + l])
        assert w & 31 == 11 - l
        assert (w >> 16) - (1 << 16 if w >> 31 else 0) == 4 * (int(base[l]) - int(first[l])), l
    nsym = len({int(e) & 255 for e in lut if e >> 8})
    ent = out[32:32 + nsym]
    assert np.array_equal((ent >> 16 & 15) | (ent >> 24 & 15) << 4, srt[:nsym].astype(np.uint32))
    for win in range(2048):
        if not lut[win] >> 8:
            continue
        v = _bitrev11(win)
        p = int(out[10])
        for k in range(10):
            if v >= out[k]:
                p = int(out[11 + k])
        idx = (v >> (p & 31)) + ((p >> 16) - (1 << 16 if p >> 31 else 0)) // 4
        e = int(out[32 + idx])
        assert (e & 255, (e >> 16 & 15) | (e >> 24 & 15) << 4) == (int(lut[win]) >> 8, int(lut[win]) & 255), win


def test_canon_table_rejects_non_canonical(lib):
    """A prefix code whose codes of one length are not in symbol order is not the canonical code: lw_canon_table
    refuses it (kernel mode 9 then refuses the matrix instead of decoding wrong symbols)."""
    def two_of_one_length(lut):
        lens = {}
        for e in lut:
            if e >> 8:
                lens.setdefault(int(e) >> 8, set()).add(int(e) & 255)
        return next((sorted(s)[:2] for l, s in sorted(lens.items()) if len(s) >= 2), None)

    luts = [np.ascontiguousarray(load_golden(c)["lut"], np.uint16) for c in golden_cases()]
    lut = next(t for t in luts if two_of_one_length(t))
    out = np.zeros(288, np.uint32)
    assert lib.lw_canon_table(1, lut.ctypes.data, out.ctypes.data) == 0
    a, b = two_of_one_length(lut)
    bad = lut.copy()
    for i, e in enumerate(lut):
        if e >> 8 and int(e) & 255 in (a, b):
            bad[i] = (int(e) & 0xFF00) | (b if int(e) & 255 == a else a)
    assert lib.lw_canon_table(1, bad.ctypes.data, out.ctypes.data) == -1
    assert lib.lw_canon_table(0, lut.ctypes.data, out.ctypes.data) == -1
