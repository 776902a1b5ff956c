"""Writes the golden fixtures in this directory from the reference's own Python codec.

Run once, in the build container only (the reference tree is not present on GPU machines):
    python tests/golden/make_golden.py [/root/reference]

It imports lazyweights/bundle.py, lazyweights/lanecodecs.py and lazyweights/huffman.py (numpy only) from the
reference tree and records, for seeded symbol matrices, the reference encoder's blob bytes (encode_huf8,
bundle.py:57-85), its decode (decode_huf8, bundle.py:88-106), the code lengths (limited_lengths,
lanecodecs.py:28-38) and, for a set of histograms with many count ties, the raw heap lengths (code_lengths,
huffman.py:8-26). These pin the byte-exact encoder and both decoders; nothing else in the tree imports the
reference. Fixtures are data only (.npz without pickles).
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def geometric_codes(rng, shape, ncodes, centre, rho):
    p = rho ** np.abs(np.arange(ncodes) - centre)
    p /= p.sum()
    return rng.choice(ncodes, size=shape, p=p).astype(np.uint8)


def pairs(q):
    return (q[:, 0::2] | (q[:, 1::2] << 4)).astype(np.uint8)


def cases():
    rng = np.random.default_rng(20261201)
    out = {}
    out["huf4p_q4k_128x1024"] = pairs(geometric_codes(rng, (128, 1024), 16, 8, 0.55))
    out["huf8_q6k_64x512"] = geometric_codes(rng, (64, 512), 64, 32, 0.8)
    out["huf8_q5k_128x256"] = geometric_codes(rng, (128, 256), 32, 16, 0.7)
    out["degenerate_64x256"] = np.full((64, 256), 0x37, np.uint8)
    # very skewed: unlimited Huffman lengths exceed 11, so the count-halving loop runs
    p = 0.5 ** np.arange(1, 41)
    p /= p.sum()
    out["limited_64x768"] = rng.choice(40, size=(64, 768), p=p).astype(np.uint8) * 5
    out["uniform_192x256"] = rng.integers(0, 256, size=(192, 256)).astype(np.uint8)
    two = rng.integers(0, 2, size=(64, 512)).astype(np.uint8)
    out["two_symbols_64x512"] = np.where(two > 0, 0xA5, 0x0F).astype(np.uint8)
    return out


def tie_histograms():
    rng = np.random.default_rng(7)
    hs = [np.ones(256, np.int64), np.arange(256, dtype=np.int64) % 5 + 1]
    h = np.zeros(256, np.int64)
    h[rng.choice(256, 60, replace=False)] = rng.integers(1, 4, 60)
    hs.append(h)
    h = np.zeros(256, np.int64)
    h[:12] = [1, 1, 2, 2, 4, 4, 8, 8, 16, 16, 32, 32]
    hs.append(h)
    return np.stack(hs)


def main():
    ref = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    sys.path.insert(0, ref)
    from lazyweights.bundle import build_lut, decode_huf8, encode_huf8  # noqa: E402
    from lazyweights.huffman import code_lengths  # noqa: E402
    from lazyweights.lanecodecs import limited_lengths  # noqa: E402

    for name, sym in cases().items():
        N, KS = sym.shape
        blob, total, hist = encode_huf8(sym)
        dec = decode_huf8(blob, N, KS)
        L = limited_lengths(hist, 11)
        if (L > 0).sum() == 1:
            L = np.where(hist > 0, 1, 0).astype(np.uint8)
        lut = build_lut(L)
        np.savez_compressed(os.path.join(HERE, name + ".npz"), sym=sym, blob=np.frombuffer(blob, np.uint8),
                            total_bits=np.int64(total), lengths=np.asarray(L, np.uint8), lut=lut, decoded=dec)
        print(name, N, KS, "blob", len(blob), "bits", total, "maxlen", int(np.max(L)),
              "roundtrip", bool(np.array_equal(dec, sym)))
    H = tie_histograms()
    lens = np.stack([code_lengths(h) for h in H]).astype(np.int64)
    lim = np.stack([limited_lengths(h, 11) for h in H]).astype(np.int64)
    np.savez_compressed(os.path.join(HERE, "huffman_lengths.npz"), hist=H, code_lengths=lens, limited=lim)
    print("huffman_lengths", H.shape)


if __name__ == "__main__":
    main()
