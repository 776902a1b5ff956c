"""Runtime boundary on the CPU: exports, manifest validation and error returns, CPU decode entry points.

Failure handling is forced from the host (bad manifests, mismatched side tensors, truncated blobs); no GPU is
touched (budget_mb = 0 opens without residency)."""
import os
import re

import numpy as np
import pytest

from conftest import ROOT, load_golden


def declared_functions():
    src = open(os.path.join(ROOT, "include", "lazyweights_amd.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return re.findall(r"\b([a-z_][a-z0-9_]*)\s*\(", src)


def test_library_exports_every_declared_symbol(lib):
    names = [n for n in declared_functions() if n.startswith(("rt_", "lw_"))]
    assert len(names) >= 25
    for n in names:
        assert hasattr(lib, n), n


def write_bundle(path, cases=("huf4p_q4k_128x1024", "huf8_q6k_64x512"), side=True):
    from lazyweights_amd.bundle import Writer, encode_huf8
    w = Writer(str(path))
    for case in cases:
        g = load_golden(case)
        N, KS = g["sym"].shape
        four = case.startswith("huf4p")
        K = 2 * KS if four else KS
        blob, _ = encode_huf8(g["sym"])
        w.add(case, "huf4p" if four else "huf8", N, K, 1.0, 0, blob)
        if side:
            kqt, sb = (1, 16) if four else (3, 18)
            w.add(case + ".kqs", "kq_Q4_K" if four else "kq_Q6_K", N, K // 256 * sb, 1.0, 0,
                  np.zeros(N * (K // 256) * sb, np.uint8).tobytes())
    w.close()
    return path


def test_open_missing_dir(lib):
    from lazyweights_amd import Runtime
    with pytest.raises(RuntimeError, match="manifest"):
        Runtime("/nonexistent/bundle", budget_mb=0)


def test_open_bad_manifest(lib, tmp_path):
    from lazyweights_amd import Runtime
    write_bundle(tmp_path)
    with open(tmp_path / "manifest.txt", "a") as f:
        f.write("t broken huf8 64\n")
    with pytest.raises(RuntimeError, match="bad tensor line"):
        Runtime(tmp_path, budget_mb=0)


def test_open_mismatched_side_tensor(lib, tmp_path):
    from lazyweights_amd import Runtime
    write_bundle(tmp_path)
    txt = open(tmp_path / "manifest.txt").read().replace("kq_Q6_K 64 36", "kq_Q6_K 64 32")
    open(tmp_path / "manifest.txt", "w").write(txt)
    with pytest.raises(RuntimeError, match="side tensor"):
        Runtime(tmp_path, budget_mb=0)


def test_open_wrong_symbol_layout(lib, tmp_path):
    from lazyweights_amd import Runtime
    write_bundle(tmp_path)
    txt = open(tmp_path / "manifest.txt").read().replace("kq_Q6_K", "kq_IQ4_XS")
    open(tmp_path / "manifest.txt", "w").write(txt)
    with pytest.raises(RuntimeError):
        Runtime(tmp_path, budget_mb=0)


def test_open_truncated_weights(lib, tmp_path):
    from lazyweights_amd import Runtime
    write_bundle(tmp_path)
    size = os.path.getsize(tmp_path / "weights.bin")
    with open(tmp_path / "weights.bin", "r+b") as f:
        f.truncate(size - 100)
    with pytest.raises(RuntimeError, match="past the end"):
        Runtime(tmp_path, budget_mb=0)


def test_open_bad_tile_shape(lib, tmp_path):
    from lazyweights_amd import Runtime
    write_bundle(tmp_path, side=False)
    txt = open(tmp_path / "manifest.txt").read().replace("huf8 64 512", "huf8 64 500")
    open(tmp_path / "manifest.txt", "w").write(txt)
    with pytest.raises(RuntimeError, match="tiles"):
        Runtime(tmp_path, budget_mb=0)


def test_cpu_decode_entry_points(lib, tmp_path, orc):
    from lazyweights_amd import Runtime
    write_bundle(tmp_path)
    with Runtime(tmp_path, budget_mb=0) as rt:
        for case in ("huf4p_q4k_128x1024", "huf8_q6k_64x512"):
            g = load_golden(case)
            for th in (1, 4):
                assert np.array_equal(rt.test_cpu_decode(case, th), g["decoded"])
        s, n = rt.cpu_decode_all(2)
        assert n == 128 * 512 + 64 * 512 and s >= 0
        # not resident: GPU entry points refuse with -1 instead of exiting
        X = np.zeros((1, 1024), np.float32)
        with pytest.raises(RuntimeError, match="not resident"):
            rt.test_matmul("huf4p_q4k_128x1024", X)
        with pytest.raises(RuntimeError, match="not resident"):
            rt.test_decode("huf4p_q4k_128x1024")
        Y = np.zeros((1, 128), np.float32)
        assert rt.lib.rt_test_matmul(rt.h, b"absent", X.ctypes.data, 1, Y.ctypes.data, 0) == -1
        assert "no tensor" in rt.lib.lw_last_error().decode()
        with pytest.raises(RuntimeError):
            rt.test_cpu_decode("huf4p_q4k_128x1024.kqs")
        assert rt.stat("resident_bytes") == 0 and rt.stat("no_such_key") == -1
        assert rt.lib.rt_forward(rt.h, None, 0, None, 0) == -1


def test_synthetic_bundle_writer(lib, tmp_path, orc):
    """The all-C++ bundle writer produces blobs that the reference-faithful oracle decodes to the seeded codes."""
    from lazyweights_amd import bundle
    mats = [("a", 1, 128, 1024, 2.3, 7), ("b", 3, 64, 512, 4.3, 8), ("c", 4, 64, 1024, 2.6, 9), ("d", 2, 64, 512, 3.4, 10)]
    bundle.write_synthetic_bundle(str(tmp_path), mats, threads=4)
    cfg, ts = bundle.read_manifest(str(tmp_path))
    by = {t["name"]: t for t in ts}
    assert all(t["offset"] % 256 == 0 for t in ts)
    for name, kqt, N, K, H, seed in mats:
        codes, side = bundle.synth_matrix(kqt, N, K, H, seed)
        t = by[name]
        assert t["enc"] == ("huf4p" if kqt in (1, 4) else "huf8") and (t["N"], t["K"]) == (N, K)
        blob = bundle.read_tensor(str(tmp_path), t)
        ks = K // 2 if kqt in (1, 4) else K
        sym = orc.decode_lockstep(blob, N, ks)
        assert np.array_equal(orc.unpack_symbols(8 if ks == K else 4, sym), codes)
        assert np.array_equal(bundle.read_tensor(str(tmp_path), by[name + ".kqs"]).reshape(side.shape), side)


def test_packed_twin_bundle(lib, tmp_path):
    """The fixed-rate twin (enc pk4 / pk8, the reference bundler's --packed output): it opens, its CPU decode
    returns the stored symbols (kernels/llmrt.cu:2547) and a packed blob shorter than N x K is rejected."""
    from lazyweights_amd import Runtime, bundle
    mats = [("p4", 1, 64, 1024, 2.3, 5), ("p8", 3, 64, 512, 4.3, 6)]
    bundle.write_packed_bundle(str(tmp_path / "ok"), mats, threads=2)
    cfg, ts = bundle.read_manifest(str(tmp_path / "ok"))
    assert {t["name"]: t["enc"] for t in ts if not t["name"].endswith(".kqs")} == {"p4": "pk4", "p8": "pk8"}
    with Runtime(tmp_path / "ok", budget_mb=0) as rt:
        for name, kqt, N, K, H, seed in mats:
            codes, _ = bundle.synth_matrix(kqt, N, K, H, seed)
            assert np.array_equal(rt.test_cpu_decode(name, 2), bundle.form_symbols(kqt, codes))
    w = bundle.Writer(str(tmp_path / "bad"))
    codes, side = bundle.synth_matrix(1, 64, 1024, 2.3, 5)
    w.add("p4", "pk4", 64, 1024, 1.0, 0, bundle.form_symbols(1, codes).tobytes()[:-1])
    w.add("p4.kqs", "kq_Q4_K", 64, side.shape[1], 1.0, 0, side.tobytes())
    w.close()
    with pytest.raises(RuntimeError, match="packed blob shorter"):
        Runtime(tmp_path / "bad", budget_mb=0)


def write_model_bundle(path, layers=2, hidden=512, inter=1024, vocab=96, seed=3):
    """A bundle laid out as the reference's model exporter writes one (scripts/a2_kq_bundle.py:189-218): cfg lines,
    a raw8 embedding with f32 row scales, f32 rope tables and norms, then per layer K-quant matrices of mixed formats
    (Q4_K / IQ4_XS as huf4p, Q6_K / Q5_K as huf8) each followed by its .kqs side tensor. Returns the matrices."""
    from lazyweights_amd import bundle
    rng = np.random.default_rng(seed)
    w = bundle.Writer(str(path))
    for k, v in dict(n_layers=layers, hidden=hidden, n_heads=8, n_kv_heads=2, head_dim=hidden // 8, inter=inter,
                     vocab=vocab, eps=1e-5, rope_rows=64, rope_half=hidden // 16, attn_scale=0.125, enc="kq_huf",
                     tied=0, eos=2).items():
        w.cfg(k, v)

    def f32(name, v):
        v = np.asarray(v, np.float32).reshape(1, -1) if np.ndim(v) == 1 else np.asarray(v, np.float32)
        w.add(name, "f32", v.shape[0], v.shape[1], 1.0, 0, v.tobytes())
    embed = rng.integers(0, 256, (vocab, hidden), dtype=np.uint8)
    w.add("embed", "raw8", vocab, hidden, 1.0, 0, embed.tobytes())
    f32("embed.rs", rng.uniform(0.01, 0.02, vocab))
    f32("embed.rsub", rng.uniform(-1, 1, vocab))
    f32("cos", rng.uniform(-1, 1, (64, hidden // 16)))
    f32("sin", rng.uniform(-1, 1, (64, hidden // 16)))
    mats = []
    for i in range(layers):
        f32("l%d.ln1" % i, rng.uniform(0.5, 1.5, hidden))
        f32("l%d.ln2" % i, rng.uniform(0.5, 1.5, hidden))
        for nm, kqt, N, K, H in (("q", 1, hidden, hidden, 2.3), ("gate", 4, inter, hidden, 2.6),
                                 ("up", 2, inter, hidden, 3.4), ("down", 3, hidden, inter, 4.3)):
            name = "l%d.%s" % (i, nm)
            codes, side = bundle.synth_matrix(kqt, N, K, H, 100 * i + kqt)
            w.add_kquant(name, kqt, codes, side)
            mats.append((name, kqt, N, K, H, 100 * i + kqt))
    f32("lnf", rng.uniform(0.5, 1.5, hidden))
    w.close()
    return mats, embed


def test_open_model_shaped_bundle(lib, tmp_path):
    """A model-shaped bundle (non-matrix f32 / raw8 tensors and cfg lines beside mixed-format K-quant matrices) opens;
    every matrix decodes on the CPU to its symbols, the raw8 tensor reads back as stored, and the matrix-only entry
    points refuse the non-matrix tensors with an error instead of exiting."""
    from lazyweights_amd import Runtime, bundle
    mats, embed = write_model_bundle(tmp_path)
    cfg, ts = bundle.read_manifest(str(tmp_path))
    assert cfg["n_layers"] == "2" and cfg["enc"] == "kq_huf"
    with Runtime(tmp_path, budget_mb=0) as rt:
        for name, kqt, N, K, H, seed in mats:
            codes, _ = bundle.synth_matrix(kqt, N, K, H, seed)
            assert np.array_equal(rt.test_cpu_decode(name, 2), bundle.form_symbols(kqt, codes)), name
        s, n = rt.cpu_decode_all(2)
        assert n == sum(N * (K // 2 if kqt in (1, 4) else K) for _, kqt, N, K, _, _ in mats)
        for name in ("embed", "lnf", "l1.ln2"):
            with pytest.raises(RuntimeError):
                rt.test_cpu_decode(name, 1)


def test_cpu_decode_rejects_truncated_and_corrupt_blobs(lib, tmp_path):
    """rt_test_cpu_decode / rt_cpu_decode_all read raw blobs that rt_open did not validate (budget_mb = 0: nothing
    resident). A blob cut inside its lane-start table, one cut inside its payload, and one whose lane starts point
    past the payload are refused with -1 and an error text, never read past the buffer."""
    from lazyweights_amd import Runtime
    from lazyweights_amd.bundle import Writer, encode_huf8
    g = load_golden("huf4p_q4k_128x1024")
    N, KS = g["sym"].shape
    blob, _ = encode_huf8(g["sym"])
    T = (N // 64) * (KS // 256)
    head = 4096 + 128 * T
    bad_start = bytearray(blob)
    bad_start[4096:4100] = np.array([1 << 30], np.uint32).tobytes()   # tile 0, lane 0 starts far past the end
    cases = {"cut_header": blob[:head - 64], "cut_payload": blob[:head + (len(blob) - head) // 2],
             "bad_start": bytes(bad_start)}
    w = Writer(str(tmp_path))
    for name, b in cases.items():
        w.add(name, "huf4p", N, 2 * KS, 1.0, 0, b)
    w.close()
    with Runtime(tmp_path, budget_mb=0) as rt:
        out = np.zeros((N, KS), np.uint8)
        for name in cases:
            assert rt.lib.rt_test_cpu_decode(rt.h, name.encode(), 2, out.ctypes.data) == -1, name
            assert "cpu decode" in rt.lib.lw_last_error().decode(), name
        s, _ = rt.cpu_decode_all(2)
        assert s == -1


def test_writer_and_manifest_round_trip(lib, tmp_path):
    """Writer (the C++ bundle writer through ctypes) and read_manifest: cfg lines, tensors at 256-byte boundaries in
    write order, bytes read back as written, and names with white space refused."""
    from lazyweights_amd import bundle
    rng = np.random.default_rng(5)
    blobs = {"a": rng.integers(0, 256, 300, dtype=np.uint8).tobytes(), "b.kqs": b"", "c": b"\x01" * 257}
    w = bundle.Writer(str(tmp_path))
    w.cfg("hidden", 512)
    w.cfg("eps", "1e-05")
    for i, (name, b) in enumerate(blobs.items()):
        w.add(name, "raw8", 1 + i, max(1, len(b)), 0.5 * (i + 1), i, b)
    with pytest.raises(ValueError):
        w.add("bad name", "raw8", 1, 1, 1.0, 0, b"x")
    w2 = bundle.Writer(str(tmp_path / "two"))
    w2.add("x", "raw8", 1, 3, 1.0, 0, b"xyz")
    w2.close()
    cfg, ts = bundle.read_manifest(str(tmp_path / "two"))
    assert cfg == {} and [t["name"] for t in ts] == ["x"] and ts[0]["offset"] == 0 and ts[0]["nbytes"] == 3
    # missing parent directories are created (the reference Writer's os.makedirs, lazyweights/bundle.py:114-120)
    w3 = bundle.Writer(str(tmp_path / "a" / "b" / "c"))
    w3.add("y", "raw8", 1, 2, 1.0, 0, b"yz")
    w3.close()
    cfg, ts = bundle.read_manifest(str(tmp_path / "a" / "b" / "c"))
    assert [t["name"] for t in ts] == ["y"] and ts[0]["nbytes"] == 2
    w.close()
    cfg, ts = bundle.read_manifest(str(tmp_path))
    assert cfg == {"hidden": "512", "eps": "1e-05"}
    assert [t["name"] for t in ts] == list(blobs)
    prev_end = 0
    for i, t in enumerate(ts):
        assert t["offset"] % 256 == 0 and t["offset"] >= prev_end
        assert (t["N"], t["scale"], t["zp"], t["enc"]) == (1 + i, 0.5 * (i + 1), i, "raw8")
        assert bundle.read_tensor(str(tmp_path), t).tobytes() == blobs[t["name"]]
        prev_end = t["offset"] + t["nbytes"]
