"""GPU parity of the HIP path through the C-ABI, against the oracle.

Bars: decoded codes bit-exact; GEMV / skinny GEMM max|y - y64| / max|y64| <= 1e-3 against the fp64
dequantize-then-matmul (the contract tolerance; the kernels accumulate in fp32 and land near 1e-6, so a tighter
internal bar of 2e-5 is also asserted to catch partial mistakes such as one wrong sub-block scale).
"""
import os
import sys

import numpy as np
import pytest

from conftest import golden_cases, load_golden

pytestmark = pytest.mark.gpu
TOL_CONTRACT, TOL_TIGHT = 1e-3, 2e-5


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def check_err(y, y64, what):
    from oracle.oracle import rel_err
    e = rel_err(y, y64)
    say("  %s rel err %.3g" % (what, e))
    assert e <= TOL_CONTRACT and e <= TOL_TIGHT, (what, e)
    return e


@pytest.fixture(scope="module")
def golden_rt(gpu, tmp_path_factory, lib):
    from lazyweights_amd import Runtime
    from lazyweights_amd.bundle import Writer, encode_huf8
    d = tmp_path_factory.mktemp("golden")
    w = Writer(str(d))
    for case in golden_cases():
        g = load_golden(case)
        N, KS = g["sym"].shape
        four = case.startswith("huf4p")
        blob, _ = encode_huf8(g["sym"])
        w.add(case, "huf4p" if four else "huf8", N, 2 * KS if four else KS, 1.0, 0, blob)
    w.close()
    rt = Runtime(d)
    yield rt
    rt.close()


@pytest.mark.parametrize("case", golden_cases())
def test_gpu_decode_golden(golden_rt, orc, case):
    say("decode golden", case)
    g = load_golden(case)
    four = case.startswith("huf4p")
    want = orc.unpack_symbols(4 if four else 8, g["decoded"])
    assert np.array_equal(golden_rt.test_decode(case), want)


FORMATS = [(1, "Q4_K", 2.3), (2, "Q5_K", 3.4), (3, "Q6_K", 4.3), (4, "IQ4_XS", 2.6)]


@pytest.fixture(scope="module")
def fmt_rt(gpu, tmp_path_factory, lib):
    from lazyweights_amd import Runtime, bundle
    d = tmp_path_factory.mktemp("fmt")
    mats = []
    for kqt, name, H in FORMATS:
        mats.append((name, kqt, 320, 3072, H, 50 + kqt))          # 5 tile rows: a partially filled block
        mats.append((name + "_small", kqt, 64, 512, H, 60 + kqt))  # one tile column
    bundle.write_synthetic_bundle(str(d), mats, threads=8)
    rt = Runtime(d)
    yield rt, {m[0]: m for m in mats}
    rt.close()


def reference_y(orc, mat, X64):
    from lazyweights_amd import bundle
    name, kqt, N, K, H, seed = mat
    codes, side = bundle.synth_matrix(kqt, N, K, H, seed)
    return codes, orc.gemv_f64(orc.dequant(kqt, codes, side), X64)


@pytest.mark.parametrize("kqt,fmt,H", FORMATS)
def test_gpu_decode_formats(fmt_rt, kqt, fmt, H):
    from lazyweights_amd import bundle
    rt, mats = fmt_rt
    for nm in (fmt, fmt + "_small"):
        say("decode", nm)
        name, kqt_, N, K, H_, seed = mats[nm]
        codes, _ = bundle.synth_matrix(kqt_, N, K, H_, seed)
        assert np.array_equal(rt.test_decode(nm), codes)


@pytest.mark.parametrize("kqt,fmt,H", FORMATS)
def test_gpu_fused_fp32_x(fmt_rt, orc, kqt, fmt, H):
    """rt_test_matmul (fp32 host X, fused path) for m = 1..8 against fp64."""
    rt, mats = fmt_rt
    rng = np.random.default_rng(kqt)
    for nm in (fmt, fmt + "_small"):
        mat = mats[nm]
        X = rng.standard_normal((8, mat[3])).astype(np.float32)
        _, y64 = reference_y(orc, mat, X.astype(np.float64))
        for m in (1, 2, 3, 5, 8):
            say("fused fp32", nm, "m", m)
            Y = rt.test_matmul(nm, X[:m], path=0)
            check_err(Y, y64[:m], "%s m=%d" % (nm, m))


@pytest.mark.parametrize("kqt,fmt,H", FORMATS)
def test_gpu_decode_gemm_path(fmt_rt, orc, kqt, fmt, H):
    """path 2 (decode to scratch + GEMM) and m > 8 (auto) against fp64."""
    rt, mats = fmt_rt
    mat = mats[fmt]
    rng = np.random.default_rng(10 + kqt)
    X = rng.uniform(-0.5, 0.5, (12, mat[3])).astype(np.float32)
    _, y64 = reference_y(orc, mat, X.astype(np.float64))
    say("path2", fmt)
    check_err(rt.test_matmul(fmt, X[:3], path=2), y64[:3], fmt + " path2 m=3")
    say("auto m=12", fmt)
    check_err(rt.test_matmul(fmt, X, path=0), y64, fmt + " auto m=12")


@pytest.mark.parametrize("kqt,fmt,H", FORMATS)
def test_gpu_prefill_gemm_matrix_cores(fmt_rt, orc, kqt, fmt, H):
    """Prefill-shaped path 2 (m = 80: two full 32-token tiles and a partial one) through every prefill GEMM (the
    hand-written matrix-core GEMMs over the codes: the default over tiled codes, k_gemm_prefill for Q4_K / Q5_K and
    k_gemm_prefill_sub for Q6_K / IQ4_XS, and the older one over row-major codes; rocBLAS over fp16 hi + lo weights in
    its forms) against fp64, and against the SIMT GEMM (kernel mode 1) to fp32 rounding."""
    rt, mats = fmt_rt
    mat = mats[fmt]
    rng = np.random.default_rng(30 + kqt)
    X = rng.uniform(-1, 1, (80, mat[3])).astype(np.float32)
    _, y64 = reference_y(orc, mat, X.astype(np.float64))
    assert rt.lib.lw_set_kernel_mode(1) == 0
    try:
        Ys = rt.test_matmul(fmt, X, path=2)
    finally:
        rt.lib.lw_set_kernel_mode(0)
    for which, what in ((0, "default (hand-written, tiled codes)"), (2, "rocBLAS two GEMMs"),
                        (3, "rocBLAS one GEMM"), (4, "rocBLAS auto"), (1, "hand-written, row-major codes")):
        say("prefill m=80", fmt, what)
        assert rt.lib.lw_set_prefill_gemm(which) == 0
        try:
            Y = rt.test_matmul(fmt, X, path=2)
        finally:
            rt.lib.lw_set_prefill_gemm(0)
        check_err(Y, y64, "%s prefill m=80 (%s)" % (fmt, what))
        assert np.abs(Y - Ys).max() <= 1e-5 * np.abs(Ys).max()


def test_gpu_prefill_gemm_row_chunks(gpu, tmp_path, orc, lib):
    """A matrix whose codes exceed the 64 MB decode scratch (17408 x 4096 Q4_K: two row chunks), m = 9 (auto path
    2), through the default prefill GEMM (hand-written, tiled codes) and rocBLAS: every chunk lands in its own rows
    of y."""
    from lazyweights_amd import Runtime, bundle
    mat = ("big", 1, 17408, 4096, 2.3, 91)
    bundle.write_synthetic_bundle(str(tmp_path), [mat], threads=8)
    rng = np.random.default_rng(91)
    X = rng.uniform(-1, 1, (9, 4096)).astype(np.float32)
    _, y64 = reference_y(orc, mat, X.astype(np.float64))
    with Runtime(tmp_path) as rt:
        for which, what in ((0, "default"), (4, "rocBLAS")):
            say("prefill row chunks m=9", what)
            assert rt.lib.lw_set_prefill_gemm(which) == 0
            try:
                check_err(rt.test_matmul("big", X), y64, "big m=9 (two row chunks, %s)" % what)
            finally:
                rt.lib.lw_set_prefill_gemm(0)


@pytest.mark.parametrize("kqt,fmt,H", FORMATS)
def test_gpu_fused_fp16_x_device(fmt_rt, orc, kqt, fmt, H):
    """lw_matmul_dev with fp16 activations resident on the GPU (the bench path), m up to 16."""
    import torch
    rt, mats = fmt_rt
    mat = mats[fmt]
    N, K = mat[2], mat[3]
    g = torch.Generator().manual_seed(kqt)
    X = torch.randn(16, K, generator=g).half()
    _, y64 = reference_y(orc, mat, X.double().numpy())
    Xd = X.cuda()
    for m in (1, 2, 4, 5, 8, 16):
        say("fused fp16", fmt, "m", m)
        Y = torch.full((m, N), float("nan"), dtype=torch.float32, device="cuda")
        rt.matmul_dev(fmt, Xd[:m], Y, x_f16=True, stream=torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        check_err(Y.cpu().numpy(), y64[:m], "%s fp16 m=%d" % (fmt, m))


@pytest.mark.parametrize("kqt,fmt,H", FORMATS)
def test_gpu_reduction_with_nan_activations(fmt_rt, orc, kqt, fmt, H):
    """The in-launch reduction takes each partial slot by an exchange with an empty marker (a signalling NaN) and
    re-sums a batch whose sum is NaN. A NaN in the activations makes every partial of its token NaN: that token's
    outputs are NaN, the other tokens' outputs stay exact (m = 5, the matrix-core kernel), nothing waits, and the
    slots are left empty, so the next calls (m = 1 and m = 5) are again within tolerance of fp64."""
    import torch
    rt, mats = fmt_rt
    mat = mats[fmt]
    N, K = mat[2], mat[3]
    g = torch.Generator().manual_seed(70 + kqt)
    X = torch.randn(5, K, generator=g).half()
    _, y64 = reference_y(orc, mat, X.double().numpy())
    st = torch.cuda.current_stream().cuda_stream
    Xn = X.clone()
    Xn[2, K // 3] = float("nan")
    Xn_d = Xn.cuda()
    for m, bad in ((1, None), (5, 2)):
        say("nan activations", fmt, "m", m)
        xin = Xn_d[:m].clone()
        if m == 1:
            xin[0, 7] = float("nan")
        Y = torch.zeros((m, N), dtype=torch.float32, device="cuda")
        rt.matmul_dev(fmt, xin, Y, x_f16=True, stream=st)
        torch.cuda.synchronize()
        y = Y.cpu().numpy()
        if m == 1:
            assert np.isnan(y).all(), fmt
        else:
            assert np.isnan(y[bad]).all(), fmt
            ok = [j for j in range(m) if j != bad]
            check_err(y[ok], y64[ok], "%s m=5 beside a NaN token" % fmt)
    for m in (1, 5):
        Y = torch.zeros((m, N), dtype=torch.float32, device="cuda")
        rt.matmul_dev(fmt, X[:m].cuda(), Y, x_f16=True, stream=st)
        torch.cuda.synchronize()
        check_err(Y.cpu().numpy(), y64[:m], "%s m=%d after the NaN calls" % (fmt, m))


def test_gpu_verify_gemm_equals_repeated_gemv(fmt_rt, orc):
    """One m = 5 launch (products on the matrix cores, sub-block scales folded into the weights: the same products
    summed in another order) against five m = 1 launches (v_dot2): the same values up to the fp32 rounding of a
    K-term sum (5e-6 of max |y|), both within tolerance of fp64; tokens are independent (token 0 alone in an m = 5
    launch with zeroed others gives the same bits as in the full launch)."""
    import torch
    rt, mats = fmt_rt
    for kqt, fmt, H in FORMATS:
        N, K = mats[fmt][2], mats[fmt][3]
        X = torch.randn(5, K).half()
        Xd = X.cuda()
        Y5 = torch.zeros(5, N, device="cuda")
        rt.matmul_dev(fmt, Xd, Y5)
        Y1 = torch.zeros(5, N, device="cuda")
        for j in range(5):
            rt.matmul_dev(fmt, Xd[j:j + 1], Y1[j:j + 1])
        X0 = Xd.clone()
        X0[1:] = 0
        Y0 = torch.zeros(5, N, device="cuda")
        rt.matmul_dev(fmt, X0, Y0)
        torch.cuda.synchronize()
        a, b = Y5.cpu().numpy(), Y1.cpu().numpy()
        _, y64 = reference_y(orc, mats[fmt], X.double().numpy())
        say("verify vs 5 x gemv", fmt, "diff %.3g" % (np.abs(a - b).max() / np.abs(b).max()))
        check_err(a, y64, fmt + " m=5 in one launch")
        check_err(b, y64, fmt + " m=5 as five m=1 launches")
        assert np.abs(a - b).max() <= 5e-6 * np.abs(b).max(), (fmt, np.abs(a - b).max() / np.abs(b).max())
        assert torch.equal(Y0[0], Y5[0])
        _, y64 = reference_y(orc, mats[fmt], X.double().numpy())
        check_err(a, y64, fmt + " m=5")


def test_gpu_decode_all_timing(fmt_rt):
    rt, _ = fmt_rt
    s = rt.gpu_decode_all(3)
    say("gpu_decode_all", s)
    assert s > 0


# ── full BASELINE shapes ─────────────────────────────────────────────────────────────────────────────────

def full_size_check(tmp_path, mats, m_list=(1,)):
    import torch
    from lazyweights_amd import Runtime, bundle
    from oracle import oracle as orc
    bundle.write_synthetic_bundle(str(tmp_path), mats, threads=16)
    with Runtime(tmp_path) as rt:
        for mat in mats:
            name, kqt, N, K, H, seed = mat
            say("full-size", name, N, K)
            codes, side = bundle.synth_matrix(kqt, N, K, H, seed, threads=16)
            assert np.array_equal(rt.test_decode(name), codes)
            X = torch.randn(max(m_list), K).half()
            y64 = orc.gemv_f64(orc.dequant(kqt, codes, side), X.double().numpy())
            Xd = X.cuda()
            for m in m_list:
                Y = torch.zeros(m, N, device="cuda")
                rt.matmul_dev(name, Xd[:m], Y)
                torch.cuda.synchronize()
                check_err(Y.cpu().numpy(), y64[:m], "%s m=%d" % (name, m))
            del codes, side


def test_full_config0(gpu, tmp_path):
    from lazyweights_amd.configs import CONFIG0
    full_size_check(tmp_path, CONFIG0, (1, 5))


def test_full_config2_layer(gpu, tmp_path):
    from lazyweights_amd.configs import config2_layer
    full_size_check(tmp_path, config2_layer(0), (1,))


def test_full_config3_mixed(gpu, tmp_path):
    from lazyweights_amd.configs import CONFIG3
    full_size_check(tmp_path, CONFIG3, (1,))


def test_full_config4_q5k_verify(gpu, tmp_path):
    from lazyweights_amd.configs import CONFIG4
    full_size_check(tmp_path, [m for m in CONFIG4 if m[0] in ("q5.gate", "q5.down")], (5,))


def grouped_matmul(rt, names, xs, m, ys):
    """One lw_group_matmul_dev call over `names` (device x / y torch tensors)."""
    import ctypes
    n = len(names)
    rc = rt.lib.lw_group_matmul_dev(rt.h, n, (ctypes.c_char_p * n)(*[nm.encode() for nm in names]),
                                    (ctypes.c_void_p * n)(*[x.data_ptr() for x in xs]), m,
                                    (ctypes.c_void_p * n)(*[y.data_ptr() for y in ys]), None)
    assert rc == 0, rt.lib.lw_last_error()


def test_full_config1_layer(gpu, tmp_path):
    """Config 1, the Phi-3-mini-shaped layer (qkv 9216 x 3072, o 3072 x 3072, gate_up 16384 x 3072, down 3072 x 8192,
    one Huffman table per matrix): decode bit-exact and m = 1 GEMV against fp64 per matrix, then the whole layer as
    one grouped call (the bench's launch shape) with the same bits as the per-matrix calls."""
    import torch
    from lazyweights_amd import Runtime, bundle
    from lazyweights_amd.configs import CONFIG1
    from oracle import oracle as orc
    bundle.write_synthetic_bundle(str(tmp_path), CONFIG1, threads=16)
    with Runtime(tmp_path) as rt:
        xs, ys, names = [], [], []
        for mat in CONFIG1:
            name, kqt, N, K, H, seed = mat
            say("config 1", name, N, K)
            codes, side = bundle.synth_matrix(kqt, N, K, H, seed, threads=16)
            assert np.array_equal(rt.test_decode(name), codes)
            X = torch.randn(1, K, generator=torch.Generator().manual_seed(seed)).half()
            y64 = orc.gemv_f64(orc.dequant(kqt, codes, side), X.double().numpy())
            Y = torch.zeros(1, N, device="cuda")
            rt.matmul_dev(name, X.cuda(), Y)
            torch.cuda.synchronize()
            check_err(Y.cpu().numpy(), y64, "config 1 %s m=1" % name)
            names.append(name)
            xs.append(X.cuda())
            ys.append(Y)
            del codes, side
        yg = [torch.full_like(y, float("nan")) for y in ys]
        say("config 1 grouped layer")
        grouped_matmul(rt, names, xs, 1, yg)
        torch.cuda.synchronize()
        for nm, a, b in zip(names, yg, ys):
            assert torch.equal(a, b), nm


def test_full_config4_q4k_verify(gpu, tmp_path):
    """Config 4's Q4_K half: the Mistral-shaped layer (H = 2.3) verified with m = 5 tokens as one grouped call, each
    matrix against fp64 (the contract) and against five m = 1 calls token by token (fp32 rounding: the m = 5 kernel
    forms its products on the matrix cores in another order; 5e-6 of max |y|). The m = 1 grouped calls are the
    bench's headline launch (the 7 config-2-shaped matrices of a layer in one launch of the whole-tile kernel): each
    token's results are checked against fp64 directly too (the reference's check, kernels/llmrt.cu:2866-2883)."""
    import torch
    from lazyweights_amd import Runtime, bundle
    from lazyweights_amd.configs import CONFIG4
    from oracle import oracle as orc
    mats = [m for m in CONFIG4 if m[0].startswith("q4.")]
    bundle.write_synthetic_bundle(str(tmp_path), mats, threads=16)
    with Runtime(tmp_path) as rt:
        names = [m[0] for m in mats]
        X = {m[0]: torch.randn(5, m[3], generator=torch.Generator().manual_seed(m[5])).half() for m in mats}
        y5 = {m[0]: torch.zeros(5, m[2], device="cuda") for m in mats}
        say("config 4 Q4_K m=5 grouped")
        grouped_matmul(rt, names, [X[n].cuda() for n in names], 5, [y5[n] for n in names])
        y1 = {m[0]: torch.zeros(5, m[2], device="cuda") for m in mats}
        for j in range(5):
            grouped_matmul(rt, names, [X[n][j:j + 1].cuda() for n in names], 1, [y1[n][j:j + 1] for n in names])
        torch.cuda.synchronize()
        for mat in mats:
            name, kqt, N, K, H, seed = mat
            a, b = y5[name].cpu().numpy(), y1[name].cpu().numpy()
            say("config 4", name, "m=5 vs 5 x m=1: %.3g" % (np.abs(a - b).max() / np.abs(b).max()))
            assert np.abs(a - b).max() <= 5e-6 * np.abs(b).max(), name
            codes, side = bundle.synth_matrix(kqt, N, K, H, seed, threads=16)
            y64 = orc.gemv_f64(orc.dequant(kqt, codes, side), X[name].double().numpy())
            check_err(a, y64, "config 4 %s m=5" % name)
            for j in range(5):  # the grouped m = 1 launch, token by token
                check_err(b[j:j + 1], y64[j:j + 1], "config 4 %s grouped m=1 token %d" % (name, j))
            del codes, side


def test_full_config3_verify(gpu, tmp_path):
    """Config 3's layer (Q6_K down, IQ4_XS gate / up) verified with m = 5 tokens as one grouped call (the
    matrix-core verify kernel for every format): each matrix against fp64 and against five m = 1 grouped calls
    (5e-6 of max |y|), which are checked against fp64 token by token too."""
    import torch
    from lazyweights_amd import Runtime, bundle
    from lazyweights_amd.configs import CONFIG3
    from oracle import oracle as orc
    bundle.write_synthetic_bundle(str(tmp_path), CONFIG3, threads=16)
    with Runtime(tmp_path) as rt:
        names = [m[0] for m in CONFIG3]
        X = {m[0]: torch.randn(5, m[3], generator=torch.Generator().manual_seed(m[5])).half() for m in CONFIG3}
        y5 = {m[0]: torch.zeros(5, m[2], device="cuda") for m in CONFIG3}
        say("config 3 m=5 grouped")
        grouped_matmul(rt, names, [X[n].cuda() for n in names], 5, [y5[n] for n in names])
        y1 = {m[0]: torch.zeros(5, m[2], device="cuda") for m in CONFIG3}
        for j in range(5):
            grouped_matmul(rt, names, [X[n][j:j + 1].cuda() for n in names], 1, [y1[n][j:j + 1] for n in names])
        torch.cuda.synchronize()
        for mat in CONFIG3:
            name, kqt, N, K, H, seed = mat
            a, b = y5[name].cpu().numpy(), y1[name].cpu().numpy()
            say("config 3", name, "m=5 vs 5 x m=1: %.3g" % (np.abs(a - b).max() / np.abs(b).max()))
            assert np.abs(a - b).max() <= 5e-6 * np.abs(b).max(), name
            codes, side = bundle.synth_matrix(kqt, N, K, H, seed, threads=16)
            y64 = orc.gemv_f64(orc.dequant(kqt, codes, side), X[name].double().numpy())
            check_err(a, y64, "config 3 %s m=5" % name)
            check_err(b, y64, "config 3 %s 5 x m=1" % name)
            del codes, side


def test_gpu_whole_tile_kernel_mode(fmt_rt, orc):
    """The whole-tile kernel (the fallback for matrices without a ring schedule) stays exact too."""
    import torch
    rt, mats = fmt_rt
    assert rt.lib.lw_set_kernel_mode(1) == 0
    try:
        for kqt, fmt, H in FORMATS:
            mat = mats[fmt]
            X = torch.randn(2, mat[3]).half()
            _, y64 = reference_y(orc, mat, X.double().numpy())
            say("whole-tile kernel", fmt)
            Y = torch.zeros(2, mat[2], device="cuda")
            rt.matmul_dev(fmt, X.cuda(), Y)
            torch.cuda.synchronize()
            check_err(Y.cpu().numpy(), y64, fmt + " whole-tile")
    finally:
        rt.lib.lw_set_kernel_mode(0)


def test_gpu_grouped_launch_matches_single(fmt_rt):
    """lw_group_matmul_dev over mixed formats (several grouped launches + whole batches of reductions) gives the
    same bits as one call per matrix."""
    import ctypes

    import torch
    rt, mats = fmt_rt
    names = list(mats)
    X = [torch.randn(1, mats[nm][3]).half().cuda() for nm in names]
    Yg = [torch.zeros(1, mats[nm][2], device="cuda") for nm in names]
    Ys = [torch.zeros(1, mats[nm][2], device="cuda") for nm in names]
    n = len(names)
    rc = rt.lib.lw_group_matmul_dev(rt.h, n, (ctypes.c_char_p * n)(*[nm.encode() for nm in names]),
                                    (ctypes.c_void_p * n)(*[x.data_ptr() for x in X]), 1,
                                    (ctypes.c_void_p * n)(*[y.data_ptr() for y in Yg]), None)
    assert rc == 0, rt.lib.lw_last_error()
    for nm, x, y in zip(names, X, Ys):
        rt.matmul_dev(nm, x, y)
    torch.cuda.synchronize()
    say("grouped vs single", n)
    for a, b in zip(Yg, Ys):
        assert torch.equal(a, b)


def verify_on_exception_tiles(rt, name, W64, K, N, orc):
    """fp16 device x at m = 2, 5 and 8 on a matrix with exception tiles: the default (the matrix-core verify kernel,
    every tile in place) against the ring kernels (mode 7, exception tiles through their separate pass) within
    5e-6 of max |y|, both within tolerance of fp64."""
    import torch
    for m in (2, 5, 8):
        X = torch.randn(m, K).half()
        y64 = orc.gemv_f64(W64, X.double().numpy())
        ys = {}
        for mode in (0, 7):
            assert rt.lib.lw_set_kernel_mode(mode) == 0
            try:
                Y = torch.zeros(m, N, device="cuda")
                rt.matmul_dev(name, X.cuda(), Y)
                torch.cuda.synchronize()
                ys[mode] = Y.cpu().numpy()
            finally:
                rt.lib.lw_set_kernel_mode(0)
            check_err(ys[mode], y64, "%s m=%d mode %d" % (name, m, mode))
        assert np.abs(ys[0] - ys[7]).max() <= 5e-6 * np.abs(ys[7]).max(), (name, m)


def test_gpu_ring_exception_tile(gpu, tmp_path, orc):
    """A matrix whose tile 5 has no ring schedule: the ring kernel skips it and an exception pass decodes it (the
    low-latency kernel for m = 1, the whole-tile kernel for m > 1); GEMV (m = 1, fp16 x) and fp32-x m = 3 against
    fp64, decode bit-exact."""
    import torch
    from lazyweights_amd import Runtime
    from lazyweights_amd.bundle import Writer
    from test_layout import skewed_tile_codes
    codes, side = skewed_tile_codes()
    w = Writer(str(tmp_path))
    w.add_kquant("skew", 2, codes, side)
    w.close()
    with Runtime(tmp_path) as rt:
        say("exception tile: decode")
        assert np.array_equal(rt.test_decode("skew"), codes)
        W64 = orc.dequant(2, codes, side)
        X = torch.randn(3, 8192).half()
        y64 = orc.gemv_f64(W64, X.double().numpy())
        Y = torch.zeros(1, 128, device="cuda")
        rt.matmul_dev("skew", X[:1].cuda(), Y)
        torch.cuda.synchronize()
        check_err(Y.cpu().numpy(), y64[:1], "exception tile m=1")
        check_err(rt.test_matmul("skew", X.float().numpy(), path=0), y64, "exception tile fp32 m=3")
        verify_on_exception_tiles(rt, "skew", W64, 8192, 128, orc)


def test_gpu_exception_tiles_in_place(gpu, tmp_path, orc):
    """Two adjacent exception tiles with 32-row schedules (one block of the flat kernel): decoded in place in two
    spare rings, alone (W = 16) and grouped with an 8-tile matrix (W = 8); the same bits as the separate one-wave
    exception pass (mode 3) and within tolerance of fp64. m = 3 (block-per-column kernel) takes the exception pass."""
    import ctypes

    import torch
    from lazyweights_amd import Runtime, bundle
    from lazyweights_amd.bundle import Writer
    from test_layout import mild_skew_codes
    codes, side = mild_skew_codes()
    small, small_side = bundle.synth_matrix(2, 64, 2048, 3.4, 11)
    w = Writer(str(tmp_path))
    w.add_kquant("mskew", 2, codes, side)
    w.add_kquant("small", 2, small, small_side)
    w.close()
    with Runtime(tmp_path) as rt:
        say("in-place exceptions: decode")
        assert np.array_equal(rt.test_decode("mskew"), codes)
        W64 = orc.dequant(2, codes, side)
        Ws = orc.dequant(2, small, small_side)
        X = torch.randn(3, 8192).half()
        xs = torch.randn(1, 2048).half()
        y64 = orc.gemv_f64(W64, X.double().numpy())
        ys64 = orc.gemv_f64(Ws, xs.double().numpy())

        def group(names, xs_):
            xd = [x.cuda() for x in xs_]
            ys = [torch.zeros(1, {"mskew": 128, "small": 64}[nm], device="cuda") for nm in names]
            n = len(names)
            rc = rt.lib.lw_group_matmul_dev(rt.h, n, (ctypes.c_char_p * n)(*[nm.encode() for nm in names]),
                                            (ctypes.c_void_p * n)(*[x.data_ptr() for x in xd]), 1,
                                            (ctypes.c_void_p * n)(*[y.data_ptr() for y in ys]), None)
            assert rc == 0, rt.lib.lw_last_error()
            torch.cuda.synchronize()
            return [y.cpu().numpy() for y in ys]

        runs = {}
        for mode in (7, 3, 0):  # ring with exceptions in place, ring with the exception pass, whole-tile kernel
            assert rt.lib.lw_set_kernel_mode(mode) == 0
            try:
                say("in-place exceptions: mode %d" % mode)
                runs[mode] = group(["mskew"], [X[:1]]) + group(["small", "mskew"], [xs, X[:1]])
            finally:
                rt.lib.lw_set_kernel_mode(0)
        for k in (3, 0):
            for a, b in zip(runs[7], runs[k]):
                assert np.array_equal(a, b), k
        check_err(runs[0][0], y64[:1], "in-place exceptions alone")
        check_err(runs[0][1], ys64, "in-place exceptions grouped: small")
        check_err(runs[0][2], y64[:1], "in-place exceptions grouped")
        check_err(rt.test_matmul("mskew", X.float().numpy(), path=0), y64, "exception pass fp32 m=3")
        verify_on_exception_tiles(rt, "mskew", W64, 8192, 128, orc)


def test_gpu_low_latency_kernel_same_bits(fmt_rt, orc, tmp_path):
    """The low-latency kernel (8 chains per lane, whole tile in LDS; mode 4) gives the same bits as the ring
    kernels (mode 5), for every format, single matrices and a group spanning several matrices; also for matrices
    with exception tiles (with and without a 32-row schedule), whose ring path takes the exception passes."""
    import ctypes

    import torch
    from lazyweights_amd import Runtime
    from lazyweights_amd.bundle import Writer
    from test_layout import mild_skew_codes, skewed_tile_codes

    def run(rt, names, xs, mode):
        assert rt.lib.lw_set_kernel_mode(mode) == 0
        try:
            ys = [torch.zeros(1, rt.info(nm)["N"], device="cuda") for nm in names]
            n = len(names)
            rc = rt.lib.lw_group_matmul_dev(rt.h, n, (ctypes.c_char_p * n)(*[nm.encode() for nm in names]),
                                            (ctypes.c_void_p * n)(*[x.data_ptr() for x in xs]), 1,
                                            (ctypes.c_void_p * n)(*[y.data_ptr() for y in ys]), None)
            assert rc == 0, rt.lib.lw_last_error()
            torch.cuda.synchronize()
            return [y.cpu() for y in ys]
        finally:
            rt.lib.lw_set_kernel_mode(0)

    rt, mats = fmt_rt
    for kqt, fmt, H in FORMATS:
        for names in ([fmt], [fmt + "_small", fmt, fmt + "_small"]):
            X = [torch.randn(1, mats[nm][3]).half() for nm in names]
            xs = [x.cuda() for x in X]
            a, b = run(rt, names, xs, 4), run(rt, names, xs, 5)
            say("low-latency kernel", fmt, len(names))
            for nm, x, ya, yb in zip(names, X, a, b):
                assert torch.equal(ya, yb), nm
                _, y64 = reference_y(orc, mats[nm], x.double().numpy())
                check_err(ya.numpy(), y64, "%s low-latency" % nm)
    w = Writer(str(tmp_path))
    for nm, (codes, side) in (("mskew", mild_skew_codes()), ("skew", skewed_tile_codes())):
        w.add_kquant(nm, 2, codes, side)
    w.close()
    with Runtime(tmp_path) as rt2:
        x = torch.randn(1, 8192).half().cuda()
        for nm in ("mskew", "skew"):
            a, b = run(rt2, [nm], [x], 4), run(rt2, [nm], [x], 5)
            say("low-latency kernel, exception tiles", nm)
            assert torch.equal(a[0], b[0]), nm


def test_gpu_tiles_kernel_same_bits(fmt_rt, orc, tmp_path):
    """The whole-tile flat kernel (a tile per wave in LDS, 8 chains per lane; the m = 1 default, mode 0) gives the
    ring kernels' bits (mode 5) for every format, for single matrices and groups spanning several matrices (blocks over
    two tables), and for matrices with exception tiles, which it decodes like any other tile."""
    import ctypes

    import torch
    from lazyweights_amd import Runtime
    from lazyweights_amd.bundle import Writer
    from test_layout import mild_skew_codes, skewed_tile_codes

    def run(rt, names, xs, mode):
        assert rt.lib.lw_set_kernel_mode(mode) == 0
        try:
            ys = [torch.zeros(1, rt.info(nm)["N"], device="cuda") for nm in names]
            n = len(names)
            rc = rt.lib.lw_group_matmul_dev(rt.h, n, (ctypes.c_char_p * n)(*[nm.encode() for nm in names]),
                                            (ctypes.c_void_p * n)(*[x.data_ptr() for x in xs]), 1,
                                            (ctypes.c_void_p * n)(*[y.data_ptr() for y in ys]), None)
            assert rc == 0, rt.lib.lw_last_error()
            torch.cuda.synchronize()
            return [y.cpu() for y in ys]
        finally:
            rt.lib.lw_set_kernel_mode(0)

    rt, mats = fmt_rt
    for kqt, fmt, H in FORMATS:
        for names in ([fmt], [fmt + "_small"], [fmt + "_small", fmt, fmt + "_small"]):
            X = [torch.randn(1, mats[nm][3]).half() for nm in names]
            xs = [x.cuda() for x in X]
            a, b, c = run(rt, names, xs, 0), run(rt, names, xs, 5), run(rt, names, xs, 7)
            say("whole-tile flat kernel", fmt, len(names))
            for nm, x, ya, yb, yc in zip(names, X, a, b, c):
                assert torch.equal(ya, yb), nm
                assert torch.equal(ya, yc), nm
                _, y64 = reference_y(orc, mats[nm], x.double().numpy())
                check_err(ya.numpy(), y64, "%s whole-tile kernel" % nm)
    w = Writer(str(tmp_path))
    cases = {"mskew": mild_skew_codes(), "skew": skewed_tile_codes()}
    for nm, (codes, side) in cases.items():
        w.add_kquant(nm, 2, codes, side)
    w.close()
    with Runtime(tmp_path) as rt2:
        x = torch.randn(1, 8192).half()
        for nm, (codes, side) in cases.items():
            a, b, c = run(rt2, [nm], [x.cuda()], 0), run(rt2, [nm], [x.cuda()], 5), run(rt2, [nm], [x.cuda()], 7)
            say("whole-tile flat kernel, exception tiles", nm)
            assert torch.equal(a[0], b[0]), nm
            assert torch.equal(a[0], c[0]), nm
            check_err(a[0].numpy(), orc.gemv_f64(orc.dequant(2, codes, side), x.double().numpy()), nm)


def test_gpu_comparator_lookup_same_bits(fmt_rt, orc, tmp_path):
    """Kernel mode 9: the whole-tile kernel looking each code up by the comparator (the canonical code's per-length
    limits, reference hw/huff/huff_engine.h:54-77, in a 256-entry table of entries in canonical order) instead of
    the 2048-entry table gives the table's bits (mode 6, the same kernel with the table) for every format, for single
    matrices and groups whose blocks span two tables, and for matrices with exception tiles."""
    import ctypes

    import torch
    from lazyweights_amd import Runtime
    from lazyweights_amd.bundle import Writer
    from test_layout import mild_skew_codes, skewed_tile_codes

    def run(rt, names, xs, mode):
        assert rt.lib.lw_set_kernel_mode(mode) == 0
        try:
            ys = [torch.zeros(1, rt.info(nm)["N"], device="cuda") for nm in names]
            n = len(names)
            rc = rt.lib.lw_group_matmul_dev(rt.h, n, (ctypes.c_char_p * n)(*[nm.encode() for nm in names]),
                                            (ctypes.c_void_p * n)(*[x.data_ptr() for x in xs]), 1,
                                            (ctypes.c_void_p * n)(*[y.data_ptr() for y in ys]), None)
            assert rc == 0, rt.lib.lw_last_error()
            torch.cuda.synchronize()
            return [y.cpu() for y in ys]
        finally:
            rt.lib.lw_set_kernel_mode(0)

    rt, mats = fmt_rt
    for kqt, fmt, H in FORMATS:
        for names in ([fmt], [fmt + "_small"], [fmt + "_small", fmt, fmt + "_small"]):
            X = [torch.randn(1, mats[nm][3]).half() for nm in names]
            xs = [x.cuda() for x in X]
            say("comparator lookup", fmt, len(names))
            a, b = run(rt, names, xs, 9), run(rt, names, xs, 6)
            for nm, x, ya, yb in zip(names, X, a, b):
                assert torch.equal(ya, yb), nm
                _, y64 = reference_y(orc, mats[nm], x.double().numpy())
                check_err(ya.numpy(), y64, "%s comparator lookup" % nm)
    w = Writer(str(tmp_path))
    cases = {"mskew": mild_skew_codes(), "skew": skewed_tile_codes()}
    for nm, (codes, side) in cases.items():
        w.add_kquant(nm, 2, codes, side)
    w.close()
    with Runtime(tmp_path) as rt2:
        x = torch.randn(1, 8192).half()
        for nm, (codes, side) in cases.items():
            say("comparator lookup, exception tiles", nm)
            a, b = run(rt2, [nm], [x.cuda()], 9), run(rt2, [nm], [x.cuda()], 6)
            assert torch.equal(a[0], b[0]), nm
            check_err(a[0].numpy(), orc.gemv_f64(orc.dequant(2, codes, side), x.double().numpy()), nm)


def test_gpu_half_tile_kernel_same_bits(gpu, tmp_path, orc):
    """The half-tile kernel (kernel mode 8; the m = 1 default where whole tiles would give a block's waves fewer than
    two each) gives the whole-tile (mode 6) and ring (mode 7) kernels' bits for every format, on matrices with 7 tiles
    per block, so that waves decode second units claimed when a wave frees up, and on a group of two (14 tiles per
    block), whose waves claim units one ahead; and mode 0 picks it for the single matrix, with the same bits."""
    import ctypes

    import torch
    from lazyweights_amd import Runtime, bundle

    mats = []
    for kqt, fmt, H in FORMATS:
        K = 4096 if kqt in (1, 4) else 2048  # 8 tile columns
        mats.append((fmt, kqt, 14336, K, H, 70 + kqt))
    bundle.write_synthetic_bundle(str(tmp_path), mats, threads=16)

    def run(rt, names, xs, mode):
        assert rt.lib.lw_set_kernel_mode(mode) == 0
        try:
            ys = [torch.zeros(1, rt.info(nm)["N"], device="cuda") for nm in names]
            n = len(names)
            rc = rt.lib.lw_group_matmul_dev(rt.h, n, (ctypes.c_char_p * n)(*[nm.encode() for nm in names]),
                                            (ctypes.c_void_p * n)(*[x.data_ptr() for x in xs]), 1,
                                            (ctypes.c_void_p * n)(*[y.data_ptr() for y in ys]), None)
            assert rc == 0, rt.lib.lw_last_error()
            torch.cuda.synchronize()
            return [y.cpu() for y in ys]
        finally:
            rt.lib.lw_set_kernel_mode(0)

    with Runtime(tmp_path) as rt:
        for name, kqt, N, K, H, seed in mats:
            x = torch.randn(1, K).half()
            xs = [x.cuda()]
            h, t, r, d = (run(rt, [name], xs, mode)[0] for mode in (8, 6, 7, 0))
            say("half-tile kernel", name)
            assert torch.equal(h, t), name
            assert torch.equal(h, r), name
            assert torch.equal(h, d), name
            codes, side = bundle.synth_matrix(kqt, N, K, H, seed, threads=16)
            check_err(h.numpy(), orc.gemv_f64(orc.dequant(kqt, codes, side), x.double().numpy()), name)
            del codes, side
            pair = [name, name]
            xs2 = [x.cuda(), torch.randn(1, K).half().cuda()]
            g8, g6 = run(rt, pair, xs2, 8), run(rt, pair, xs2, 6)
            say("half-tile kernel, group of two", name)
            for a, b in zip(g8, g6):
                assert torch.equal(a, b), name
            assert torch.equal(g8[0], h), name


def test_gpu_packed_twin_same_bits(gpu, tmp_path, orc):
    """The packed twin (pk4 / pk8) of every format gives the coded matrix's bits: m = 1 (grouped, several matrices,
    with a one-tile IQ4_XS matrix so the flat launch runs one-wave blocks that use all 256 table entries), m = 5, the
    fp32-x path and the prefill path; its GPU decode returns the codes."""
    import ctypes

    import torch
    from lazyweights_amd import Runtime, bundle
    mats = [("m%d" % kqt, kqt, N, K, H, 20 + kqt) for kqt, N, K, H in
            ((1, 128, 2048, 2.3), (2, 128, 1024, 3.4), (3, 64, 1024, 4.3), (4, 128, 2048, 2.6))]
    mats.append(("m4s", 4, 64, 512, 2.6, 30))
    bundle.write_synthetic_bundle(str(tmp_path / "coded"), mats, threads=4)
    bundle.write_packed_bundle(str(tmp_path / "packed"), mats, threads=4)
    with Runtime(tmp_path / "coded") as rc, Runtime(tmp_path / "packed") as rp:
        names = [m[0] for m in mats]
        xs = [torch.randn(1, m[3]).half().cuda() for m in mats]

        def group(rt):
            ys = [torch.zeros(1, m[2], device="cuda") for m in mats]
            n = len(names)
            assert rt.lib.lw_group_matmul_dev(rt.h, n, (ctypes.c_char_p * n)(*[nm.encode() for nm in names]),
                                              (ctypes.c_void_p * n)(*[x.data_ptr() for x in xs]), 1,
                                              (ctypes.c_void_p * n)(*[y.data_ptr() for y in ys]), None) == 0
            torch.cuda.synchronize()
            return [y.cpu() for y in ys]
        for (name, kqt, N, K, H, seed), a, b in zip(mats, group(rc), group(rp)):
            say("packed twin m=1", name)
            assert torch.equal(a, b), name
            codes, side = bundle.synth_matrix(kqt, N, K, H, seed)
            assert np.array_equal(rp.test_decode(name), codes)
            # m = 5: the ring kernel (mode 7) gives the packed twin's bits; the default (the matrix-core whole-tile
            # kernel) the same values up to the fp32 order of its sums
            X5 = torch.randn(5, K).half().cuda()
            y5c, y5p, y5d = (torch.zeros(5, N, device="cuda") for _ in range(3))
            assert rc.lib.lw_set_kernel_mode(7) == 0
            try:
                rc.matmul_dev(name, X5, y5c)
            finally:
                rc.lib.lw_set_kernel_mode(0)
            rp.matmul_dev(name, X5, y5p)
            rc.matmul_dev(name, X5, y5d)
            torch.cuda.synchronize()
            assert torch.equal(y5c, y5p), name
            a5, b5 = y5d.cpu().numpy(), y5p.cpu().numpy()
            assert np.abs(a5 - b5).max() <= 5e-6 * np.abs(b5).max(), name
            X3 = np.random.default_rng(kqt).standard_normal((3, K)).astype(np.float32)
            yc, yp = rc.test_matmul(name, X3), rp.test_matmul(name, X3)
            assert np.array_equal(yc, yp), name
            y64 = orc.gemv_f64(orc.dequant(kqt, codes, side), X3.astype(np.float64))
            check_err(yp, y64, name + " packed fp32 m=3")
            # prefill path: the coded matrix's decode and the packed one's unpack give the same tiled codes (IQ4_XS:
            # grid bytes), so the same GEMM bits
            X12 = np.random.default_rng(kqt + 7).standard_normal((12, K)).astype(np.float32)
            yc, yp = rc.test_matmul(name, X12, path=2), rp.test_matmul(name, X12, path=2)
            assert np.array_equal(yc, yp), name
            check_err(yp, orc.gemv_f64(orc.dequant(kqt, codes, side), X12.astype(np.float64)), name + " prefill m=12")


def test_gpu_flat_kernel_spans_and_modes(fmt_rt, orc):
    """The m = 1 flat kernel: one launch over matrices of different sizes (blocks spanning two matrices and two
    tile columns) gives the same bits as one call per matrix and as the block-per-column ring kernel (mode 2),
    and every result is within tolerance of fp64."""
    import ctypes

    import torch
    rt, mats = fmt_rt
    for kqt, fmt, H in FORMATS:
        names = [fmt, fmt + "_small", fmt, fmt + "_small"]
        X = [torch.randn(1, mats[nm][3]).half() for nm in names]
        Xd = [x.cuda() for x in X]
        Yg = [torch.zeros(1, mats[nm][2], device="cuda") for nm in names]
        n = len(names)
        rc = rt.lib.lw_group_matmul_dev(rt.h, n, (ctypes.c_char_p * n)(*[nm.encode() for nm in names]),
                                        (ctypes.c_void_p * n)(*[x.data_ptr() for x in Xd]), 1,
                                        (ctypes.c_void_p * n)(*[y.data_ptr() for y in Yg]), None)
        assert rc == 0, rt.lib.lw_last_error()
        assert rt.lib.lw_set_kernel_mode(2) == 0
        try:
            Yb = [torch.zeros_like(y) for y in Yg]
            for nm, x, y in zip(names, Xd, Yb):
                rt.matmul_dev(nm, x, y)
        finally:
            rt.lib.lw_set_kernel_mode(0)
        Ys = [torch.zeros_like(y) for y in Yg]
        for nm, x, y in zip(names, Xd, Ys):
            rt.matmul_dev(nm, x, y)
        torch.cuda.synchronize()
        say("flat kernel spans / modes", fmt)
        for nm, x, a, b, c in zip(names, X, Yg, Yb, Ys):
            assert torch.equal(a, c) and torch.equal(a, b), nm
            _, y64 = reference_y(orc, mats[nm], x.double().numpy())
            check_err(a.cpu().numpy(), y64, "%s flat" % nm)


@pytest.mark.parametrize("m", [1, 5])
def test_gpu_mixed_format_whole_tile_launch(fmt_rt, orc, m):
    """m = 1 and m = 5 (the matrix-core kernel) over matrices of several K-quant types in one grouped call: two types
    share a whole-tile launch (FlatPlan::nfa: entries of the smaller type code first, blocks spanning a matrix of each
    type). The bits equal one call per matrix (each its own single-type launch) and every result is within tolerance
    of fp64."""
    import ctypes

    import torch
    rt, mats = fmt_rt
    for names in (["Q4_K", "Q6_K_small", "IQ4_XS", "Q5_K", "Q6_K"], ["IQ4_XS", "Q6_K", "IQ4_XS_small"],
                  ["Q5_K_small", "Q4_K", "Q4_K_small", "Q5_K"]):
        say("mixed-format launch m=%d" % m, names)
        X = [torch.randn(m, mats[nm][3]).half() for nm in names]
        Xd = [x.cuda() for x in X]
        Yg = [torch.zeros(m, mats[nm][2], device="cuda") for nm in names]
        n = len(names)
        rc = rt.lib.lw_group_matmul_dev(rt.h, n, (ctypes.c_char_p * n)(*[nm.encode() for nm in names]),
                                        (ctypes.c_void_p * n)(*[x.data_ptr() for x in Xd]), m,
                                        (ctypes.c_void_p * n)(*[y.data_ptr() for y in Yg]), None)
        assert rc == 0, rt.lib.lw_last_error()
        Ys = [torch.zeros_like(y) for y in Yg]
        for nm, x, y in zip(names, Xd, Ys):
            rt.matmul_dev(nm, x, y)
        torch.cuda.synchronize()
        for nm, x, a, c in zip(names, X, Yg, Ys):
            assert torch.equal(a, c), nm
            _, y64 = reference_y(orc, mats[nm], x.double().numpy())
            check_err(a.cpu().numpy(), y64, "%s in a mixed launch, m=%d" % (nm, m))


def test_gpu_model_shaped_bundle(gpu, tmp_path, orc):
    """A bundle laid out as the reference's model exporter writes one (cfg lines, raw8 / f32 tensors, mixed-format
    K-quant matrices with their side tensors): every matrix resident, its GPU decode equal to the codes, m = 1 and
    m = 3 products within the contract, one grouped call over a layer's four formats equal to per-matrix calls; the
    raw8 tensor reads back as stored and the f32 tensors are refused by the matrix entry points; with a 1 MB
    residency budget the first matrices are resident and the last is refused."""
    import ctypes

    import torch
    from lazyweights_amd import Runtime, bundle
    from test_runtime_cpu import write_model_bundle
    mats, embed = write_model_bundle(tmp_path)
    rng = np.random.default_rng(4)
    with Runtime(tmp_path) as rt:
        assert rt.stat("resident_bytes") > 0
        for name, kqt, N, K, H, seed in mats:
            say("model bundle", name)
            codes, side = bundle.synth_matrix(kqt, N, K, H, seed)
            assert np.array_equal(rt.test_decode(name), codes), name
            X = rng.standard_normal((3, K)).astype(np.float32)
            y64 = orc.gemv_f64(orc.dequant(kqt, codes, side), X.astype(np.float64))
            check_err(rt.test_matmul(name, X[:1]), y64[:1], name + " m=1")
            check_err(rt.test_matmul(name, X), y64, name + " m=3")
        assert np.array_equal(rt.test_decode("embed"), embed)
        with pytest.raises(RuntimeError):
            rt.test_matmul("lnf", np.zeros((1, 512), np.float32))
        layer = [m for m in mats if m[0].startswith("l1.")]
        names = [m[0] for m in layer]
        xs = [torch.randn(1, m[3]).half().cuda() for m in layer]
        ys = [torch.zeros(1, m[2], device="cuda") for m in layer]
        n = len(names)
        assert rt.lib.lw_group_matmul_dev(rt.h, n, (ctypes.c_char_p * n)(*[s.encode() for s in names]),
                                          (ctypes.c_void_p * n)(*[x.data_ptr() for x in xs]), 1,
                                          (ctypes.c_void_p * n)(*[y.data_ptr() for y in ys]), None) == 0
        for nm, x, y in zip(names, xs, ys):
            y1 = torch.zeros_like(y)
            rt.matmul_dev(nm, x, y1)
            torch.cuda.synchronize()
            assert torch.equal(y, y1), nm
    # residency budget (the reference's budget_mb, kernels/llmrt.cu:2037-2061): matrices in manifest order until the
    # next one would pass the budget; the rest stay host-only and the GPU entry points refuse them
    with Runtime(tmp_path, budget_mb=1) as rt:
        say("model bundle, budget 1 MB: resident %.0f bytes" % rt.stat("resident_bytes"))
        assert 0 < rt.stat("resident_bytes") < 2 << 20  # the budget counts coded bytes; sides come on top
        first, last = mats[0], mats[-1]
        codes, side = bundle.synth_matrix(*first[1:])
        X = rng.standard_normal((1, first[3])).astype(np.float32)
        check_err(rt.test_matmul(first[0], X), orc.gemv_f64(orc.dequant(first[1], codes, side), X.astype(np.float64)),
                  first[0] + " within budget")
        with pytest.raises(RuntimeError, match="not resident"):
            rt.test_matmul(last[0], np.zeros((1, last[3]), np.float32))
