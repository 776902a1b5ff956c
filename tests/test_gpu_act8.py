"""GPU parity of the int8-activation path (lw_set_act8) through the C-ABI, against the oracle.

The reference's act8 kernels (kernels/llmrt.cu:1035-1169) quantize x per block of 32 and take integer dot products
per sub-block, for up to 8 tokens in one pass over the weights. Bars: the quantization (q, d, d sum q) bit-exact
against oracle.quant_x8, for fp32 and fp16 x; the GEMV within 2e-5 of max |y| of oracle.gemv_act8_f64 (the fp64 value
of the same integer sums and scales: only the fp32 scale products and the accumulation over sub-blocks round); coded,
packed, ring and low-latency kernels the same bits; a several-token pass of the ring and low-latency kernels the same
bits, token by token, as m = 1 calls, and of the default matrix-core kernel (the same exact sub-block sums, scaled
and added in another order) within 5e-6 of max |y| of them. Against the fp64 product with the unquantized x the int8
result carries the quantization error (about 0.5 % of max |y| for Gaussian x), asserted below 2e-2 as a sanity bound.
"""
import ctypes
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu
TOL_ACT8, TOL_QUANT = 2e-5, 2e-2
FORMATS = [(1, "Q4_K", 2.3), (2, "Q5_K", 3.4), (3, "Q6_K", 4.3), (4, "IQ4_XS", 2.6)]


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture
def act8(lib):
    assert lib.lw_set_act8(1) == 0
    yield
    lib.lw_set_act8(0)
    lib.lw_set_kernel_mode(0)


@pytest.fixture(scope="module")
def a8_rt(gpu, tmp_path_factory, lib):
    from lazyweights_amd import Runtime, bundle
    d = tmp_path_factory.mktemp("act8")
    mats = []
    for kqt, name, H in FORMATS:
        mats.append((name, kqt, 320, 3072, H, 70 + kqt))
        mats.append((name + "_small", kqt, 64, 512, H, 80 + kqt))
    bundle.write_synthetic_bundle(str(d / "coded"), mats, threads=8)
    bundle.write_packed_bundle(str(d / "packed"), mats, threads=8)
    rc, rp = Runtime(d / "coded"), Runtime(d / "packed")
    yield rc, rp, {m[0]: m for m in mats}
    rc.close()
    rp.close()


def quant_dev(lib, x, f16):
    m, K = x.shape
    q = np.zeros((m, K), np.int8)
    d = np.zeros((m, K // 32), np.float32)
    s = np.zeros((m, K // 32), np.float32)
    x = np.ascontiguousarray(x)
    assert lib.lw_test_quant_x8(x.ctypes.data, int(f16), m, K, q.ctypes.data, d.ctypes.data, s.ctypes.data) == 0
    return q, d, s


def test_gpu_quant_x8_bit_exact(gpu, lib, orc):
    rng = np.random.default_rng(8)
    x = (rng.standard_normal((3, 4096)) * rng.uniform(1e-3, 1e2, (3, 1))).astype(np.float32)
    x[0, :32] = 0                                                   # a zero block
    x[0, 32:64] = np.arange(32, dtype=np.float32) - 15.5            # halves: max 15.5 -> d = 15.5 / 127
    x[1, 64:96] = 0
    x[1, 70] = -1e-30                                               # one tiny value
    x[2, 96:128] = np.float32(127) * (np.arange(32) % 2) + 0.5      # d = 127.5 / 127, ties near
    for f16 in (False, True):
        xin = x.astype(np.float16) if f16 else x
        say("quant_x8 f16=%d" % f16)
        q, d, s = quant_dev(lib, xin, f16)
        q0, d0, s0 = orc.quant_x8(xin.astype(np.float32))
        assert np.array_equal(q, q0)
        assert np.array_equal(d.view(np.uint32), d0.view(np.uint32))
        assert np.array_equal(s.view(np.uint32), s0.view(np.uint32))


def y_act8(orc, mat, x):
    from lazyweights_amd import bundle
    name, kqt, N, K, H, seed = mat
    codes, side = bundle.synth_matrix(kqt, N, K, H, seed)
    q, d, s = orc.quant_x8(x)
    return orc.gemv_act8_f64(kqt, codes, side, q, d, s), orc.gemv_f64(orc.dequant(kqt, codes, side),
                                                                       x.astype(np.float64))


def same_token(a, b, mode, what):
    """A token of a several-token pass against its own m = 1 call: the same bits, except for the default mode's
    matrix-core kernel (the same exact integer sums per sub-block, folded in another order): 5e-6 of max |y|."""
    if mode == 0:
        assert np.abs(a - b).max() <= 5e-6 * np.abs(b).max(), what
    else:
        assert np.array_equal(a, b), what


def check(y, ref, tol, what):
    from oracle.oracle import rel_err
    e = rel_err(y, ref)
    say("  %s rel err %.3g" % (what, e))
    assert e <= tol, (what, e)


@pytest.mark.parametrize("kqt,fmt,H", FORMATS)
def test_gpu_act8_gemv(a8_rt, orc, lib, act8, kqt, fmt, H):
    """rt_test_matmul (fp32 host x) and lw_matmul_dev (fp16 and fp32 device x) at m = 1 against the oracle's int8
    GEMV; m = 3 and m = 8 (one pass over the weights, the matrix-core kernel by default, the ring kernel in mode 7):
    every token against the oracle and against its own m = 1 call; m = 12 (beyond the int8 range) keeps fp32
    activations on the prefill path (within 2e-5 of fp64)."""
    import torch
    rc, rp, mats = a8_rt
    rng = np.random.default_rng(kqt)
    for nm in (fmt, fmt + "_small"):
        mat = mats[nm]
        N, K = mat[2], mat[3]
        x = rng.standard_normal((1, K)).astype(np.float32)
        y8, y64 = y_act8(orc, mat, x)
        say("act8", nm)
        Y = rc.test_matmul(nm, x)
        check(Y, y8, TOL_ACT8, nm + " act8 fp32 host")
        check(Y, y64, TOL_QUANT, nm + " act8 vs fp32-x fp64")
        # device fp32 x: the same quantization, so the same bits
        Yd = torch.zeros(1, N, device="cuda")
        rc.matmul_dev(nm, torch.from_numpy(x).cuda(), Yd, x_f16=False)
        # device fp16 x, quantized from the fp16 values
        x16 = torch.from_numpy(x).half()
        Yh = torch.zeros(1, N, device="cuda")
        rc.matmul_dev(nm, x16.cuda(), Yh, x_f16=True)
        torch.cuda.synchronize()
        assert np.array_equal(Yd.cpu().numpy(), Y), nm
        check(rp.test_matmul(nm, x), y8, TOL_ACT8, nm + " act8 packed twin")
        y8h, _ = y_act8(orc, mat, x16.float().numpy())
        check(Yh.cpu().numpy(), y8h, TOL_ACT8, nm + " act8 fp16 device")
        for m in (3, 8):
            Xm = rng.standard_normal((m, K)).astype(np.float32)
            y8_m, _ = y_act8(orc, mat, Xm)
            ones = [rc.test_matmul(nm, Xm[j:j + 1])[0] for j in range(m)]
            for mode in (0, 7):
                assert lib.lw_set_kernel_mode(mode) == 0
                Ym = rc.test_matmul(nm, Xm)
                check(Ym, y8_m, TOL_ACT8, nm + " act8 m=%d mode %d" % (m, mode))
                for j in range(m):
                    same_token(Ym[j], ones[j], mode, (nm, m, mode, j))
            lib.lw_set_kernel_mode(0)
        X12 = rng.standard_normal((12, K)).astype(np.float32)
        _, y64_12 = y_act8(orc, mat, X12)
        check(rc.test_matmul(nm, X12), y64_12, 2e-5, nm + " m=12 stays fp32 (prefill path)")


def group(rt, names, xs, m=1):
    """lw_group_matmul_dev over `names` with fp16 x [m][K] per matrix; y [m][N] per matrix, as numpy."""
    import torch
    ys = [torch.zeros(m, rt.info(nm)["N"], device="cuda") for nm in names]
    n = len(names)
    rc = rt.lib.lw_group_matmul_dev(rt.h, n, (ctypes.c_char_p * n)(*[nm.encode() for nm in names]),
                                    (ctypes.c_void_p * n)(*[x.data_ptr() for x in xs]), m,
                                    (ctypes.c_void_p * n)(*[y.data_ptr() for y in ys]), None)
    assert rc == 0, rt.lib.lw_last_error()
    torch.cuda.synchronize()
    return [y.cpu().numpy() for y in ys]


def test_gpu_act8_kernels_same_bits(a8_rt, orc, lib, act8):
    """One grouped m = 1 call over matrices of every size (one shared x, quantized once, and distinct ones): the
    default (the whole-tile kernel for m = 1, mode 0), the ring kernels (modes 5, 7), the low-latency kernel (mode 4),
    the whole-tile kernel with one pass per token (mode 6) and the packed twin give the
    same bits, within
    tolerance of the oracle."""
    import torch
    rc, rp, mats = a8_rt
    for kqt, fmt, H in FORMATS:
        names = [fmt, fmt + "_small", fmt, fmt + "_small"]
        shared = torch.randn(1, mats[fmt][3]).half().cuda()
        xs = [shared, torch.randn(1, 512).half().cuda(), shared, torch.randn(1, 512).half().cuda()]
        runs = {}
        for mode in (0, 4, 5, 6, 7, 9):
            assert lib.lw_set_kernel_mode(mode) == 0
            runs[mode] = group(rc, names, xs)
        lib.lw_set_kernel_mode(0)
        runs["packed"] = group(rp, names, xs)
        say("act8 kernels same bits", fmt)
        for k in (0, 4, 5, 6, 7, 9, "packed"):
            for nm, x, y in zip(names, xs, runs[k]):
                y8, _ = y_act8(orc, mats[nm], x.float().cpu().numpy())
                check(y, y8, TOL_ACT8, "%s act8 grouped (%s)" % (nm, k))
        for k in (4, 5, 6, 7, 9, "packed"):
            for a, b in zip(runs[0], runs[k]):
                assert np.array_equal(a, b), (fmt, k)
        # m = 5 in one pass (modes 0, 4, 5, 7) or one pass per token (modes 6 and 9, packed): every token the bits of
        # its own m = 1 call (mode 0, the matrix-core kernel: within 5e-6 of max |y|), and within tolerance of the oracle
        x5 = [torch.randn(5, mats[nm][3]).half().cuda() for nm in names]
        ones = [group(rc, names, [x[j:j + 1].contiguous() for x in x5]) for j in range(5)]
        say("act8 m=5 grouped", fmt)
        for mode in (0, 4, 5, 6, 7, 9):
            assert lib.lw_set_kernel_mode(mode) == 0
            y5 = group(rc, names, x5, 5)
            for i in range(len(names)):
                for j in range(5):
                    same_token(y5[i][j], ones[j][i][0], mode, (fmt, mode, i, j))
            if mode == 0:
                for nm, x, y in zip(names, x5, y5):
                    y8, _ = y_act8(orc, mats[nm], x.float().cpu().numpy())
                    check(y, y8, TOL_ACT8, "%s act8 m=5 matrix cores" % nm)
        lib.lw_set_kernel_mode(0)
        y5 = group(rp, names, x5, 5)
        for i in range(len(names)):
            for j in range(5):
                assert np.array_equal(y5[i][j], ones[j][i][0]), (fmt, "packed", i, j)


def test_gpu_act8_exception_tiles(gpu, tmp_path, orc, lib, act8):
    """Matrices with exception tiles (32-row schedules decoded in place or by the one-wave pass; tiles without a
    ring schedule by the low-latency kernel; every tile by the whole-tile kernel): modes 0, 3-7 the same bits, within
    tolerance of the oracle."""
    import torch
    from lazyweights_amd import Runtime
    from lazyweights_amd.bundle import Writer
    from test_layout import mild_skew_codes, skewed_tile_codes
    w = Writer(str(tmp_path))
    cases = {"mskew": mild_skew_codes(), "skew": skewed_tile_codes()}
    for nm, (codes, side) in cases.items():
        w.add_kquant(nm, 2, codes, side)
    w.close()
    with Runtime(tmp_path) as rt:
        x = torch.randn(1, 8192).half().cuda()
        for nm, (codes, side) in cases.items():
            runs = {}
            for mode in (0, 3, 4, 5, 6, 7):
                assert lib.lw_set_kernel_mode(mode) == 0
                runs[mode] = group(rt, [nm], [x])[0]
            lib.lw_set_kernel_mode(0)
            say("act8 exception tiles", nm)
            for mode in (3, 4, 5, 6, 7):
                assert np.array_equal(runs[0], runs[mode]), (nm, mode)
            q, d, s = orc.quant_x8(x.float().cpu().numpy())
            check(runs[0], orc.gemv_act8_f64(2, codes, side, q, d, s), TOL_ACT8, nm + " act8")
            # 4 tokens in one pass (modes 0, 3-5, 7; mode 6 one pass per token): the bits of m = 1 calls (mode 0,
            # the matrix-core kernel: within 5e-6 of max |y|)
            x4 = torch.randn(4, 8192).half().cuda()
            ones = [group(rt, [nm], [x4[j:j + 1].contiguous()])[0][0] for j in range(4)]
            q, d, s = orc.quant_x8(x4.float().cpu().numpy())
            y4ref = orc.gemv_act8_f64(2, codes, side, q, d, s)
            for mode in (0, 3, 4, 5, 6, 7):
                assert lib.lw_set_kernel_mode(mode) == 0
                y4 = group(rt, [nm], [x4], 4)[0]
                for j in range(4):
                    same_token(y4[j], ones[j], mode, (nm, mode, j))
                check(y4, y4ref, TOL_ACT8, nm + " act8 m=4 mode %d" % mode)
            lib.lw_set_kernel_mode(0)


def test_gpu_act8_rejects_block_kernel_modes(a8_rt, lib, act8):
    import torch
    rc, rp, mats = a8_rt
    x = torch.randn(1, 512).half().cuda()
    y = torch.zeros(1, 64, device="cuda")
    for mode in (1, 2):
        assert lib.lw_set_kernel_mode(mode) == 0
        with pytest.raises(RuntimeError, match="int8 activations"):
            rc.matmul_dev("Q4_K_small", x, y)
    lib.lw_set_kernel_mode(0)


def test_gpu_act8_full_config2_layer(gpu, tmp_path, orc, lib, act8):
    """Int8 activations on one full config-2 layer (Mistral-shaped Q4_K, H = 2.3) as one grouped m = 1 call, the
    bench's launch shape: every matrix within 2e-5 of the oracle's int8 GEMV, and q / k / v sharing one x (quantized
    once) equal to the same matrices called with copies of it; the same layer at m = 5 (the verify shape, the
    matrix-core kernel) within 2e-5 of the oracle for every token."""
    import torch
    from lazyweights_amd import Runtime, bundle
    from lazyweights_amd.configs import config2_layer
    mats = config2_layer(0)
    bundle.write_synthetic_bundle(str(tmp_path), mats, threads=16)
    with Runtime(tmp_path) as rt:
        names = [m[0] for m in mats]
        shared = torch.randn(1, 4096).half().cuda()
        xs = [shared if m[0].endswith((".q", ".k", ".v")) else torch.randn(1, m[3]).half().cuda() for m in mats]
        say("act8 config 2 layer grouped")
        ys = group(rt, names, xs)
        copies = group(rt, names[:3], [shared.clone() for _ in range(3)])
        for a, b in zip(ys[:3], copies):
            assert np.array_equal(a, b)
        x5 = [torch.randn(5, m[3]).half().cuda() for m in mats]
        say("act8 config 2 layer grouped, m = 5")
        y5 = group(rt, names, x5, 5)
        for mat, x, y, xx, yy in zip(mats, xs, ys, x5, y5):
            name, kqt, N, K, H, seed = mat
            codes, side = bundle.synth_matrix(kqt, N, K, H, seed, threads=16)
            q, d, s = orc.quant_x8(x.float().cpu().numpy())
            check(y, orc.gemv_act8_f64(kqt, codes, side, q, d, s), TOL_ACT8, name + " act8 full layer")
            q, d, s = orc.quant_x8(xx.float().cpu().numpy())
            check(yy, orc.gemv_act8_f64(kqt, codes, side, q, d, s), TOL_ACT8, name + " act8 full layer m=5")
            del codes, side
