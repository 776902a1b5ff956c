"""lw_matmul_dev_noalloc: the fused matmul with every scratch buffer in the library's static per-device array.

Through the C-ABI, against lw_matmul_dev (same kernels, so the same bits) on consecutive calls, the second with a
smaller input, for fp16 and fp32 activations, and against the fp64 oracle; a call whose partials exceed the 16 MiB
array is refused with an error before any launch.
"""
import ctypes
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def na_rt(gpu, tmp_path_factory, lib):
    from lazyweights_amd import Runtime, bundle
    d = tmp_path_factory.mktemp("noalloc")
    mats = [("big", 1, 14336, 4096, 2.3, 501), ("mid", 3, 1024, 4096, 4.3, 502), ("small", 2, 64, 512, 3.4, 503),
            ("huge", 1, 8192, 16384, 2.3, 504)]
    bundle.write_synthetic_bundle(str(d), mats, threads=16)
    rt = Runtime(d)
    yield rt, {m[0]: m for m in mats}
    rt.close()


def call(rt, fn, name, X, Y, f16):
    import torch
    rc = fn(rt.h, name.encode(), ctypes.c_void_p(X.data_ptr()), 1 if f16 else 0, X.shape[0],
            ctypes.c_void_p(Y.data_ptr()), Y.stride(0), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    return rc


def test_noalloc_matches_allocating_entry_point(na_rt, orc, lib):
    import torch
    from lazyweights_amd import bundle
    rt, mats = na_rt
    cases = [("big", 4, True), ("small", 1, True), ("mid", 3, False), ("small", 2, False), ("big", 1, True)]
    for name, m, f16 in cases:
        _, kqt, N, K, H, seed = mats[name]
        g = torch.Generator().manual_seed(seed + m)
        X = torch.randn(m, K, generator=g)
        X = (X.half() if f16 else X).cuda()
        Ya = torch.full((m, N), float("nan"), device="cuda")
        Yb = torch.full((m, N), float("nan"), device="cuda")
        say("noalloc", name, "m", m, "fp16" if f16 else "fp32")
        assert call(rt, lib.lw_matmul_dev, name, X, Ya, f16) == 0, lib.lw_last_error()
        assert call(rt, lib.lw_matmul_dev_noalloc, name, X, Yb, f16) == 0, lib.lw_last_error()
        torch.cuda.synchronize()
        assert torch.equal(Ya, Yb), name
        codes, side = bundle.synth_matrix(kqt, N, K, H, seed, threads=16)
        y64 = orc.gemv_f64(orc.dequant(kqt, codes, side), X.float().cpu().double().numpy())
        e = orc.rel_err(Yb.cpu().numpy(), y64)
        say("  rel err %.3g" % e)
        assert e <= 2e-5


def test_noalloc_refuses_oversized_calls(na_rt, lib):
    """8192 x 16384 with 16 fp16 tokens needs 32 x 16 x 8192 x 4 B = 16.8 MB of partials: refused, nothing launched;
    the same matrix with 8 tokens fits and still runs."""
    import torch
    rt, mats = na_rt
    X = torch.randn(16, 16384).half().cuda()
    Y = torch.zeros(16, 8192, device="cuda")
    say("noalloc oversized")
    assert call(rt, lib.lw_matmul_dev_noalloc, "huge", X, Y, True) == -1
    assert "too small" in lib.lw_last_error().decode()
    assert call(rt, lib.lw_matmul_dev_noalloc, "huge", X[:8], Y[:8], True) == 0, lib.lw_last_error()
    Ya = torch.zeros(8, 8192, device="cuda")
    assert call(rt, lib.lw_matmul_dev, "huge", X[:8], Ya, True) == 0
    torch.cuda.synchronize()
    assert torch.equal(Y[:8], Ya)
    assert call(rt, lib.lw_matmul_dev_noalloc, "huge", X[:1].float(), Y[:1], False) == 0
    assert call(rt, lib.lw_matmul_dev_noalloc, "huge", X[:9].float(), Y[:9], False) == -1  # fp32: m <= 8
