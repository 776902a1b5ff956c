"""Python mirror of the runtime's C-ABI: a handle on an opened bundle and its reference-named entry points.

Mirrors how the reference drives its runtime from Python (scripts/a2_act8_ppl.py:56-77: ctypes, rt_open with the
same arguments) and its CLI self-checks (kernels/llmrt.cu:2842-2885: rt_test_decode vs rt_test_cpu_decode,
rt_test_matmul paths). Errors raise RuntimeError carrying lw_last_error().
"""
import ctypes

import numpy as np

from ._lib import last_error, load_library


class Runtime:
    """rt_open(dir, max_ctx, max_batch, budget_mb, floor_mb, verbose) ... rt_close."""

    def __init__(self, bundle_dir, max_ctx=512, max_batch=8, budget_mb=-1, floor_mb=0, verbose=0):
        self.lib = load_library()
        self.h = self.lib.rt_open(str(bundle_dir).encode(), max_ctx, max_batch, budget_mb, floor_mb, verbose)
        if not self.h:
            raise RuntimeError("rt_open failed: " + last_error())
        self.dir = str(bundle_dir)

    def close(self):
        if self.h:
            self.lib.rt_close(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def info(self, name):
        out = np.zeros(9, np.int64)
        if self.lib.lw_tensor_info(self.h, name.encode(), out.ctypes.data) != 0:
            raise KeyError(name)
        keys = ("N", "K", "kqt", "symbits", "blob_bytes", "side_bytes", "device_bytes", "tiles", "resident")
        return dict(zip(keys, (int(v) for v in out)))

    def test_matmul(self, name, X, path=0):
        """Y[m, N] = X[m, K] @ dequant(W)^T (fp32 host arrays)."""
        X = np.ascontiguousarray(X, np.float32)
        if X.ndim == 1:
            X = X[None]
        inf = self.info(name)
        Y = np.zeros((X.shape[0], inf["N"]), np.float32)
        if X.shape[1] != inf["K"]:
            raise ValueError("X has %d columns, %s has K = %d" % (X.shape[1], name, inf["K"]))
        rc = self.lib.rt_test_matmul(self.h, name.encode(), X.ctypes.data, X.shape[0], Y.ctypes.data, path)
        if rc != 0:
            raise RuntimeError("rt_test_matmul(%s): %s" % (name, last_error()))
        return Y

    def test_decode(self, name):
        """GPU decode to codes [N, K] (one byte per weight)."""
        inf = self.info(name)
        out = np.zeros((inf["N"], inf["K"]), np.uint8)
        if self.lib.rt_test_decode(self.h, name.encode(), out.ctypes.data) != 0:
            raise RuntimeError("rt_test_decode(%s): %s" % (name, last_error()))
        return out

    def test_cpu_decode(self, name, threads=4):
        """CPU decode of the raw blob to symbols [N, KS]."""
        inf = self.info(name)
        ks = inf["K"] // 2 if inf["symbits"] == 4 else inf["K"]
        out = np.zeros((inf["N"], ks), np.uint8)
        if self.lib.rt_test_cpu_decode(self.h, name.encode(), threads, out.ctypes.data) != 0:
            raise RuntimeError("rt_test_cpu_decode(%s): %s" % (name, last_error()))
        return out

    def gpu_decode_all(self, reps=5):
        return self.lib.rt_gpu_decode_all(self.h, reps)

    def cpu_decode_all(self, threads=4):
        n = ctypes.c_longlong(0)
        s = self.lib.rt_cpu_decode_all(self.h, threads, ctypes.byref(n))
        return s, n.value

    def stat(self, key):
        return self.lib.rt_stat(self.h, key.encode())

    def matmul_dev(self, name, X, Y, x_f16=True, stream=None):
        """Device-pointer path on torch tensors (X [m, K] fp16 or fp32 on the GPU, Y [m, N] fp32)."""
        m = X.shape[0]
        st = ctypes.c_void_p(stream) if stream else None
        rc = self.lib.lw_matmul_dev(self.h, name.encode(), X.data_ptr(), 1 if x_f16 else 0, m, Y.data_ptr(),
                                    Y.stride(0), st)
        if rc != 0:
            raise RuntimeError("lw_matmul_dev(%s): %s" % (name, last_error()))
