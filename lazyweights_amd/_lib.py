"""ctypes binding of liblazyweights_amd.so (the C-ABI in include/lazyweights_amd.h).

Argument types follow the reference's own ctypes binding of its runtime (scripts/a2_act8_ppl.py:56-62) for the
rt_* entry points. There is no fallback: if the shared library is missing, loading raises.
"""
import ctypes
import os

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG, "liblazyweights_amd.so")

_c = ctypes
_vp, _cp, _i, _ll, _d, _u64 = _c.c_void_p, _c.c_char_p, _c.c_int, _c.c_longlong, _c.c_double, _c.c_uint64

SIGNATURES = {
    # reference-compatible
    "rt_open": (_vp, [_cp, _i, _i, _ll, _i, _i]),
    "rt_close": (None, [_vp]),
    "rt_test_matmul": (_i, [_vp, _cp, _vp, _i, _vp, _i]),
    "rt_test_decode": (_i, [_vp, _cp, _vp]),
    "rt_gpu_decode_all": (_d, [_vp, _i]),
    "rt_test_cpu_decode": (_i, [_vp, _cp, _i, _vp]),
    "rt_cpu_decode_all": (_d, [_vp, _i, _c.POINTER(_ll)]),
    "rt_stat": (_d, [_vp, _cp]),
    "rt_forward": (_i, [_vp, _vp, _i, _vp, _i]),
    "rt_reset": (None, [_vp]),
    "rt_set_window": (None, [_vp, _i]),
    "rt_set_pos": (None, [_vp, _i]),
    "rt_pos": (_i, [_vp]),
    "rt_vocab": (_i, [_vp]),
    # extensions
    "lw_last_error": (_cp, []),
    "lw_tensor_info": (_i, [_vp, _cp, _vp]),
    "lw_matmul_dev": (_i, [_vp, _cp, _vp, _i, _i, _vp, _i, _vp]),
    "lw_matmul_dev_noalloc": (_i, [_vp, _cp, _vp, _i, _i, _vp, _i, _vp]),
    "lw_group_matmul_dev": (_i, [_vp, _i, _vp, _vp, _i, _vp, _vp]),
    "lw_bench_groups": (_i, [_vp, _i, _vp, _vp, _vp, _i, _vp, _i, _i, _vp]),
    "lw_stream_read_gbps": (_d, [_ll, _i]),
    "lw_synth_matrix": (_i, [_i, _i, _i, _d, _u64, _vp, _vp, _i]),
    "lw_form_symbols": (_i, [_i, _vp, _i, _i, _vp]),
    "lw_encode": (_ll, [_vp, _i, _i, _vp, _ll, _c.POINTER(_u64)]),
    "lw_write_bundle": (_i, [_cp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _i]),
    "lw_bundle_create": (_vp, [_cp]),
    "lw_bundle_cfg": (_i, [_vp, _cp, _cp]),
    "lw_bundle_add": (_i, [_vp, _cp, _cp, _ll, _ll, _d, _i, _vp, _ll]),
    "lw_bundle_finish": (_i, [_vp]),
    "lw_huffman_lengths": (_i, [_vp, _i, _i, _vp]),
    "lw_build_layout": (_ll, [_vp, _ll, _i, _i, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _ll]),
    "lw_canon_table": (_i, [_i, _vp, _vp]),
    "lw_set_kernel_mode": (_i, [_i]),
    "lw_set_prefill_gemm": (_i, [_i]),
    "lw_set_act8": (_i, [_i]),
    "lw_test_quant_x8": (_i, [_vp, _i, _i, _i, _vp, _vp, _vp]),
}

_LIB = None


def load_library(path=None):
    """Loads the shared library once and declares every exported signature."""
    global _LIB
    if _LIB is not None and path is None:
        return _LIB
    p = path or os.environ.get("LAZYWEIGHTS_AMD_LIB", LIB_PATH)
    try:  # one HIP runtime per process: torch's copy (same soname) is loaded first when torch is present
        import torch  # noqa: F401
    except ImportError:
        pass
    if not os.path.exists(p):
        raise RuntimeError("lazyweights_amd: %s is not built (run __graft_entry__.build() or "
                           "python -m lazyweights_amd.build)" % p)
    lib = _c.CDLL(p)
    for name, (res, args) in SIGNATURES.items():
        f = getattr(lib, name)
        f.restype = res
        f.argtypes = args
    if path is None:
        _LIB = lib
    return lib


def last_error():
    return (load_library().lw_last_error() or b"").decode(errors="replace")
