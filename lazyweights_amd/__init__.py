"""lazyweights_amd: MI355X-native decode-on-demand weight path of LazyWeights.

Coded K-quant matrices (lane-interleaved Huffman bundles) are decoded on gfx950 and fused into the batch-1 GEMV and
the skinny verify GEMM, behind the reference runtime's C-ABI (include/lazyweights_amd.h).
"""
from ._lib import LIB_PATH, last_error, load_library  # noqa: F401
from .runtime import Runtime  # noqa: F401
