"""The synthetic workloads of the benchmark contract (five configurations).

Each matrix is (name, kqt, N, K, entropy bits per code, seed). Codes follow a two-sided geometric distribution
P(q) ∝ rho^|q - centre| (centre 8 for 4-bit formats, 16 for Q5_K, 32 for Q6_K), rho solved for the entropy;
d / dmin ~ U(0.005, 0.02) rounded to fp16, 6-bit sub-scales and mins uniform (lw_codec.cpp synth_matrix).
"""
Q4_K, Q5_K, Q6_K, IQ4_XS = 1, 2, 3, 4

# 0: CPU-runnable single matrix
CONFIG0 = [("m0", Q4_K, 4096, 4096, 2.6, 1000)]

# 1: Phi-3-mini-shaped layer (one table per matrix)
CONFIG1 = [("qkv", Q4_K, 9216, 3072, 2.6, 1100), ("o", Q4_K, 3072, 3072, 2.6, 1101),
           ("gate_up", Q4_K, 16384, 3072, 2.6, 1102), ("down", Q4_K, 3072, 8192, 2.6, 1103)]

# 2: Mistral-7B-shaped layer, entropy narrowed to 2.3 bits (the headline roofline configuration)
MISTRAL = [("q", 4096, 4096), ("k", 1024, 4096), ("v", 1024, 4096), ("o", 4096, 4096),
           ("gate", 14336, 4096), ("up", 14336, 4096), ("down", 4096, 14336)]


def config2_layer(layer, entropy=2.3):
    return [("l%d.%s" % (layer, n), Q4_K, N, K, entropy, 2000 + 16 * layer + i)
            for i, (n, N, K) in enumerate(MISTRAL)]


# 3: mixed formats: Q6_K down (entropy 4.3), IQ4_XS gate / up (entropy 2.6, geometric about grid index 8)
CONFIG3 = [("down", Q6_K, 4096, 14336, 4.3, 3000), ("gate", IQ4_XS, 14336, 4096, 2.6, 3001),
           ("up", IQ4_XS, 14336, 4096, 2.6, 3002)]

# 4: verify GEMM (m = 5) on Mistral shapes: Q4_K as config 2 and Q5_K (entropy 3.4)
CONFIG4 = [("q4.%s" % n, Q4_K, N, K, 2.3, 4000 + i) for i, (n, N, K) in enumerate(MISTRAL)] + \
          [("q5.%s" % n, Q5_K, N, K, 3.4, 4100 + i) for i, (n, N, K) in enumerate(MISTRAL)]


def scaled(mats, rows_div=1, cols_div=1):
    """Same formats / distributions at reduced shape (for CPU-side parity at oracle-friendly sizes)."""
    out = []
    for name, kqt, N, K, H, seed in mats:
        cw = 512 if kqt in (Q4_K, IQ4_XS) else 256
        n = max(64, (N // rows_div) // 64 * 64)
        k = max(cw, (K // cols_div) // cw * cw)
        out.append((name, kqt, n, k, H, seed))
    return out
