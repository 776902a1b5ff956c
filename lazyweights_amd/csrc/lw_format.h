// Shared constants of the LazyWeights coded-weight format (host and device).
//
// Bundle blob (reference lazyweights/bundle.py:14-21): u16 lut[2048] (entry = sym | len << 8, indexed by the next
// 11 stream bits LSB-first), u32 lane_start[T][32] (absolute bit offsets), u32 payload[W + 2].
// Tiles are 64 rows x 256 symbols; lane l of a tile codes row l then row l + 32, 256 symbols each.
// K-quant side bytes (reference scripts/a2_kq_bundle.py:1-14, kernels/llmrt.cu:113-119): per 256-weight
// super-block, SB = 16 (Q4_K, Q5_K), 18 (Q6_K), 8 (IQ4_XS) bytes.
#pragma once
#include <cstdint>

#if !defined(__HIPCC__) && !defined(__host__)
#define __host__
#define __device__
#endif

namespace lw {

constexpr int TN = 64;             // tile rows
constexpr int TK = 256;            // tile symbols per row
constexpr int LMAX = 11;           // maximum code length
constexpr int LUTN = 1 << LMAX;    // bundle LUT entries
constexpr int LANES = 32;          // lanes per tile
constexpr int LANE_SYMS = 2 * TK;  // symbols per lane (two rows)
constexpr int SPLITS = 16;         // chain starts per lane stream, every 32 symbols (the low-latency kernel uses
                                   // every second one, the whole-tile kernel all)

// K-quant type ids, numbered as the reference's Tensor::kqt (kernels/llmrt.cu:113-116)
enum : int { KQ_NONE = 0, KQ_Q4_K = 1, KQ_Q5_K = 2, KQ_Q6_K = 3, KQ_IQ4_XS = 4 };

__host__ __device__ constexpr int kq_sbytes(int kqt) { return kqt == KQ_Q6_K ? 18 : kqt == KQ_IQ4_XS ? 8 : 16; }
// weights per sub-block (one scale each)
__host__ __device__ constexpr int kq_gw(int kqt) { return kqt == KQ_Q6_K ? 16 : 32; }
// symbol layout: 4 = two 4-bit codes per symbol (enc huf4p), 8 = one code per symbol (enc huf8)
__host__ __device__ constexpr int kq_symbits(int kqt) { return (kqt == KQ_Q4_K || kqt == KQ_IQ4_XS) ? 4 : 8; }
// code range of the format
__host__ __device__ constexpr int kq_ncodes(int kqt) {
  return kqt == KQ_Q5_K ? 32 : kqt == KQ_Q6_K ? 64 : 16;
}

// Device order of the side records (load-time permutation of the bundle's [N][K/256][SB]): tile-major, so that the
// 64 rows of one tile and one of its super-blocks are 64 consecutive records and a wave reads them as whole cache
// lines once. Record of row n, super-block b (nsb = super-blocks per tile column: 2 for 4-bit symbols, 1 for 8-bit;
// KT = tile columns): ((tile * nsb + b % nsb) * 64 + n % 64), tile = (n / 64) * KT + b / nsb.
__host__ __device__ inline uint64_t side_record(int n, int b, int KT, int nsb) {
  const uint64_t tile = (uint64_t)(n / TN) * (uint64_t)KT + (uint64_t)(b / nsb);
  return (tile * (uint64_t)nsb + (uint64_t)(b % nsb)) * TN + (uint64_t)(n % TN);
}

// IQ4_XS non-linear grid (reference kernels/llmrt.cu:117, scripts/a2_kq_bundle.py:42)
constexpr int8_t IQ4_GRID[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};

}  // namespace lw
