// gfx950 kernels of the decode-on-demand weight path.
//
// Fused Huffman decode + K-quant dequant + GEMV / skinny GEMM (reference kernels/llmrt.cu:892-1033, k_gemvm_kq),
// re-designed for CDNA4:
//   * one wave64 decodes one 64 x 256-symbol tile; each lane's stream is split at its second row (the per-lane
//     offset `mid` built at load time), so lane L of the wave runs the chain of tile row L: 64 independent chains
//     per tile instead of 32, which doubles the decode parallelism of a layer;
//   * the wave stages its tile's interleaved word rows (word i of lane l at 32 i + l) in LDS with coalesced 16-byte
//     loads, and every symbol reads its 64-bit window with one ds_read2 (rows r and r + 1 of the lane's column);
//   * the 2048-entry table is expanded per block into LDS as {fp16 pair of grid values, code length}: one 8-byte
//     LDS read yields the two dequantized grid values f(q) of a pair symbol, ready for v_dot2_f32_f16;
//   * activations are fp16 pairs staged in LDS (broadcast reads); products are exact in fp32 and accumulate in
//     fp32 per sub-block; the sub-block scale s and offset o (and the per-sub-block sums of x for o) are applied
//     once per sub-block;
//   * partial sums per tile column go to P[tc][j][n] and are summed in tile-column order by k_reduce
//     (deterministic, as the reference's k_sum_kt, llmrt.cu:1171-1180).
#include <hip/hip_runtime.h>

#include "lw_format.h"
#include "lw_kernels.h"

namespace lw {

typedef _Float16 h2v __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(h2v, a), __builtin_bit_cast(h2v, b), c, false);
}
__device__ __forceinline__ float h2f(uint32_t bits16) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(bits16 & 0xFFFFu));
}
__device__ __forceinline__ uint32_t f2h(float v) { return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v); }

// grid value f(q) of a code (reference llmrt.cu:151-154): Q4_K/Q5_K q, Q6_K q - 32, IQ4_XS kv[q]
template <int KQ>
__device__ __forceinline__ float grid_value(uint32_t q) {
  if (KQ == KQ_IQ4_XS) return (float)IQ4_GRID[q & 15];
  if (KQ == KQ_Q6_K) return (float)q - 32.f;
  return (float)q;
}

// side bytes of one super-block as words (byte i at bits 8 (i & 3) of w[i / 4]); Q6_K records are 2-byte aligned
template <int KQ>
__device__ __forceinline__ void side_load(const uint8_t* p, uint32_t* w) {
  if (KQ == KQ_Q6_K) {
    const uint16_t* h = reinterpret_cast<const uint16_t*>(p);
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = (uint32_t)h[2 * i] | (uint32_t)h[2 * i + 1] << 16;
    w[4] = h[8];
  } else if (KQ == KQ_IQ4_XS) {
    const uint2 v = *reinterpret_cast<const uint2*>(p);
    w[0] = v.x;
    w[1] = v.y;
  } else {
    const uint4 v = *reinterpret_cast<const uint4*>(p);
    w[0] = v.x;
    w[1] = v.y;
    w[2] = v.z;
    w[3] = v.w;
  }
}
__device__ __forceinline__ uint32_t side_byte(const uint32_t* w, int i) { return (w[i >> 2] >> (8 * (i & 3))) & 255u; }

// (s, o) of sub-block j (reference llmrt.cu:125-149; llama.cpp get_scale_min_k4 for Q4_K/Q5_K)
template <int KQ>
__device__ __forceinline__ void side_scale(const uint32_t* w, int j, float& s, float& o) {
  if (KQ == KQ_Q4_K || KQ == KQ_Q5_K) {
    uint32_t sc, m;
    if (j < 4) {
      sc = side_byte(w, 4 + j) & 63;
      m = side_byte(w, 8 + j) & 63;
    } else {
      sc = (side_byte(w, 8 + j) & 15) | ((side_byte(w, j) >> 6) << 4);
      m = (side_byte(w, 8 + j) >> 4) | ((side_byte(w, 4 + j) >> 6) << 4);
    }
    s = h2f(w[0]) * (float)sc;
    o = h2f(w[0] >> 16) * (float)m;
  } else if (KQ == KQ_Q6_K) {
    s = h2f(w[4]) * (float)(int8_t)side_byte(w, j);
    o = 0.f;
  } else {
    const uint32_t ls = ((side_byte(w, 4 + j / 2) >> (4 * (j & 1))) & 15) | (((w[0] >> (16 + 2 * j)) & 3) << 4);
    s = h2f(w[0]) * (float)((int)ls - 32);
    o = 0.f;
  }
}

// Next symbol of a chain whose lane words are staged in LDS at tw[32 i] (tw = tile base + lane). pos = bit
// position in the lane stream. Returns the table entry {value, length}.
__device__ __forceinline__ uint2 next_sym(const uint32_t* tw, uint32_t& pos, const uint2* lut8) {
  const uint32_t r = pos >> 5;
  const uint32_t lo = tw[32 * r], hi = tw[32 * r + 32];
  const uint32_t win = __builtin_amdgcn_alignbit(hi, lo, pos);
  const uint2 e = lut8[win & (LUTN - 1)];
  pos += e.y;
  return e;
}

// Stage rows [0, rows] (one extra row for the window's read-ahead) of tile t into the wave's LDS region.
__device__ __forceinline__ void stage_tile(const DevMat& M, int t, uint32_t* tw, int lane64) {
  const int R = (int)M.rows[t] + 1;
  const uint4* src = reinterpret_cast<const uint4*>(M.words + M.tbase[t]);
  uint4* dst = reinterpret_cast<uint4*>(tw);
  for (int i = lane64; i < 8 * R; i += 64) dst[i] = src[i];
}

// ── fused decode + dequant + GEMV / GEMM (m <= 16 pseudo-tokens) ─────────────────────────────────────────
// block = 4 waves = 4 tile rows [4 b_r, 4 b_r + 4) of one tile column tc; lane L of wave w: tile row 4 b_r + w,
// matrix row 64 tr + L (lanes 32..63 start at their lane's `mid` offset).
template <int KQ, int MT>
__global__ void __launch_bounds__(256) k_fused(DevMat M, const uint32_t* __restrict__ X2, int mt,
                                                float* __restrict__ P) {
  constexpr int SYMB = kq_symbits(KQ);
  constexpr int TW = SYMB == 4 ? 2 * TK : TK;  // weights per tile column
  constexpr int GW = kq_gw(KQ), NG = TW / GW, SB = kq_sbytes(KQ), NPAIR = TW / 2;
  extern __shared__ __align__(16) uint32_t smem[];
  uint2* lut8 = reinterpret_cast<uint2*>(smem);
  uint32_t* xs = smem + 2 * LUTN;                        // [NPAIR][MT] fp16 pairs
  float* xg = reinterpret_cast<float*>(xs + NPAIR * MT);  // [NG][MT]
  uint32_t* tiles = reinterpret_cast<uint32_t*>(xg + NG * MT);
  const int RS = M.max_rows + 1;
  const int KT = M.KT, NT = M.NT, K = M.K, N = M.N;
  const int tc = blockIdx.x % KT, wave = threadIdx.x >> 6;
  const int tr = (blockIdx.x / KT) * 4 + wave;
  const int lane = threadIdx.x & 63, l = lane & 31, half = lane >> 5;
  for (int i = threadIdx.x; i < LUTN; i += 256) {
    const uint32_t e = M.lut[i], sym = e & 255u;
    uint32_t v;
    if (SYMB == 4) v = f2h(grid_value<KQ>(sym & 15u)) | f2h(grid_value<KQ>(sym >> 4)) << 16;
    else v = f2h(grid_value<KQ>(sym));
    lut8[i] = make_uint2(v, e >> 8);
  }
  for (int i = threadIdx.x; i < NPAIR * MT; i += 256) {
    const int j = i / NPAIR, c = i - j * NPAIR;
    xs[c * MT + j] = j < mt ? X2[(size_t)j * (K / 2) + (size_t)tc * NPAIR + c] : 0u;
  }
  const bool active = tr < NT;
  const int t = tr * KT + tc;
  uint32_t* tw = tiles + wave * 32 * RS;
  if (active) stage_tile(M, t, tw, lane);
  __syncthreads();
  for (int i = threadIdx.x; i < NG * MT; i += 256) {
    const int g = i / MT, j = i - g * MT;
    float a = 0.f;
    for (int c = g * (GW / 2); c < (g + 1) * (GW / 2); ++c) {
      const uint32_t v = xs[c * MT + j];
      a += h2f(v) + h2f(v >> 16);
    }
    xg[g * MT + j] = a;
  }
  __syncthreads();
  if (!active) return;
  uint32_t pos = half ? (uint32_t)M.mid[(size_t)t * 32 + l] : 0u;
  const uint32_t* lw = tw + l;
  const int n = tr * TN + half * 32 + l;
  float tot[MT];
#pragma unroll
  for (int j = 0; j < MT; ++j) tot[j] = 0.f;
#pragma unroll 1
  for (int sb = 0; sb < TW / 256; ++sb) {
    uint32_t sw[5];
    side_load<KQ>(M.side + ((size_t)n * (K / 256) + (size_t)tc * (TW / 256) + sb) * SB, sw);
#pragma unroll
    for (int jj = 0; jj < 256 / GW; ++jj) {
      const int g = sb * (256 / GW) + jj;
      float s, o;
      side_scale<KQ>(sw, jj, s, o);
      float acc[MT];
#pragma unroll
      for (int j = 0; j < MT; ++j) acc[j] = 0.f;
      if (SYMB == 4) {
#pragma unroll 4
        for (int c = 0; c < GW / 2; ++c) {
          const uint2 e = next_sym(lw, pos, lut8);
          const uint32_t* xp = xs + (g * (GW / 2) + c) * MT;
#pragma unroll
          for (int j = 0; j < MT; ++j) acc[j] = dot2(e.x, xp[j], acc[j]);
        }
      } else {
#pragma unroll 4
        for (int c = 0; c < GW; c += 2) {
          const uint2 e0 = next_sym(lw, pos, lut8);
          const uint2 e1 = next_sym(lw, pos, lut8);
          const uint32_t w = e0.x | (e1.x << 16);
          const uint32_t* xp = xs + ((g * GW + c) / 2) * MT;
#pragma unroll
          for (int j = 0; j < MT; ++j) acc[j] = dot2(w, xp[j], acc[j]);
        }
      }
#pragma unroll
      for (int j = 0; j < MT; ++j) tot[j] += s * acc[j] - o * xg[g * MT + j];
    }
  }
#pragma unroll
  for (int j = 0; j < MT; ++j)
    if (j < mt) P[((size_t)tc * mt + j) * N + n] = tot[j];
}

static size_t fused_smem(const DevMat& M, int MT) {
  const int TW = M.symbits == 4 ? 2 * TK : TK, GW = kq_gw(M.kqt);
  return (size_t)LUTN * 8 + (size_t)(TW / 2) * MT * 4 + (size_t)(TW / GW) * MT * 4 +
         (size_t)4 * 32 * (M.max_rows + 1) * 4;
}

template <int KQ, int MT>
static hipError_t fused_mt(const DevMat& M, const void* X16, int mt, float* P, hipStream_t s) {
  const size_t smem = fused_smem(M, MT);
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_fused<KQ, MT>),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
  if (e != hipSuccess) return e;
  const int blocks = M.KT * ((M.NT + 3) / 4);
  hipLaunchKernelGGL((k_fused<KQ, MT>), dim3(blocks), dim3(256), smem, s, M,
                     reinterpret_cast<const uint32_t*>(X16), mt, P);
  return hipGetLastError();
}

template <int KQ>
static hipError_t fused_kq(const DevMat& M, const void* X16, int mt, float* P, hipStream_t s) {
  if (mt <= 1) return fused_mt<KQ, 1>(M, X16, mt, P, s);
  if (mt <= 2) return fused_mt<KQ, 2>(M, X16, mt, P, s);
  if (mt <= 4) return fused_mt<KQ, 4>(M, X16, mt, P, s);
  if (mt <= 8) return fused_mt<KQ, 8>(M, X16, mt, P, s);
  return fused_mt<KQ, 16>(M, X16, mt, P, s);
}

hipError_t launch_fused(const DevMat& M, const void* X16, int mt, float* P, hipStream_t s) {
  if (mt < 1 || mt > 16) return hipErrorInvalidValue;
  switch (M.kqt) {
    case KQ_Q4_K: return fused_kq<KQ_Q4_K>(M, X16, mt, P, s);
    case KQ_Q5_K: return fused_kq<KQ_Q5_K>(M, X16, mt, P, s);
    case KQ_Q6_K: return fused_kq<KQ_Q6_K>(M, X16, mt, P, s);
    case KQ_IQ4_XS: return fused_kq<KQ_IQ4_XS>(M, X16, mt, P, s);
    default: return hipErrorInvalidValue;
  }
}

// ── ordered reduction over tile columns ──────────────────────────────────────────────────────────────────
__global__ void k_reduce(const float* __restrict__ P, float* __restrict__ Y, int m, int per, int N, int ldy, int KT) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= m * N) return;
  const int j = i / N, n = i - j * N, mt = m * per;
  float a = 0.f;
  for (int tc = 0; tc < KT; ++tc)
    for (int q = 0; q < per; ++q) a += P[((size_t)tc * mt + j * per + q) * N + n];
  Y[(size_t)j * ldy + n] = a;
}

hipError_t launch_reduce(const float* P, float* Y, int m, int per, int N, int ldy, int KT, hipStream_t s) {
  hipLaunchKernelGGL(k_reduce, dim3((m * N + 255) / 256), dim3(256), 0, s, P, Y, m, per, N, ldy, KT);
  return hipGetLastError();
}

// ── fp32 activations -> fp16 hi / lo pseudo-tokens ──────────────────────────────────────────────────────
__global__ void k_split_x(const float* __restrict__ X, uint16_t* __restrict__ X16, int m, int K) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (size_t)m * K) return;
  const size_t j = i / K, k = i - j * K;
  const float x = X[i];
  const _Float16 hi = (_Float16)x;
  const _Float16 lo = (_Float16)(x - (float)hi);
  X16[(2 * j) * K + k] = __builtin_bit_cast(uint16_t, hi);
  X16[(2 * j + 1) * K + k] = __builtin_bit_cast(uint16_t, lo);
}

hipError_t launch_split_x(const float* X, void* X16, int m, int K, hipStream_t s) {
  const size_t n = (size_t)m * K;
  hipLaunchKernelGGL(k_split_x, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, X,
                     reinterpret_cast<uint16_t*>(X16), m, K);
  return hipGetLastError();
}

// ── decode only: codes [N][K] bytes ──────────────────────────────────────────────────────────────────────
// block = 4 waves = 4 consecutive tiles of [tr0 KT, tr1 KT); output rows relative to tile row tr0.
template <int SYMB>
__global__ void __launch_bounds__(256) k_decode(DevMat M, uint8_t* __restrict__ out, int tr0, int tr1) {
  constexpr int TW = SYMB == 4 ? 2 * TK : TK;
  extern __shared__ __align__(16) uint32_t smem[];
  uint2* lut8 = reinterpret_cast<uint2*>(smem);
  uint32_t* tiles = smem + 2 * LUTN;
  const int RS = M.max_rows + 1, KT = M.KT, K = M.K;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, l = lane & 31, half = lane >> 5;
  for (int i = threadIdx.x; i < LUTN; i += 256) {
    const uint32_t e = M.lut[i];
    lut8[i] = make_uint2(e & 255u, e >> 8);
  }
  const int t = tr0 * KT + blockIdx.x * 4 + wave;
  const bool active = t < tr1 * KT;
  uint32_t* tw = tiles + wave * 32 * RS;
  if (active) stage_tile(M, t, tw, lane);
  __syncthreads();
  if (!active) return;
  const int tr = t / KT, tc = t - tr * KT;
  uint32_t pos = half ? (uint32_t)M.mid[(size_t)t * 32 + l] : 0u;
  const uint32_t* lw = tw + l;
  uint8_t* row = out + (size_t)((tr - tr0) * TN + half * 32 + l) * K + (size_t)tc * TW;
#pragma unroll 1
  for (int c = 0; c < TK; c += 4) {
    const uint32_t s0 = next_sym(lw, pos, lut8).x, s1 = next_sym(lw, pos, lut8).x;
    const uint32_t s2 = next_sym(lw, pos, lut8).x, s3 = next_sym(lw, pos, lut8).x;
    if (SYMB == 8) {
      *reinterpret_cast<uint32_t*>(row + c) = s0 | s1 << 8 | s2 << 16 | s3 << 24;
    } else {
      const uint32_t a = (s0 & 15u) | (s0 >> 4) << 8 | (s1 & 15u) << 16 | (s1 >> 4) << 24;
      const uint32_t b = (s2 & 15u) | (s2 >> 4) << 8 | (s3 & 15u) << 16 | (s3 >> 4) << 24;
      *reinterpret_cast<uint2*>(row + 2 * c) = make_uint2(a, b);
    }
  }
}

hipError_t launch_decode(const DevMat& M, uint8_t* out, int tr0, int tr1, hipStream_t s) {
  const size_t smem = (size_t)LUTN * 8 + (size_t)4 * 32 * (M.max_rows + 1) * 4;
  const int tiles = (tr1 - tr0) * M.KT, blocks = (tiles + 3) / 4;
  if (blocks <= 0) return hipSuccess;
  hipError_t e;
  if (M.symbits == 4) {
    e = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_decode<4>), hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)smem);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_decode<4>, dim3(blocks), dim3(256), smem, s, M, out, tr0, tr1);
  } else {
    e = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_decode<8>), hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)smem);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_decode<8>, dim3(blocks), dim3(256), smem, s, M, out, tr0, tr1);
  }
  return hipGetLastError();
}

// ── GEMM from decoded codes (prefill-shaped m > 8, or path 2); plain SIMT, fp32 accumulation ────────────
// block (64 rows x 4 tokens); thread: row n = row0 + 64 bx + (tid & 63), token j = 4 by + (tid >> 6)
template <int KQ>
__global__ void __launch_bounds__(256) k_gemm_codes(DevMat M, const uint8_t* __restrict__ codes, int row0, int nrows,
                                                     const float* __restrict__ X, int m, float* __restrict__ Y,
                                                     int ldy) {
  constexpr int GW = kq_gw(KQ), SB = kq_sbytes(KQ);
  const int nl = blockIdx.x * 64 + (threadIdx.x & 63), j = blockIdx.y * 4 + (threadIdx.x >> 6);
  if (nl >= nrows || j >= m) return;
  const int K = M.K, n = row0 + nl;
  const uint8_t* cr = codes + (size_t)nl * K;
  const float* xr = X + (size_t)j * K;
  float tot = 0.f;
  for (int b = 0; b < K / 256; ++b) {
    uint32_t sw[5];
    side_load<KQ>(M.side + ((size_t)n * (K / 256) + b) * SB, sw);
    for (int jj = 0; jj < 256 / GW; ++jj) {
      float s, o;
      side_scale<KQ>(sw, jj, s, o);
      float a = 0.f, xs = 0.f;
      for (int k = b * 256 + jj * GW; k < b * 256 + (jj + 1) * GW; ++k) {
        a = fmaf(grid_value<KQ>(cr[k]), xr[k], a);
        xs += xr[k];
      }
      tot += s * a - o * xs;
    }
  }
  Y[(size_t)j * ldy + n] = tot;
}

hipError_t launch_gemm_codes(const DevMat& M, const uint8_t* codes, int row0, int nrows, const float* X, int m,
                             float* Y, int ldy, hipStream_t s) {
  const dim3 grid((nrows + 63) / 64, (m + 3) / 4);
  switch (M.kqt) {
    case KQ_Q4_K: hipLaunchKernelGGL(k_gemm_codes<KQ_Q4_K>, grid, dim3(256), 0, s, M, codes, row0, nrows, X, m, Y, ldy); break;
    case KQ_Q5_K: hipLaunchKernelGGL(k_gemm_codes<KQ_Q5_K>, grid, dim3(256), 0, s, M, codes, row0, nrows, X, m, Y, ldy); break;
    case KQ_Q6_K: hipLaunchKernelGGL(k_gemm_codes<KQ_Q6_K>, grid, dim3(256), 0, s, M, codes, row0, nrows, X, m, Y, ldy); break;
    case KQ_IQ4_XS: hipLaunchKernelGGL(k_gemm_codes<KQ_IQ4_XS>, grid, dim3(256), 0, s, M, codes, row0, nrows, X, m, Y, ldy); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// ── HBM streaming-read control ──────────────────────────────────────────────────────────────────────────
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
__global__ void __launch_bounds__(256) k_stream_read(const u32x4* __restrict__ src, size_t n16, float* __restrict__ out) {
  uint32_t acc = 0;
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += (size_t)gridDim.x * 256) {
    const u32x4 v = __builtin_nontemporal_load(src + i);
    acc ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  out[(size_t)blockIdx.x * 256 + threadIdx.x] = __builtin_bit_cast(float, acc);
}

hipError_t launch_stream_read(const void* src, size_t n16, float* out, int blocks, hipStream_t s) {
  hipLaunchKernelGGL(k_stream_read, dim3(blocks), dim3(256), 0, s, reinterpret_cast<const u32x4*>(src), n16, out);
  return hipGetLastError();
}

}  // namespace lw
