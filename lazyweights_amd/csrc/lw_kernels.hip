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
#include <type_traits>

#include "lw_format.h"
#include "lw_kernels.h"

namespace lw {

typedef _Float16 h2v __attribute__((ext_vector_type(2)));

// leading zero bits of every device lane stream (lw_layout.h GUARD)
constexpr int GUARD_BITS = 2;
constexpr int kBufferRsrcWord3 = 0x00020000;  // buffer descriptor word 3 for raw dword loads on CDNA (32-bit data format)

typedef _Float16 h4v __attribute__((ext_vector_type(4)));
typedef float f4v __attribute__((ext_vector_type(4)));
typedef int v4i32 __attribute__((ext_vector_type(4)));
typedef float f16x16 __attribute__((ext_vector_type(16)));

// Activations of MT pseudo-tokens staged in LDS as fp16 pairs: pair c (weights 2c, 2c + 1) of token j. With
// MT >= 4 (the MFMA path) the two pairs of one 4-weight step are adjacent per token, so a lane reads its token's
// four weights with one 8-byte load.
template <int MT>
__device__ __forceinline__ int xs_index(int c, int j) {
  return MT >= 4 ? ((c >> 1) * MT + j) * 2 + (c & 1) : c * MT + j;
}

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

// Sub-block scales of one super-block packed as bytes, consumed low byte first (reference llmrt.cu:125-149; Q4_K /
// Q5_K fields per llama.cpp get_scale_min_k4, four at a time): s_j = dA * byte_j (Q6_K: signed bytes, 16 of them in
// scq then scq2; IQ4_XS: ls_j - 32, also signed), o_j = dB * m_j (side_mins).
template <int KQ>
__device__ __forceinline__ void side_packed(const uint32_t* w, uint64_t& scq, uint64_t& scq2, float& dA, float& dB) {
  if (KQ == KQ_Q4_K || KQ == KQ_Q5_K) {
    const uint32_t sc_lo = w[1] & 0x3F3F3F3Fu;
    const uint32_t sc_hi = (w[3] & 0x0F0F0F0Fu) | ((w[1] >> 2) & 0x30303030u);
    scq = (uint64_t)sc_lo | (uint64_t)sc_hi << 32;
    scq2 = 0;
    dA = h2f(w[0]);
    dB = h2f(w[0] >> 16);
  } else if (KQ == KQ_Q6_K) {
    scq = (uint64_t)w[0] | (uint64_t)w[1] << 32;
    scq2 = (uint64_t)w[2] | (uint64_t)w[3] << 32;
    dA = h2f(w[4]);
    dB = 0.f;
  } else {
    const uint32_t hi = w[0] >> 16, lo = w[1];
    uint64_t q = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t ls = ((lo >> (4 * i)) & 15u) | (((hi >> (2 * i)) & 3u) << 4);
      q |= (uint64_t)((ls - 32u) & 255u) << (8 * i);
    }
    scq = q;
    scq2 = 0;
    dA = h2f(w[0]);
    dB = 0.f;
  }
}
// Q4_K / Q5_K sub-block mins as floats
__device__ __forceinline__ void side_mins(const uint32_t* w, float* mf) {
  const uint32_t m_lo = w[2] & 0x3F3F3F3Fu;
  const uint32_t m_hi = ((w[3] >> 4) & 0x0F0F0F0Fu) | ((w[2] >> 2) & 0x30303030u);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    mf[i] = (float)((m_lo >> (8 * i)) & 255u);
    mf[4 + i] = (float)((m_hi >> (8 * i)) & 255u);
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
// matrix row 64 tr + L (lanes 32..63 start at their lane's `mid` offset). With a tile list: one-wave blocks, block
// b decodes tile list[b] (the ring kernel's exception tiles).
template <int KQ, int MT>
__global__ void __launch_bounds__(256) k_fused(DevMat M, const uint32_t* __restrict__ X2, int mt,
                                                float* __restrict__ P, const uint32_t* __restrict__ list) {
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
  const int NTHR = blockDim.x, wave = threadIdx.x >> 6;
  const int tc = list ? (int)(list[blockIdx.x] % (uint32_t)KT) : (int)blockIdx.x % KT;
  const int tr = list ? (int)(list[blockIdx.x] / (uint32_t)KT) : ((int)blockIdx.x / KT) * 4 + wave;
  const int lane = threadIdx.x & 63, l = lane & 31, half = lane >> 5;
  for (int i = threadIdx.x; i < LUTN; i += NTHR) {
    const uint32_t e = M.lut[i], sym = e & 255u;
    uint32_t v;
    if (SYMB == 4) v = f2h(grid_value<KQ>(sym & 15u)) | f2h(grid_value<KQ>(sym >> 4)) << 16;
    else v = f2h(grid_value<KQ>(sym));
    lut8[i] = make_uint2(v, e >> 8);
  }
  for (int i = threadIdx.x; i < NPAIR * MT; i += NTHR) {
    const int j = i / NPAIR, c = i - j * NPAIR;
    xs[c * MT + j] = j < mt ? X2[(size_t)j * (K / 2) + (size_t)tc * NPAIR + c] : 0u;
  }
  const bool active = tr < NT;
  const int t = tr * KT + tc;
  uint32_t* tw = tiles + wave * 32 * RS;
  if (active) stage_tile(M, t, tw, lane);
  __syncthreads();
  for (int i = threadIdx.x; i < NG * MT; i += NTHR) {
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
  uint32_t pos = half ? (uint32_t)M.mid[(size_t)t * 32 + l] : (uint32_t)GUARD_BITS;
  const uint32_t* lw = tw + l;
  const int n = tr * TN + half * 32 + l;
  float tot[MT];
#pragma unroll
  for (int j = 0; j < MT; ++j) tot[j] = 0.f;
#pragma unroll 1
  for (int sb = 0; sb < TW / 256; ++sb) {
    uint32_t sw[5];
    side_load<KQ>(M.side + side_record(n, tc * (TW / 256) + sb, M.KT, TW / 256) * SB, sw);
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
static hipError_t fused_mt(const DevMat& M, const void* X16, int mt, float* P, const uint32_t* list, int nlist,
                           hipStream_t s) {
  const size_t smem = fused_smem(M, MT);
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_fused<KQ, MT>),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
  if (e != hipSuccess) return e;
  const int blocks = list ? nlist : M.KT * ((M.NT + 3) / 4);
  hipLaunchKernelGGL((k_fused<KQ, MT>), dim3(blocks), dim3(list ? 64 : 256), smem, s, M,
                     reinterpret_cast<const uint32_t*>(X16), mt, P, list);
  return hipGetLastError();
}

template <int KQ>
static hipError_t fused_kq(const DevMat& M, const void* X16, int mt, float* P, const uint32_t* list, int nlist,
                           hipStream_t s) {
  if (mt <= 1) return fused_mt<KQ, 1>(M, X16, mt, P, list, nlist, s);
  if (mt <= 2) return fused_mt<KQ, 2>(M, X16, mt, P, list, nlist, s);
  if (mt <= 4) return fused_mt<KQ, 4>(M, X16, mt, P, list, nlist, s);
  if (mt <= 8) return fused_mt<KQ, 8>(M, X16, mt, P, list, nlist, s);
  return fused_mt<KQ, 16>(M, X16, mt, P, list, nlist, s);
}

static hipError_t fused_any(const DevMat& M, const void* X16, int mt, float* P, const uint32_t* list, int nlist,
                            hipStream_t s) {
  if (mt < 1 || mt > 16 || (list && nlist < 1)) return hipErrorInvalidValue;
  switch (M.kqt) {
    case KQ_Q4_K: return fused_kq<KQ_Q4_K>(M, X16, mt, P, list, nlist, s);
    case KQ_Q5_K: return fused_kq<KQ_Q5_K>(M, X16, mt, P, list, nlist, s);
    case KQ_Q6_K: return fused_kq<KQ_Q6_K>(M, X16, mt, P, list, nlist, s);
    case KQ_IQ4_XS: return fused_kq<KQ_IQ4_XS>(M, X16, mt, P, list, nlist, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_fused(const DevMat& M, const void* X16, int mt, float* P, hipStream_t s) {
  return fused_any(M, X16, mt, P, nullptr, 0, s);
}

hipError_t launch_fused_exceptions(const DevMat& M, const void* X16, int mt, float* P, hipStream_t s) {
  if (M.nexc <= 0) return hipSuccess;
  return fused_any(M, X16, mt, P, M.exc, M.nexc, s);
}

// Sum of x over one sub-block (GW weights = GW / 2 fp16 pairs, pair(c) for c < GW / 2) in a fixed order shared by
// every kernel: four quarter sums, each sequential, combined as (q0 + q1) + (q2 + q3).
template <int GW, class Pair>
__device__ __forceinline__ float xsum_sub(Pair pair) {
  constexpr int Q = GW / 8;  // pairs per quarter
  float q[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    q[k] = 0.f;
    for (int c = 0; c < Q; ++c) {
      const uint32_t v = pair(k * Q + c);
      q[k] += h2f(v) + h2f(v >> 16);
    }
  }
  return (q[0] + q[1]) + (q[2] + q[3]);
}

// Ring staging of one front: chunk k = rows [2k, 2k + 2) after the front's base row; lane l carries row
// 2k + l / 16, words 2 (l % 16) .. + 1 (`src` points at that lane's 8 bytes of chunk 0, `lane_slot` at its place in
// ring slot 0). At the start of group g the chunks loaded at g - 2 are written and group g's loads are issued
// (2-bit counts per group). Tiles whose two fronts share one schedule use the scalar form (wave-uniform counts,
// branches and offsets); the others keep one schedule per front (per-lane counts).
template <class I, class U>
struct RingStager {
  uint2* lane_slot;
  const uint2* src;
  U counts;
  uint32_t rmask;  // ring rows - 1 (16 or 32 rows, wave-uniform)
  I written, issued, pend0, pend1;
  uint2 s00, s01, s10, s11;  // chunks in flight, by group parity

  __device__ __forceinline__ void put(I k, uint2 v) { lane_slot[((2 * k) & (I)rmask) * 16] = v; }
  __device__ __forceinline__ void init(I n) {
    for (I k = 0; k < n; ++k) put(k, src[32 * k]);
    written = issued = n;
    pend0 = pend1 = 0;
    s00 = s01 = s10 = s11 = make_uint2(0, 0);
  }
  __device__ __forceinline__ void step(int g, I& pend, uint2& a, uint2& b) {
    if (pend > 0) put(written++, a);
    if (pend > 1) put(written++, b);
    const I nload = (I)((counts >> (2 * g)) & 3u);
    if (nload > 0) a = src[32 * issued++];
    if (nload > 1) b = src[32 * issued++];
    pend = nload;
  }
  __device__ __forceinline__ void stage(int g) {
    if (g & 1) step(g, pend1, s10, s11);
    else step(g, pend0, s00, s01);
  }
};

// ── ring-staged fused kernel, grouped over the matrices of a layer ────────────────────────────────────────
// As k_fused, but a wave does not stage its whole tile: each front (lanes 0-31 from bit GUARD, lanes 32-63 from
// their `mid` offsets) keeps a ring of RS word rows and streams 2-row chunks (one 8-byte load per lane) from HBM on
// the tile's load-time schedule (Layout::sched): chunks loaded at group g are written to the ring at the start of
// group g + 2, so their latency hides behind two groups of decode.
// Each lane holds its window rows r, r + 1 in registers (A, B) and the next row r + 2 (C), re-read from its ring
// column after every pair of symbols; when a pair crosses into row r + 1 the window slides (A = B, B = C). A pair
// decodes from one 32-bit window w1 = alignbit(B, A, pos): the first symbol at the guard-aligned offset, the second
// from w1 >> len1. So the only LDS reads on a pair's dependency chain are its two table lookups.
//
// The decode table holds 4-byte entries (8 KB, built at load time: DevMat::lut4, decode_table4): bits 0-7 = code
// length; 4-bit formats: bytes 2 and 3 = the pair's two grid bytes (Q4_K: q; IQ4_XS: kv[q] + 128), which one byte
// permute turns into two fp16 denormals g * 2^-24 for v_dot2 (exact: g < 256; the 2^24 is folded into d); 8-bit
// formats: bits 16-31 = fp16(f(q)). The position update adds whole entries: only bits 0-15 of the position are
// used (ring slot and bit offset), and the entries' upper halves only disturb bits >= 16.
// block = WPB tile rows of one tile column of one matrix of the plan.

// LDS address of the table entry indexed by window bits 2..12 of w: (w & 0x1FFC) | table base, one instruction (the
// base is a multiple of 8 KB and wave-uniform)
__device__ __forceinline__ uint32_t table_addr(uint32_t w, uint32_t base, uint32_t mask) {
  uint32_t a;  // VOP3 takes no literal here: the mask 0x1FFC lives in a register
  asm("v_and_or_b32 %0, %1, %3, %2" : "=v"(a) : "v"(w), "s"(base), "v"(mask));
  return a;
}

// LDS address of the entry of the code at window bits 2..12 of w by the comparator lookup (reference
// hw/huff/huff_engine.h:54-77) over a matrix's comparator table (canon_table): v = the 11 window bits with the
// code's first bit most significant; its length l is 1 + the number of limits lim[0..9] that v reaches, and
// pk[l - 1] = (table base + 4 (base_l - first_l)) << 16 | (11 - l) turns v into the entry's address. lim and pk
// are wave-uniform (SGPRs): 10 subtract / shift / insert steps per code.
// compile-time loop: f(std::integral_constant<int, i>) for i = 0 .. N - 1 (indices that must be constants: MFMA
// broadcast fields, register-array indices; bodies past the loop unroller's size limit)
template <int I, int N, class F>
__device__ __forceinline__ void static_for_from(F& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for_from<I + 1, N>(f);
  }
}
template <int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_from<0, N>(f);
}

__device__ __forceinline__ uint32_t canon_addr(uint32_t w, const uint32_t* lim, const uint32_t* pk) {
  const uint32_t v = __builtin_amdgcn_ubfe(__builtin_bitreverse32(w), 19, 11);
  uint32_t p = pk[0];
#pragma unroll
  for (int k = 0; k < 10; ++k) {  // p = v < lim[k] ? p : pk[k + 1] by the sign of v - lim[k] (11-bit values) and a
                                   // bitfield insert: no VCC, and no per-lane indexed load of pk
    uint32_t t;
    asm("v_subrev_u32 %1, %3, %2\n\tv_ashrrev_i32 %1, 31, %1\n\tv_bfi_b32 %0, %1, %0, %4"
        : "+v"(p), "=&v"(t)
        : "v"(v), "s"(lim[k]), "s"(pk[k + 1]));
  }
  return ((v >> (p & 31u)) << 2) + (uint32_t)((int)p >> 16);
}

// x sub-block sums held in LDS per block ([NG][MT], the block-per-column kernel)
struct XgLds {
  const float* xg;
  int MT, nsub;
  __device__ __forceinline__ float operator()(int sb, int jj, int j) const { return xg[(sb * nsub + jj) * MT + j]; }
};
// one token's x sub-block sums of the wave's tile column in scalar registers (the flat kernel): super-block 0, 1
struct XgRegs {
  float x0[8], x1[8];
  __device__ __forceinline__ float operator()(int sb, int jj, int) const { return sb ? x1[jj] : x0[jj]; }
};

// One tile's decode + dequant + dot products for both fronts of a wave (see k_fused_ring); `st` stages the ring,
// `xgf(sub, j)` = sum of token j's x over sub-block `sub` of the tile column, `lutsel` = byte offset of the tile's
// decode table within `lut4` (0 or 8192, OR-ed into the index).
// Symbol source of tile_gemv: the ring decoder. Window rows r, r + 1 in registers (A, B), row r + 2 (C) re-read
// from the lane's ring column after every pair; P = bit position + 64 (bits 0-4: window offset, bits 5+: the row C
// holds). pair() decodes the next two symbols and returns their table entries.
template <class Stager>
struct RingSrc {
  static constexpr bool kFullUnroll = false, kPrefetchSide = false, kXLds = false;
  static constexpr const uint32_t* xl = nullptr;
  typedef __attribute__((address_space(3))) const uint32_t LdsU32;
  Stager& st;
  uint32_t P, rlb, tsel, tmask, rmask, rbits, slot, A, B, C;
  __device__ __forceinline__ RingSrc(Stager& s, const uint32_t* lut4, uint32_t lutsel, uint32_t P0, uint32_t rlb0)
      : st(s), P(P0), rlb(rlb0) {
    rmask = st.rmask;
    rbits = rmask == 15u ? 4u : 5u;  // ring of 16 or 32 rows
    // LDS byte address of the tile's table (a multiple of 8 KB: the tables are the kernels' only static LDS object)
    tsel = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const uint32_t*)lut4 + lutsel;
    tmask = 0x1FFCu;
    asm volatile("" : "+v"(tmask));
    __builtin_amdgcn_s_setprio(3);
    slot = __builtin_amdgcn_ubfe(P, 5, rbits);
    A = *(LdsU32*)(rlb + (((slot - 2u) & rmask) << 7));
    B = *(LdsU32*)(rlb + (((slot - 1u) & rmask) << 7));
    C = *(LdsU32*)(rlb + (slot << 7));
  }
  // group g (16 symbols) begins: issue priority falls with progress (3 for the first quarter of the tile .. 0 for the
  // last), so the waves sharing a SIMD keep pace instead of the oldest finishing first and the youngest running
  // alone at the end; then the ring staging step
  __device__ __forceinline__ void stage(int g) {
    if (g == 4) __builtin_amdgcn_s_setprio(2);
    if (g == 8) __builtin_amdgcn_s_setprio(1);
    if (g == 12) __builtin_amdgcn_s_setprio(0);
    st.stage(g);
  }
  __device__ __forceinline__ void pair(int, uint32_t& e1, uint32_t& e2) {
    const uint32_t w1 = __builtin_amdgcn_alignbit(B, A, P);
    e1 = *(LdsU32*)table_addr(w1, tsel, tmask);
    // the second symbol lies within w1: it starts len1 <= 11 bits further and its table index ends by bit 24
    const uint32_t w2 = w1 >> (e1 & 31u);
    e2 = *(LdsU32*)table_addr(w2, tsel, tmask);
    P = P + e1 + e2;  // lengths land in bits 0-15 exactly; entry values only disturb bits >= 16
    // a pair advances at most 22 bits: the window slides by at most one row
    const uint32_t nslot = __builtin_amdgcn_ubfe(P, 5, rbits);
    const bool slide = nslot != slot;
    A = slide ? B : A;
    B = slide ? C : B;
    slot = nslot;
    C = *(LdsU32*)(rlb + (nslot << 7));
  }
};

// Symbol source of tile_gemv: the packed (fixed-rate) twin. Lane L reads the 16 symbol bytes of group g of its
// tile row as one 16-byte chunk (chunk g at src + 64 g, one group ahead in registers) and looks each symbol up in
// the 256-entry symbol table, whose entries carry the same payload bits as the decode table's: the products, and
// so the results, are those of the coded matrix with the same codes.
// Q4_K needs no table: a symbol's grid bytes are its two nibbles, placed in bytes 2 and 3 of the entry with one
// byte permute of the word's low and high nibbles.
// The chunks stream through a per-wave LDS ring of PK_SLOTS 1 KB slots by direct-to-LDS loads, PK_DEPTH groups
// ahead, so several KB per wave are in flight without holding registers. kFullUnroll: the pairs of a group are
// unrolled (pair(p) selects its word by p).
constexpr int PK_DEPTH = 3, PK_SLOTS = PK_DEPTH + 1;
// m = 1 (kXLds): the tile column's x pairs are staged in LDS too (xl, 1 KB per wave), since without a decode chain
// the scalar-cache latency of x per group would be exposed.
template <int KQ>
struct PackedSrc {
  static constexpr bool kFullUnroll = true, kPrefetchSide = false, kXLds = true;
  typedef __attribute__((address_space(3))) const uint32_t LdsU32;
  const uint4* src;  // this lane's chunk of group 0; group g at src + 64 g
  uint4* ring;       // the wave's PK_SLOTS x 64 chunks
  const uint32_t* xl;
  uint4 cur;
  uint32_t tsel, lo, hi, lane;
  __device__ __forceinline__ void fetch(int g) {
    __builtin_amdgcn_global_load_lds(src + 64 * g, (__attribute__((address_space(3))) void*)(ring + (g % PK_SLOTS) * 64),
                                     16, 0, 0);
  }
  // x: the tile column's pairs (TW / 2 dwords) into xs, with direct-to-LDS loads (null: not staged)
  __device__ __forceinline__ PackedSrc(const uint4* s, uint4* r, const uint32_t* tab, uint32_t l, const uint32_t* xcol,
                                       uint32_t* xs)
      : src(s), ring(r), xl(xs), lane(l) {
    tsel = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const uint32_t*)tab;
    if (xs) {
      constexpr int NPAIR = (kq_symbits(KQ) == 4 ? 2 * TK : TK) / 2;
#pragma unroll
      for (int i = 0; i < NPAIR / 64; ++i)
        __builtin_amdgcn_global_load_lds(xcol + 64 * i + l, (__attribute__((address_space(3))) void*)(xs + 64 * i), 4, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < PK_DEPTH; ++i) fetch(i);
  }
  // group g: fetch group g + PK_DEPTH (into the slot group g - 1 used), wait for group g's chunk (loads complete in
  // order: at most PK_DEPTH younger ones may stay outstanding), read it
  __device__ __forceinline__ void stage(int g) {
    if (g + PK_DEPTH < 16) {
      fetch(g + PK_DEPTH);
      __builtin_amdgcn_s_waitcnt(PK_DEPTH == 3 ? 0x0F73 : 0x0F70);  // vmcnt(PK_DEPTH)
    } else {
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    }
    // the read is opaque to the compiler, which would otherwise wait for every direct-to-LDS load before any LDS
    // read (the explicit vmcnt above already orders this one)
    const uint32_t a = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint4*)(ring + (g % PK_SLOTS) * 64 + lane);
    asm volatile("ds_read_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(cur) : "v"(a));
  }
  __device__ __forceinline__ void pair(int p, uint32_t& e1, uint32_t& e2) {
    const uint32_t w = p < 2 ? cur.x : p < 4 ? cur.y : p < 6 ? cur.z : cur.w;
    if (KQ == KQ_Q4_K) {
      if (!(p & 1)) {
        lo = w & 0x0F0F0F0Fu;
        hi = (w >> 4) & 0x0F0F0F0Fu;
      }
      const uint32_t k = 2 * (p & 1);  // symbols k, k + 1 of the word: entry bytes 2, 3 = their low, high nibble
      e1 = __builtin_amdgcn_perm(hi, lo, 0x00000C0Cu | (k << 16) | ((4u + k) << 24));
      e2 = __builtin_amdgcn_perm(hi, lo, 0x00000C0Cu | ((k + 1) << 16) | ((5u + k) << 24));
    } else {
      const uint32_t h = (p & 1) ? w >> 16 : w;
      e1 = *(LdsU32*)(tsel + ((h & 255u) << 2));
      e2 = *(LdsU32*)(tsel + (((h >> 8) & 255u) << 2));
    }
  }
};

// One tile's dequant + dot products for both fronts of a wave, from a symbol source (`src.stage(g)` at each
// 16-symbol group, `src.pair(p, e1, e2)` for the table entries of the group's pair p: see decode_table4).
// `xgf(sb, jj, j)` = sum of token j's x over sub-block jj of super-block sb of the tile column.
template <int KQ, int MT, bool COH = false, class Src, class Xg>
__device__ __forceinline__ void tile_gemv(Src& src, const uint32_t* xs, const Xg& xgf,
                                          __attribute__((address_space(4))) const uint32_t* xcol,
                                          const uint8_t* srow, int mt, int N, float* out) {
  constexpr int SYMB = kq_symbits(KQ);
  constexpr int TW = SYMB == 4 ? 2 * TK : TK;
  constexpr int GW = kq_gw(KQ), SB = kq_sbytes(KQ);
  constexpr bool XS_SGPR = MT == 1;
  constexpr int NSB = TW / 256;      // super-blocks per tile column
  constexpr int GPS = 16 / NSB;      // staging groups (16 symbols) per super-block
  constexpr int NSUB = 256 / GW;     // sub-blocks per super-block
  constexpr int GPSUB = GPS / NSUB;  // groups per sub-block (2 for Q5_K, else 1)
  // 4-bit formats accumulate in units of 2^-24 (denormal grid values); IQ4_XS grid bytes carry a +128 bias
  constexpr float VSCALE = SYMB == 4 ? 16777216.f : 1.f;
  float tot[MT], acc[MT];
#pragma unroll
  for (int j = 0; j < MT; ++j) tot[j] = acc[j] = 0.f;
  // MT >= 4: the products go to the matrix cores. v_mfma_f32_4x4x4f16 computes, per block of 4 lanes, D[i][j] =
  // sum_k A[lane 4b + i][k] B[lane 4b + j][k] into lane 4b + j, register i. With A = the four x values of token
  // 4q + i (lane 4b + i reads token i) and B = the lane's own four weights, lane 4b + j gets its own row's dot
  // products for tokens 4q .. 4q + 3, as acc[4q + i] does on the dot2 path.
  constexpr bool MMA = MT >= 4;
  constexpr int NQ = MMA ? MT / 4 : 1;
  f4v accm[NQ];
#pragma unroll
  for (int q = 0; q < NQ; ++q) accm[q] = f4v{0.f, 0.f, 0.f, 0.f};
  const uint32_t ltok = __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)) & 3u;
  uint32_t wprev = 0;
  // sources without a decode chain (kPrefetchSide) load the next super-block's side words a super-block ahead, so
  // their HBM latency hides behind a super-block of work; the ring decoder's registers are too tight for that
  uint32_t swn[5] = {0, 0, 0, 0, 0};
  if (Src::kPrefetchSide) side_load<KQ>(srow, swn);

#pragma unroll 1
  for (int sb = 0; sb < NSB; ++sb) {
    uint32_t sw[5];
    if (Src::kPrefetchSide) {
#pragma unroll
      for (int i = 0; i < 5; ++i) sw[i] = swn[i];
      if (sb + 1 < NSB) side_load<KQ>(srow + (sb + 1) * (TN * SB), swn);
    } else {
      side_load<KQ>(srow + sb * (TN * SB), sw);
    }
    float dA, dB;
    uint64_t scq, scq2;  // sub-block scales as bytes (signed for Q6_K / IQ4_XS), consumed low byte first
    side_packed<KQ>(sw, scq, scq2, dA, dB);
    // per super-block x terms, applied first: y -= dmin sum_j m_j (sum x)_j (Q4_K / Q5_K mins) or
    // 128 d sum_j s_j (sum x)_j (the IQ4_XS +128 grid bias); y += d sum_j sc_j (x . q)_j follows at the end
    float tsum[MT];
#pragma unroll
    for (int j = 0; j < MT; ++j) {
      tsum[j] = 0.f;
      if (KQ == KQ_Q4_K || KQ == KQ_Q5_K) {
        float mf[8], msum = 0.f;
        side_mins(sw, mf);
#pragma unroll
        for (int jj = 0; jj < NSUB; ++jj) msum = fmaf(mf[jj], xgf(sb, jj, j), msum);
        tot[j] = fmaf(-dB, msum, tot[j]);
      }
      if (KQ == KQ_IQ4_XS) {
        float csum = 0.f;
#pragma unroll
        for (int jj = 0; jj < NSUB; ++jj)
          csum = fmaf((float)(int)(int8_t)(uint8_t)(scq >> (8 * jj)), xgf(sb, jj, j), csum);
        tot[j] = fmaf(-128.f * dA, csum, tot[j]);
      }
    }
#pragma unroll 1
    for (int gg2 = 0; gg2 < GPS; gg2 += 2) {
      if (KQ == KQ_Q6_K && gg2 == 8) scq = scq2;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int g = sb * GPS + gg2 + h;
        src.stage(g);
        // m = 1 unrolls the group fully; more tokens unroll less (their x operands come from LDS per pair)
#pragma unroll((MT == 1 || Src::kFullUnroll) ? 8 : (MMA && SYMB == 4 ? 1 : 2))
        for (int p = 0; p < 8; ++p) {
          uint32_t e1, e2;
          src.pair(p, e1, e2);
          if (SYMB == 4) {
            const uint32_t v1 = __builtin_amdgcn_perm(e1, e1, 0x0C030C02u), v2 = __builtin_amdgcn_perm(e2, e2, 0x0C030C02u);
            const int c = 16 * g + 2 * p;
            if (XS_SGPR) {
              if (Src::kXLds) acc[0] = dot2(v2, src.xl[c + 1], dot2(v1, src.xl[c], acc[0]));
              else acc[0] = dot2(v2, xcol[c + 1], dot2(v1, xcol[c], acc[0]));
            } else if (MMA) {
              const h4v wv = __builtin_bit_cast(h4v, make_uint2(v1, v2));
#pragma unroll
              for (int q = 0; q < NQ; ++q) {
                const uint2 xv = *reinterpret_cast<const uint2*>(xs + xs_index<MT>(c, 4 * q + (int)ltok));
                accm[q] = __builtin_amdgcn_mfma_f32_4x4x4f16(__builtin_bit_cast(h4v, xv), wv, accm[q], 0, 0, 0);
              }
            } else {
              const uint32_t* x1 = xs + c * MT;
#pragma unroll
              for (int j = 0; j < MT; ++j) acc[j] = dot2(v2, x1[MT + j], dot2(v1, x1[j], acc[j]));
            }
          } else {
            const uint32_t w = __builtin_amdgcn_perm(e2, e1, 0x07060302u);
            const int c = 8 * g + p;
            if (XS_SGPR) {
              if (Src::kXLds) acc[0] = dot2(w, src.xl[c], acc[0]);
              else acc[0] = dot2(w, xcol[c], acc[0]);
            } else if (MMA) {  // one 4-weight product per two pairs (c odd: pairs c - 1, c)
              if (p & 1) {
                const h4v wv = __builtin_bit_cast(h4v, make_uint2(wprev, w));
#pragma unroll
                for (int q = 0; q < NQ; ++q) {
                  const uint2 xv = *reinterpret_cast<const uint2*>(xs + xs_index<MT>(c - 1, 4 * q + (int)ltok));
                  accm[q] = __builtin_amdgcn_mfma_f32_4x4x4f16(__builtin_bit_cast(h4v, xv), wv, accm[q], 0, 0, 0);
                }
              } else {
                wprev = w;
              }
            } else {
              const uint32_t* x1 = xs + c * MT;
#pragma unroll
              for (int j = 0; j < MT; ++j) acc[j] = dot2(w, x1[j], acc[j]);
            }
          }
        }
        if (GPSUB == 1 || h == 1) {  // sub-block end: scale x partial dot, next scale byte
          const float scv = (KQ == KQ_Q6_K || KQ == KQ_IQ4_XS) ? (float)(int)(int8_t)(uint8_t)scq
                                                               : (float)(uint32_t)(scq & 255u);
          scq >>= 8;
          if (MMA) {
#pragma unroll
            for (int q = 0; q < NQ; ++q) {
#pragma unroll
              for (int i = 0; i < 4; ++i) tsum[4 * q + i] = fmaf(scv, accm[q][i], tsum[4 * q + i]);
              accm[q] = f4v{0.f, 0.f, 0.f, 0.f};
            }
          } else {
#pragma unroll
            for (int j = 0; j < MT; ++j) {
              tsum[j] = fmaf(scv, acc[j], tsum[j]);
              acc[j] = 0.f;
            }
          }
        }
      }
    }
    // super-block end: y += d sum_j sc_j (x . q)_j
#pragma unroll
    for (int j = 0; j < MT; ++j) tot[j] = fmaf(dA * VSCALE, tsum[j], tot[j]);
  }
#pragma unroll
  for (int j = 0; j < MT; ++j)
    if (j < mt) {
      if (COH)  // coherent across the device's caches, for a reduction inside the launch
        __hip_atomic_store(out + (size_t)j * N, tot[j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      else
        out[(size_t)j * N] = tot[j];
    }
}


template <int KQ, int MT, int WPB, int RS>
__global__ void __launch_bounds__(WPB * 64, MT <= 2 ? 8 : (MT <= 8 ? 4 : 2)) k_fused_ring(GroupPlan plan) {
  constexpr int SYMB = kq_symbits(KQ);
  constexpr int TW = SYMB == 4 ? 2 * TK : TK;
  constexpr int GW = kq_gw(KQ), NG = TW / GW, SB = kq_sbytes(KQ), NPAIR = TW / 2;
  static_assert(RS == 16 || RS == 32, "ring of 16 or 32 rows");
  constexpr int RING_WORDS = RS * 32;
  constexpr int NTHR = WPB * 64;
  constexpr bool XS_SGPR = MT == 1;  // m = 1: activations straight from the scalar cache
  __shared__ uint32_t lut4[LUTN];
  extern __shared__ __align__(16) uint32_t smem[];
  uint32_t* xs = smem;                                          // [NPAIR][MT] fp16 pairs
  float* xg = reinterpret_cast<float*>(xs + NPAIR * MT);        // [NG][MT] sub-block sums of x
  uint32_t* rings = reinterpret_cast<uint32_t*>(xg + NG * MT);  // WPB x 2 fronts x RS rows

  // the block's matrix: a uniform index into the plan, read through the kernel-argument segment (scalar loads)
  int mi = 0;
#pragma unroll
  for (int i = 1; i < MAX_GROUP; ++i)
    if (i < plan.n && (int)blockIdx.x >= plan.e[i].block0) mi = i;
  typedef __attribute__((address_space(4))) const char KChar;
  typedef __attribute__((address_space(4))) const GroupEntry KEntry;
  KChar* kbase = (KChar*)__builtin_amdgcn_kernarg_segment_ptr();
  KEntry* ep = (KEntry*)(kbase + offsetof(GroupPlan, e) + (size_t)mi * sizeof(GroupEntry));
  const auto& E = *ep;
  const auto& M = E.M;
  const int mt = plan.mt;
  const int bl = (int)blockIdx.x - E.block0;
  const int KT = M.KT, NT = M.NT, K = M.K, N = M.N;
  // wave-uniform indices are made explicit (scalar registers): the tile, its schedule and its base addresses
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int tc = bl % KT, tr = (bl / KT) * WPB + wave;
  const int lane = threadIdx.x & 63, l = lane & 31, f = lane >> 5;

  for (int i = threadIdx.x; i < LUTN / 4; i += NTHR) reinterpret_cast<uint4*>(lut4)[i] = reinterpret_cast<const uint4*>(M.lut4)[i];
  for (int i = threadIdx.x; i < NPAIR * MT; i += NTHR) {
    const int j = i / NPAIR, c = i - j * NPAIR;
    xs[xs_index<MT>(c, j)] = j < mt ? E.X2[(size_t)j * (K / 2) + (size_t)tc * NPAIR + c] : 0u;
  }
  __syncthreads();
  for (int i = threadIdx.x; i < NG * MT; i += NTHR) {
    const int g = i / MT, j = i - g * MT;
    xg[g * MT + j] = xsum_sub<GW>([&](int c) { return xs[xs_index<MT>(g * (GW / 2) + c, j)]; });
  }
  __syncthreads();
  if (tr >= NT) return;

  const int t = tr * KT + tc;
  const uint4 sc = M.sched[t];
  if (sc.w & 1u) return;  // no ring schedule for this tile: decoded by the whole-tile kernel's exception pass
  typedef __attribute__((address_space(4))) const uint32_t KU32;
  const int base_f = f ? (int)(sc.z & 255u) : 0;
  uint32_t* ring = rings + (wave * 2 + f) * RING_WORDS;
  const uint2* src = reinterpret_cast<const uint2*>(M.words + M.tbase[t]) + (uint32_t)(16 * base_f + l);
  uint2* lane_slot = reinterpret_cast<uint2*>(ring) + (l >> 4) * 16 + (l & 15);
  // P = the lane's bit position (relative to the front's base row) + 64: bits 0-4 are the window offset and the
  // row field (bits 5+) names row r + 2, the row C holds
  const uint32_t P = (f ? (uint32_t)M.mid[(size_t)t * 32 + (uint32_t)l] - GUARD_BITS : 0u) - 32u * (uint32_t)base_f + 64u;
  // this lane's column of the ring as one opaque byte address, so a row address is (slot * 128) + base
  uint32_t rlb = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint32_t*)(ring + l);
  asm volatile("" : "+v"(rlb));
  // this tile's side records (uniform base) + the lane's record (super-block sb: + sb * 64 records)
  const uint8_t* srow = M.side + side_record(tr * TN, tc * (TW / 256), KT, TW / 256) * SB + (uint32_t)((f * 32 + l) * SB);
  KU32* xcol = (KU32*)(E.X2 + (size_t)tc * NPAIR);  // uniform: this tile column's x pairs (m = 1)
  float* out = E.P + (size_t)tc * mt * N + (size_t)tr * TN + (uint32_t)(f * 32 + l);
  const uint32_t init0 = (sc.z >> 8) & 255u, init1 = (sc.z >> 16) & 255u;
  if (sc.x == sc.y && init0 == init1) {  // one schedule for both fronts: scalar staging
    RingStager<int, uint32_t> st;
    st.lane_slot = lane_slot;
    st.src = src;
    st.counts = sc.x;
    st.rmask = RS - 1;
    st.init((int)init0);
    RingSrc<RingStager<int, uint32_t>> src(st, lut4, 0u, P, rlb);
    tile_gemv<KQ, MT>(src, xs, XgLds{xg, MT, 256 / GW}, xcol, srow, mt, N, out);
  } else {
    RingStager<int, uint32_t> st;
    st.lane_slot = lane_slot;
    st.src = src;
    st.counts = f ? sc.y : sc.x;
    st.rmask = RS - 1;
    st.init((int)(f ? init1 : init0));
    RingSrc<RingStager<int, uint32_t>> src(st, lut4, 0u, P, rlb);
    tile_gemv<KQ, MT>(src, xs, XgLds{xg, MT, 256 / GW}, xcol, srow, mt, N, out);
  }
}

// ── flat launches (m = 1): shared pieces ─────────────────────────────────────────────────────────────────
// Reduction in the launch. A wave stores its tile's 64 partials (relaxed agent-scope atomic stores) and lane 0 counts
// the tile in its tile row with a relaxed agent-scope atomic (no wait between the two); the wave that counts the
// row's last tile resets the counter and sums the row's partials in tile-column order (the order of k_reduce_group,
// so the bits are the same). No ordering between the partials and the counter is assumed (an
// agent-scope release / acquire on gfx950 is a buffer_wbl2 / buffer_inv per wave, which measured 106-143 us per
// config-2 layer against 45 us): a partial slot holds kNoPartial from the end of one reduction to the store of the
// next partial, so the summing wave takes each slot by an atomic exchange with kNoPartial until what it takes is not
// kNoPartial (coherence of that one location: it sees the last reduction's kNoPartial, which a launch boundary
// orders before, or the new partial). The counter only elects the summing wave. No-op when the entry has no Y
// (reduced by a separate launch, which resets the slots likewise). Slots start as kNoPartial (filled when the
// partials buffer is allocated).

// The sum over columns c < KT, in order, of the partial slots q + c cs. Each slot is taken by an exchange with
// kNoPartial, 32 in flight. A slot still holding kNoPartial (its partial counted but not yet visible here) makes the
// running sum NaN, so one test per batch finds it; the batch is then summed again once every such slot has its
// partial (at most kPartialSpins re-reads each, a few hundred cycles apiece; past that the sum is NaN rather than a
// hang). A NaN of the data itself only costs the re-summation: no arithmetic result has kNoPartial's bits.
__device__ __forceinline__ float sum_partials(uint32_t* q, size_t cs, int KT) {
  constexpr int B = 32;
  auto take = [&](int c) {
    return __hip_atomic_exchange(q + (size_t)c * cs, kNoPartial, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  };
  float a = 0.f;
  for (int c0 = 0; c0 < KT; c0 += B) {
    uint32_t v[B];
#pragma unroll
    for (int u = 0; u < B; ++u) v[u] = c0 + u < KT ? take(c0 + u) : 0u;
    const float a0 = a;
#pragma unroll
    for (int u = 0; u < B; ++u)
      if (c0 + u < KT) a += __builtin_bit_cast(float, v[u]);
    if (__builtin_expect(a != a, 0)) {
      a = a0;
      for (int u = 0; u < B && c0 + u < KT; ++u) {
        uint32_t w = v[u];
        for (int i = 0; w == kNoPartial && i < kPartialSpins; ++i) {
          __builtin_amdgcn_s_sleep(2);
          w = take(c0 + u);
        }
        a += w == kNoPartial ? __builtin_nanf("") : __builtin_bit_cast(float, w);
      }
    }
  }
  return a;
}
// The sums of tile row tr's partials, per token j < mt, by the wave that counted the row's last tile (it also resets
// the counter). P is [KT][mt][N]: token j's partial of tile column c at P + (c mt + j) N.
// (reset = false: the row was counted elsewhere, its counter is untouched)
template <class KEntryRef>
__device__ __forceinline__ void row_sum(const KEntryRef& E, int tr, int KT, int N, int lane, int mt = 1,
                                        bool reset = true) {
  if (reset && lane == 0) __hip_atomic_store(E.cnt + tr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  uint32_t* const q = reinterpret_cast<uint32_t*>(E.P + (size_t)tr * TN + (uint32_t)lane);
#pragma unroll 1
  for (int j = 0; j < mt; ++j)
    E.Y[(size_t)j * (mt > 1 ? E.ldy : 0) + (size_t)tr * TN + (uint32_t)lane] =
        sum_partials(q + (size_t)j * N, (size_t)mt * N, KT);
}

template <class KEntryRef>
__device__ __forceinline__ void row_reduce(const KEntryRef& E, int tr, int KT, int N, int lane, int mt = 1) {
  if (!E.Y) return;
  uint32_t old = 0;
  if (lane == 0) old = __hip_atomic_fetch_add(E.cnt + tr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  old = __builtin_amdgcn_readlane(old, 0);
  if (old != (uint32_t)(KT - 1)) return;
  row_sum(E, tr, KT, N, lane, mt);
}

// One tile column's x sums per sub-block (m = 1), as wave-uniform values: lane 4 g + k sums quarter k of sub-block
// g; two exchanges give (q0 + q1) + (q2 + q3), the order of xsum_sub (so all kernels give the same bits).
template <int KQ>
__device__ __forceinline__ XgRegs column_xsums(const uint32_t* X2, int tc, int lane) {
  constexpr int SYMB = kq_symbits(KQ);
  constexpr int TW = SYMB == 4 ? 2 * TK : TK;
  constexpr int GW = kq_gw(KQ);
  XgRegs xgr;
  if (KQ != KQ_Q6_K) {
    constexpr int NSUBT = TW / GW, Q = GW / 8;  // sub-blocks per tile column, pairs per quarter
    float a = 0.f;
    if (lane < 4 * NSUBT) {
      const uint32_t* xl = X2 + (size_t)tc * (TW / 2) + (uint32_t)(lane * Q);
      for (int c = 0; c < Q; ++c) {
        const uint32_t v = xl[c];
        a += h2f(v) + h2f(v >> 16);
      }
    }
    a += __shfl_xor(a, 1);
    a += __shfl_xor(a, 2);
#pragma unroll
    for (int g = 0; g < 8; ++g) {
      xgr.x0[g] = g < NSUBT ? __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, a), 4 * g)) : 0.f;
      xgr.x1[g] = g + 8 < NSUBT ? __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, a), 4 * (g + 8))) : 0.f;
    }
  }
  return xgr;
}

// ── int8 activations (m = 1), the reference's k_quant_x8 + k_gemvm_kq8 (kernels/llmrt.cu:1035-1169) ───────
// Quantization: one block of 32 activations per half-wave.
__device__ __forceinline__ void quant_x8_block(const void* __restrict__ X, int x_f16, int8_t* __restrict__ XQ,
                                               float* __restrict__ DX, float* __restrict__ SX, int b, int l) {
  const size_t i = (size_t)b * 32 + l;
  const float v = x_f16 ? h2f(static_cast<const uint16_t*>(X)[i]) : static_cast<const float*>(X)[i];
  float a = fabsf(v);
#pragma unroll
  for (int o = 16; o; o >>= 1) a = fmaxf(a, __shfl_xor(a, o));
  const float d = a / 127.f;
  const int q = d > 0.f ? (int)rintf(v / d) : 0;  // round to nearest even, as __float2int_rn
  int sm = q;
#pragma unroll
  for (int o = 16; o; o >>= 1) sm += __shfl_xor(sm, o);
  XQ[i] = (int8_t)q;
  if (l == 0) {
    DX[b] = d;
    SX[b] = d * (float)sm;
  }
}

__global__ void __launch_bounds__(256) k_quant_x8(const void* __restrict__ X, int x_f16, int8_t* __restrict__ XQ,
                                                  float* __restrict__ DX, float* __restrict__ SX, int nb) {
  const int b = blockIdx.x * 8 + (threadIdx.x >> 5), l = threadIdx.x & 31;
  if (b >= nb) return;  // a half-wave's exchanges stay inside it (xor offsets < 32)
  quant_x8_block(X, x_f16, XQ, DX, SX, b, l);
}

// several vectors in one launch (the distinct activation vectors of a grouped call)
__global__ void __launch_bounds__(256) k_quant_x8_group(QuantJobs q) {
  int j = 0;
#pragma unroll
  for (int i = 1; i < MAX_GROUP; ++i)
    if (i < q.n && (int)blockIdx.x >= q.b0[i]) j = i;
  const int b = ((int)blockIdx.x - q.b0[j]) * 8 + (threadIdx.x >> 5), l = threadIdx.x & 31;
  if (b >= q.nb[j]) return;
  quant_x8_block(q.X[j], q.x_f16, q.XQ[j], q.DX[j], q.SX[j], b, l);
}

hipError_t launch_quant_x8(const void* X, int x_f16, int m, int K, int8_t* XQ, float* DX, float* SX, hipStream_t s) {
  if (m < 1 || K % 32) return hipErrorInvalidValue;
  const int nb = m * K / 32;
  hipLaunchKernelGGL(k_quant_x8, dim3((nb + 7) / 8), dim3(256), 0, s, X, x_f16, XQ, DX, SX, nb);
  return hipGetLastError();
}

hipError_t launch_quant_x8_group(const QuantJobs& q, hipStream_t s) {
  if (q.n < 1 || q.n > MAX_GROUP) return hipErrorInvalidValue;
  int blocks = 0;
  for (int i = 0; i < q.n; ++i) {
    if (q.nb[i] < 1 || q.b0[i] != blocks) return hipErrorInvalidValue;
    blocks += (q.nb[i] + 7) / 8;
  }
  hipLaunchKernelGGL(k_quant_x8_group, dim3(blocks), dim3(256), 0, s, q);
  return hipGetLastError();
}

// One tile's int8-activation GEMV from a symbol source (table entries from decode_table_i8): per sub-block an
// integer dot product of the int8 grid values with the quantized x (v_dot4_i32_i8, 4 weights per step), then
// y += s d_x acc - o s_x with s = d sc, o = dmin m per sub-block and d_x, s_x of the sub-block's 32-block.
// xq4 = the tile column's quantized x as 4-byte words, dx / sx its 32-block scales (scalar loads).
// MT > 1 (the reference's MT-token kernel, kernels/llmrt.cu:1057-1169): tokens j < mt in one pass over the codes;
// token j's x lies xw words (xq4) and xb blocks (dx, sx) after token 0's and its partial at out + j ostride. A
// group's 8 pairs are decoded into 8 (4-bit formats) or 4 (8-bit formats) words of 4 grid bytes, then each token
// takes them in pair order: every token gets the operations, in the same order, of an m = 1 pass.
template <int KQ, int MT = 1, class Src>
__device__ __forceinline__ void tile_gemv_i8(Src& src, __attribute__((address_space(4))) const uint32_t* xq4,
                                             __attribute__((address_space(4))) const float* dx,
                                             __attribute__((address_space(4))) const float* sx,
                                             const uint8_t* srow, float* out, int mt = 1, int xw = 0, int xb = 0,
                                             int ostride = 0) {
  constexpr int SYMB = kq_symbits(KQ);
  constexpr int TW = SYMB == 4 ? 2 * TK : TK;
  constexpr int GW = kq_gw(KQ), SB = kq_sbytes(KQ);
  constexpr int NSB = TW / 256, GPS = 16 / NSB, NSUB = 256 / GW, GPSUB = GPS / NSUB;
  constexpr int NW = SYMB == 4 ? 8 : 4;  // words of 4 grid bytes per 16-symbol group
  float tot[MT];
  int acc[MT];
#pragma unroll
  for (int j = 0; j < MT; ++j) tot[j] = 0.f;
#pragma unroll 1
  for (int sb = 0; sb < NSB; ++sb) {
    uint32_t sw[5];
    side_load<KQ>(srow + sb * (TN * SB), sw);
    float dA, dB, mf[8];
    uint64_t scq, scq2;
    side_packed<KQ>(sw, scq, scq2, dA, dB);
    if (KQ == KQ_Q4_K || KQ == KQ_Q5_K) side_mins(sw, mf);
#pragma unroll
    for (int j = 0; j < MT; ++j) acc[j] = 0;
    uint32_t wprev = 0;
#pragma unroll 1
    for (int gg2 = 0; gg2 < GPS; gg2 += 2) {
      if (KQ == KQ_Q6_K && gg2 == 8) scq = scq2;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int g = sb * GPS + gg2 + h;
        src.stage(g);
        if (MT == 1) {
#pragma unroll 8
          for (int p = 0; p < 8; ++p) {
            uint32_t e1, e2;
            src.pair(p, e1, e2);
            if (SYMB == 4) {
              acc[0] = __builtin_amdgcn_sdot4((int)__builtin_amdgcn_perm(e2, e1, 0x07060302u), (int)xq4[8 * g + p],
                                              acc[0], false);
            } else {
              const uint32_t w2 = __builtin_amdgcn_perm(e2, e1, 0x0C0C0602u);  // f(q1), f(q2) in bytes 0, 1
              if (p & 1) acc[0] = __builtin_amdgcn_sdot4((int)(wprev | (w2 << 16)), (int)xq4[4 * g + p / 2], acc[0], false);
              else wprev = w2;
            }
          }
        } else {
          uint32_t wv[NW];
#pragma unroll
          for (int p = 0; p < 8; ++p) {
            uint32_t e1, e2;
            src.pair(p, e1, e2);
            if (SYMB == 4) {
              wv[p] = __builtin_amdgcn_perm(e2, e1, 0x07060302u);
            } else {
              const uint32_t w2 = __builtin_amdgcn_perm(e2, e1, 0x0C0C0602u);
              if (p & 1) wv[p / 2] = wprev | (w2 << 16);
              else wprev = w2;
            }
          }
          // the tokens' x walk from token 0's by xw words; the stride is made opaque here so that the compiler does
          // not keep MT precomputed addresses live across the loop (they would not fit the scalar registers)
          int xws = xw;
          asm volatile("" : "+s"(xws));
          __attribute__((address_space(4))) const uint32_t* xj = xq4 + NW * g;
#pragma unroll
          for (int j = 0; j < MT; ++j) {
            if (j < mt) {
#pragma unroll
              for (int q = 0; q < NW; ++q) acc[j] = __builtin_amdgcn_sdot4((int)wv[q], (int)xj[q], acc[j], false);
            }
            xj += xws;
          }
        }
        if (GPSUB == 1 || h == 1) {  // sub-block end
          const int jj = (gg2 + h) / GPSUB, b = (sb * 256 + jj * GW) / 32;
          const float scv = (KQ == KQ_Q6_K || KQ == KQ_IQ4_XS) ? (float)(int)(int8_t)(uint8_t)scq
                                                               : (float)(uint32_t)(scq & 255u);
          scq >>= 8;
          int xbs = xb;
          if (MT > 1) asm volatile("" : "+s"(xbs));
          __attribute__((address_space(4))) const float *dj = dx + b, *sj = sx + b;
#pragma unroll
          for (int j = 0; j < MT; ++j) {
            if (j < mt) {
              tot[j] = fmaf(dA * scv * dj[0], (float)acc[j], tot[j]);
              if (KQ == KQ_Q4_K || KQ == KQ_Q5_K) tot[j] = fmaf(-(dB * mf[jj]), sj[0], tot[j]);
              acc[j] = 0;
            }
            dj += xbs;
            sj += xbs;
          }
        }
      }
    }
  }
#pragma unroll
  for (int j = 0; j < MT; ++j)
    if (j < mt) __hip_atomic_store(out + (size_t)j * ostride, tot[j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ── packed (fixed-rate) twin: decode-free fused GEMV / skinny GEMM ─────────────────────────────────────────
// The control the reference keeps beside its coded bundles (enc pk4 / pk8, kernels/llmrt.cu:538-630, 1731-1777):
// the same codes stored as plain bytes, so the kernel reads 4 (pk4) or 8 (pk8) bits per weight instead of the
// Huffman stream and runs no decode chain. Block = 16 waves = 16 tile rows of one tile column (as k_fused_ring), x
// staged in LDS for m > 1; tile_gemv with the packed source gives the coded path's bits.
template <int KQ, int MT>
__global__ void __launch_bounds__(1024, MT <= 2 ? 2 : 1) k_fused_packed(GroupPlan plan) {
  constexpr int WPB = 16;
  constexpr int SYMB = kq_symbits(KQ);
  constexpr int TW = SYMB == 4 ? 2 * TK : TK;
  constexpr int GW = kq_gw(KQ), NG = TW / GW, SB = kq_sbytes(KQ), NPAIR = TW / 2;
  constexpr int NTHR = WPB * 64;
  __shared__ uint32_t tab[256];
  extern __shared__ __align__(16) uint32_t smem[];
  uint32_t* xs = smem;                                    // [NPAIR][MT] fp16 pairs (xs_index)
  float* xg = reinterpret_cast<float*>(xs + NPAIR * MT);  // [NG][MT] sub-block sums of x
  uint4* rings = reinterpret_cast<uint4*>(smem + ((NPAIR + NG) * MT + 3) / 4 * 4);  // WPB x PK_SLOTS x 64 chunks
  int mi = 0;
#pragma unroll
  for (int i = 1; i < MAX_GROUP; ++i)
    if (i < plan.n && (int)blockIdx.x >= plan.e[i].block0) mi = i;
  typedef __attribute__((address_space(4))) const char KChar;
  typedef __attribute__((address_space(4))) const GroupEntry KEntry;
  typedef __attribute__((address_space(4))) const uint32_t KU32;
  KChar* kbase = (KChar*)__builtin_amdgcn_kernarg_segment_ptr();
  KEntry* ep = (KEntry*)(kbase + offsetof(GroupPlan, e) + (size_t)mi * sizeof(GroupEntry));
  const auto& E = *ep;
  const auto& M = E.M;
  const int mt = plan.mt;
  const int bl = (int)blockIdx.x - E.block0;
  const int KT = M.KT, NT = M.NT, K = M.K, N = M.N;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int tc = bl % KT, tr = (bl / KT) * WPB + wave;
  const int lane = threadIdx.x & 63;
  if (threadIdx.x < 256) tab[threadIdx.x] = M.lut4[threadIdx.x];
  if (MT > 1) {
    for (int i = threadIdx.x; i < NPAIR * MT; i += NTHR) {
      const int j = i / NPAIR, c = i - j * NPAIR;
      xs[xs_index<MT>(c, j)] = j < mt ? E.X2[(size_t)j * (K / 2) + (size_t)tc * NPAIR + c] : 0u;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < NG * MT; i += NTHR) {
      const int g = i / MT, j = i - g * MT;
      xg[g * MT + j] = xsum_sub<GW>([&](int c) { return xs[xs_index<MT>(g * (GW / 2) + c, j)]; });
    }
  }
  __syncthreads();
  if (tr >= NT) return;
  const int t = tr * KT + tc;
  const uint8_t* srow = M.side + side_record(tr * TN, tc * (TW / 256), KT, TW / 256) * SB + (uint32_t)(lane * SB);
  KU32* xcol = (KU32*)(E.X2 + (size_t)tc * NPAIR);
  float* out = E.P + (size_t)tc * mt * N + (size_t)tr * TN + (uint32_t)lane;
  PackedSrc<KQ> src(reinterpret_cast<const uint4*>(M.words) + (size_t)t * 16 * 64 + (uint32_t)lane,
                    rings + wave * PK_SLOTS * 64, tab, (uint32_t)lane, E.X2 + (size_t)tc * NPAIR,
                    MT == 1 ? reinterpret_cast<uint32_t*>(rings + WPB * PK_SLOTS * 64) + wave * NPAIR : nullptr);
  if (MT == 1)
    tile_gemv<KQ, MT>(src, xs, column_xsums<KQ>(E.X2, tc, lane), xcol, srow, mt, N, out);
  else
    tile_gemv<KQ, MT>(src, xs, XgLds{xg, MT, 256 / GW}, xcol, srow, mt, N, out);
}

// One tile of a flat launch: fp16 activations, m = 1 (tile_gemv) or int8 activations (tile_gemv_i8, the entry's XQ /
// DX / SX for tile column tc; MT > 1: tokens j < mt, partials N apart)
template <int KQ, bool I8, int MT = 1, class Src, class KEntryRef>
__device__ __forceinline__ void tile_body(Src& src, const KEntryRef& E, int tc, const XgRegs& xgr,
                                          __attribute__((address_space(4))) const uint32_t* xcol, const uint8_t* srow,
                                          int N, float* out, int mt = 1) {
  constexpr int TW = kq_symbits(KQ) == 4 ? 2 * TK : TK;
  typedef __attribute__((address_space(4))) const uint32_t KU32;
  typedef __attribute__((address_space(4))) const float KF32;
  if (I8) {
    // tc and K are wave-uniform: said so, the tokens' x addresses stay in scalar registers
    const int tcu = __builtin_amdgcn_readfirstlane(tc), K = MT > 1 ? __builtin_amdgcn_readfirstlane(E.M.K) : 0;
    tile_gemv_i8<KQ, MT>(src, (KU32*)(E.XQ + (size_t)tcu * TW), (KF32*)(E.DX + (size_t)tcu * (TW / 32)),
                         (KF32*)(E.SX + (size_t)tcu * (TW / 32)), srow, out, mt, K / 4, K / 32, N);
  } else
    tile_gemv<KQ, 1, true>(src, nullptr, xgr, xcol, srow, 1, N, out);
}

// The packed twin for m = 1 over a flat tile list, as k_fused_flat: block b decodes tiles [b W, b W + W), one per
// wave, x through the scalar cache, the reduction over tile columns in the launch. A block spans at most two
// matrices: both symbol tables sit in LDS.
template <int KQ, bool I8>
__global__ void __launch_bounds__(1024) k_fused_packed_flat(FlatPlan plan) {
  constexpr int SYMB = kq_symbits(KQ);
  constexpr int TW = SYMB == 4 ? 2 * TK : TK;
  constexpr int SB = kq_sbytes(KQ), NPAIR = TW / 2;
  __shared__ uint32_t tab[2 * 256];
  extern __shared__ __align__(16) uint4 pk_rings[];  // W x PK_SLOTS x 64 chunks, then W x the column's x pairs
  typedef __attribute__((address_space(4))) const char KChar;
  typedef __attribute__((address_space(4))) const FlatEntry KEntry;
  typedef __attribute__((address_space(4))) const uint32_t KU32;
  KChar* kbase = (KChar*)__builtin_amdgcn_kernarg_segment_ptr();
  const int W = plan.W, T0 = (int)blockIdx.x * W, Tl = min(T0 + W, plan.ntiles) - 1;
  int ma = 0, mb = 0;
#pragma unroll
  for (int i = 1; i < MAX_GROUP; ++i) {
    if (i < plan.n && T0 >= plan.e[i].tile0) ma = i;
    if (i < plan.n && Tl >= plan.e[i].tile0) mb = i;
  }
  KEntry* ea = (KEntry*)(kbase + offsetof(FlatPlan, e) + (size_t)ma * sizeof(FlatEntry));
  KEntry* eb = (KEntry*)(kbase + offsetof(FlatPlan, e) + (size_t)mb * sizeof(FlatEntry));
  // the tables (blocks of W = 1..16 waves: any number of threads)
  for (int i = threadIdx.x; i < 256; i += W * 64) {
    tab[i] = (I8 ? ea->M.luti8 : ea->M.lut4)[i];
    if (mb != ma) tab[256 + i] = (I8 ? eb->M.luti8 : eb->M.lut4)[i];
  }
  __syncthreads();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int T = T0 + wave;
  if (T >= plan.ntiles) return;
  const bool second = mb != ma && T >= eb->tile0;
  KEntry* ep = second ? eb : ea;
  const auto& E = *ep;
  const auto& M = E.M;
  const int KT = M.KT, NT = M.NT, N = M.N;
  const int u = T - E.tile0;
  const int t = (u % NT) * KT + u / NT;
  const int tc = t % KT, tr = t / KT;
  const int lane = threadIdx.x & 63;
  XgRegs xgr;
  if (!I8) xgr = column_xsums<KQ>(E.X2, tc, lane);
  KU32* xcol = (KU32*)(E.X2 + (size_t)tc * NPAIR);
  const uint8_t* srow = M.side + side_record(tr * TN, tc * (TW / 256), KT, TW / 256) * SB + (uint32_t)(lane * SB);
  float* out = E.P + (size_t)tc * N + (size_t)tr * TN + (uint32_t)lane;
  // int8 activations: x through the scalar cache (tile_gemv_i8), nothing staged
  uint32_t* xw = I8 ? nullptr : reinterpret_cast<uint32_t*>(pk_rings + W * PK_SLOTS * 64) + wave * NPAIR;
  PackedSrc<KQ> src(reinterpret_cast<const uint4*>(M.words) + (size_t)t * 16 * 64 + (uint32_t)lane,
                    pk_rings + wave * PK_SLOTS * 64, tab + (second ? 256 : 0), (uint32_t)lane,
                    E.X2 + (size_t)tc * NPAIR, xw);
  tile_body<KQ, I8>(src, E, tc, xgr, xcol, srow, N, out);
  row_reduce(E, tr, KT, N, lane);
}

// ── ring kernel over a flat tile list (m = 1): balanced blocks ───────────────────────────────────────────
// One tile of the flat kernel: lanes of front f stage into `ring` (RS rows of 32 words).
template <int KQ, bool I8, int MT, class KEntryRef>
__device__ __forceinline__ void flat_tile(const KEntryRef& E, int t, const uint4& sc, uint32_t* ring, uint32_t rmask,
                                          const uint32_t* lut4, uint32_t lutsel, const XgRegs& xgr, int lane,
                                          int mt) {
  constexpr int SYMB = kq_symbits(KQ);
  constexpr int TW = SYMB == 4 ? 2 * TK : TK;
  constexpr int NPAIR = TW / 2;
  typedef __attribute__((address_space(4))) const uint32_t KU32;
  const auto& M = E.M;
  const int KT = M.KT, N = M.N, tc = t % KT, tr = t / KT;
  const int l = lane & 31, f = lane >> 5;
  KU32* xcol = (KU32*)(E.X2 + (size_t)tc * NPAIR);
  const int base_f = f ? (int)(sc.z & 255u) : 0;
  const uint2* src = reinterpret_cast<const uint2*>(M.words + M.tbase[t]) + (uint32_t)(16 * base_f + l);
  uint2* lane_slot = reinterpret_cast<uint2*>(ring) + (l >> 4) * 16 + (l & 15);
  const uint32_t P = (f ? (uint32_t)M.mid[(size_t)t * 32 + (uint32_t)l] - GUARD_BITS : 0u) - 32u * (uint32_t)base_f + 64u;
  uint32_t rlb = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint32_t*)(ring + l);
  asm volatile("" : "+v"(rlb));
  const uint8_t* srow = M.side + side_record(tr * TN, tc * (TW / 256), KT, TW / 256) * kq_sbytes(KQ) +
                        (uint32_t)((f * 32 + l) * kq_sbytes(KQ));
  float* out = E.P + (size_t)tc * mt * N + (size_t)tr * TN + (uint32_t)(f * 32 + l);
  const uint32_t init0 = (sc.z >> 8) & 255u, init1 = (sc.z >> 16) & 255u;
  if (sc.x == sc.y && init0 == init1) {  // one schedule for both fronts: scalar staging
    RingStager<int, uint32_t> st;
    st.lane_slot = lane_slot;
    st.src = src;
    st.counts = sc.x;
    st.rmask = rmask;
    st.init((int)init0);
    RingSrc<RingStager<int, uint32_t>> src(st, lut4, lutsel, P, rlb);
    tile_body<KQ, I8, MT>(src, E, tc, xgr, xcol, srow, N, out, mt);
  } else {
    RingStager<int, uint32_t> st;
    st.lane_slot = lane_slot;
    st.src = src;
    st.counts = f ? sc.y : sc.x;
    st.rmask = rmask;
    st.init((int)(f ? init1 : init0));
    RingSrc<RingStager<int, uint32_t>> src(st, lut4, lutsel, P, rlb);
    tile_body<KQ, I8, MT>(src, E, tc, xgr, xcol, srow, N, out, mt);
  }
  row_reduce(E, tr, KT, N, lane, mt);
}

// The tiles of the plan's matrices form one list (matrix by matrix, each column-major: tile rows of one tile
// column are consecutive) and block b decodes tiles [b W, b W + W), one per wave. W is chosen so that every CU gets
// the same number of waves (the block-per-column kernel leaves a third of the CUs at half load for a Mistral
// layer). A block spans at most two matrices (W <= the smallest matrix's tile count): both decode tables sit in LDS
// (slot 0, slot 1) and a wave ORs its slot into every table index. Activations come through the scalar cache; each
// wave sums its column's x per sub-block itself.
// Exception tiles (no 16-row schedule) are skipped, except with plan.nspare > 0 in a 16-row launch: then a tile
// with a 32-row schedule is decoded in place, front 0 in the wave's own two rings (4 KB) and front 1 in spare ring
// k of the block, k = the number of such tiles before it in the block (the host sizes nspare to the block maximum).
// MT > 1 (int8 activations only; 4 for up to 4 tokens, 8 for up to 8): tokens j < plan.mt in one pass, partials
// [KT][mt][N].
template <int KQ, int RS, int NTAB, bool I8, int MT = 1>
__global__ void __launch_bounds__(1024, MT == 4 ? 7 : (MT == 8 ? 1 : 2)) k_fused_flat(FlatPlan plan) {
  constexpr int SYMB = kq_symbits(KQ);
  constexpr int TW = SYMB == 4 ? 2 * TK : TK;
  constexpr int GW = kq_gw(KQ);
  static_assert(RS == 16 || RS == 32, "ring of 16 or 32 rows");
  constexpr int RING_WORDS = RS * 32;
  __shared__ uint32_t lut4[NTAB * LUTN];             // NTAB = 1: every block holds one matrix (W = 1 launches)
  extern __shared__ __align__(16) uint32_t rings[];  // (W + nspare) x 2 fronts x RS rows

  typedef __attribute__((address_space(4))) const char KChar;
  typedef __attribute__((address_space(4))) const FlatEntry KEntry;
  KChar* kbase = (KChar*)__builtin_amdgcn_kernarg_segment_ptr();
  const int W = plan.W, T0 = (int)blockIdx.x * W, Tl = min(T0 + W, plan.ntiles) - 1;
  int ma = 0, mb = 0;
#pragma unroll
  for (int i = 1; i < MAX_GROUP; ++i) {
    if (i < plan.n && T0 >= plan.e[i].tile0) ma = i;
    if (i < plan.n && Tl >= plan.e[i].tile0) mb = i;
  }
  KEntry* ea = (KEntry*)(kbase + offsetof(FlatPlan, e) + (size_t)ma * sizeof(FlatEntry));
  KEntry* eb = (KEntry*)(kbase + offsetof(FlatPlan, e) + (size_t)mb * sizeof(FlatEntry));
  const int NTHR = blockDim.x;
  const uint4* ta = reinterpret_cast<const uint4*>(I8 ? ea->M.luti8 : ea->M.lut4);
  const uint4* tb = reinterpret_cast<const uint4*>(I8 ? eb->M.luti8 : eb->M.lut4);
  for (int i = threadIdx.x; i < LUTN / 4; i += NTHR) reinterpret_cast<uint4*>(lut4)[i] = ta[i];
  if (NTAB > 1 && mb != ma)
    for (int i = threadIdx.x; i < LUTN / 4; i += NTHR) reinterpret_cast<uint4*>(lut4 + LUTN)[i] = tb[i];
  __syncthreads();

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int T = T0 + wave;
  if (T >= plan.ntiles) return;
  const int tile0b = eb->tile0;
  const bool second = mb != ma && T >= tile0b;
  KEntry* ep = second ? eb : ea;
  const auto& E = *ep;
  const auto& M = E.M;
  const uint32_t lutsel = second ? (uint32_t)(LUTN * 4) : 0u;
  const int KT = M.KT, NT = M.NT;
  const int u = T - E.tile0;
  // wave-uniform (one tile per wave): said so, the tile's addresses and schedule stay in scalar registers
  const int t = __builtin_amdgcn_readfirstlane(E.list ? (int)E.list[u] : (u % NT) * KT + u / NT);
  const int tc = t % KT;
  const int lane = threadIdx.x & 63;
  const uint4 sc0 = M.sched[t];
  const uint4 sc = make_uint4(__builtin_amdgcn_readfirstlane(sc0.x), __builtin_amdgcn_readfirstlane(sc0.y),
                              __builtin_amdgcn_readfirstlane(sc0.z), __builtin_amdgcn_readfirstlane(sc0.w));
  int spare = -1;
  if (!E.list && (sc.w & 1u)) {  // exception tile
    if (RS != 16 || !plan.nspare || !(sc.w & 2u)) return;  // decoded by the exception pass
    spare = 0;
    for (int q = T0; q < T; ++q) {  // 32-row exception tiles earlier in this block
      const bool qs = mb != ma && q >= tile0b;
      KEntry* eq = qs ? eb : ea;
      const int uq = q - eq->tile0, NTq = eq->M.NT, KTq = eq->M.KT;
      const uint32_t wq = reinterpret_cast<const uint32_t*>(eq->M.sched)[4 * ((uq % NTq) * KTq + uq / NTq) + 3];
      spare += (wq & 3u) == 3u;
    }
    if (spare >= plan.nspare) return;  // cannot happen with the host's sizing; never overrun the spare rings
  }

  XgRegs xgr;
  if (!I8) xgr = column_xsums<KQ>(E.X2, tc, lane);

  // the ring of the lane's front: 16-row launches place a 32-row exception tile's front 0 in the wave's two rings
  // and its front 1 in spare ring pair `spare`
  const int f = lane >> 5;
  const bool x32 = RS == 16 && spare >= 0;
  uint32_t* ring = rings + (x32 ? (f ? 2 * W + 2 * spare : 2 * wave) : 2 * wave + f) * RING_WORDS;
  flat_tile<KQ, I8, MT>(E, t, sc, ring, x32 ? 31u : (uint32_t)(RS - 1), lut4, lutsel, xgr, lane, MT == 1 ? 1 : plan.mt);
}

// ── low-latency kernel (m = 1): one tile per block, 8 chains per lane ───────────────────────────────────
// A launch of few tiles per CU takes about one tile's decode time, whatever its size: the chain of 128 dependent
// symbol pairs per lane front. Here a block of 4 waves stages its whole tile in LDS and splits every lane stream
// into 8 chains of 64 symbols at load-time offsets (Layout::split): wave w decodes symbols [64 w, 64 w + 64) of
// both rows of every lane (lanes 0-31 row l, lanes 32-63 row l + 32, the same x columns), with the ring kernel's
// register window reading the tile image directly. Each chain stores its sub-block dot products in LDS; wave 0
// then forms each row's partial exactly as tile_gemv does (same operations in the same order), so the result has
// the same bits as the ring kernels'. Exception tiles need nothing special: no staging schedule is involved.
// MT > 1 (int8 activations only): tokens j < plan.mt in one pass (chain dot products per token), partials
// [KT][mt][N].
template <int KQ, bool I8, int MT = 1>
__global__ void __launch_bounds__(256) k_fused_split(FlatPlan plan, int stage_rows) {
  constexpr int SYMB = kq_symbits(KQ);
  constexpr int TW = SYMB == 4 ? 2 * TK : TK;
  constexpr int GW = kq_gw(KQ), SB = kq_sbytes(KQ);
  constexpr int NSUBT = TW / GW;                  // sub-blocks per tile row
  constexpr int NSB = TW / 256;                   // super-blocks per tile row
  constexpr int NSUB = 256 / GW;                  // sub-blocks per super-block
  constexpr int GPSUB = (GW / (SYMB == 4 ? 2 : 1)) / 16;  // 16-symbol groups per sub-block (2 for Q5_K, else 1)
  constexpr float VSCALE = SYMB == 4 ? 16777216.f : 1.f;
  typedef __attribute__((address_space(3))) const uint32_t LdsU32;
  // one static LDS object, so the table sits at LDS address 0 (table_addr ORs its base into the index bits)
  __shared__ uint32_t lds_static[LUTN + TN * NSUBT * MT];
  uint32_t* lut4 = lds_static;
  float* accb = reinterpret_cast<float*>(lds_static + LUTN);  // [row][sub-block][token] dot products of the chains
  const int mt = MT == 1 ? 1 : plan.mt;
  extern __shared__ __align__(16) uint32_t tw[];              // the tile's word rows [stage_rows][32]

  typedef __attribute__((address_space(4))) const char KChar;
  typedef __attribute__((address_space(4))) const FlatEntry KEntry;
  typedef __attribute__((address_space(4))) const uint32_t KU32;
  KChar* kbase = (KChar*)__builtin_amdgcn_kernarg_segment_ptr();
  const int T = (int)blockIdx.x;
  int mi = 0;
#pragma unroll
  for (int i = 1; i < MAX_GROUP; ++i)
    if (i < plan.n && T >= plan.e[i].tile0) mi = i;
  KEntry* ep = (KEntry*)(kbase + offsetof(FlatPlan, e) + (size_t)mi * sizeof(FlatEntry));
  const auto& E = *ep;
  const auto& M = E.M;
  const int KT = M.KT, NT = M.NT, N = M.N;
  const int u = T - E.tile0;
  const int t = E.list ? (int)E.list[u] : (u % NT) * KT + u / NT;
  const int tc = t % KT, tr = t / KT;
  const int R = min((int)M.rows[t] + 2, stage_rows);  // rows read: up to 2 past the longest lane's last row
  const uint4* tab = reinterpret_cast<const uint4*>(I8 ? M.luti8 : M.lut4);
  for (int i = threadIdx.x; i < LUTN / 4; i += 256) reinterpret_cast<uint4*>(lut4)[i] = tab[i];
  const uint4* src = reinterpret_cast<const uint4*>(M.words + M.tbase[t]);
  for (int i = threadIdx.x; i < 8 * R; i += 256) reinterpret_cast<uint4*>(tw)[i] = src[i];
  __syncthreads();

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63, l = lane & 31, f = lane >> 5;
  // wave 0 forms the row partials after the decode: its side records and x sums are fetched first, so their
  // latency hides behind the decode
  const uint8_t* srow = M.side + side_record(tr * TN, tc * NSB, KT, NSB) * SB + (uint32_t)(lane * SB);
  uint32_t sw[NSB][5];
  XgRegs xgr;
  if (wave == 0) {
#pragma unroll
    for (int sb = 0; sb < NSB; ++sb) side_load<KQ>(srow + sb * (TN * SB), sw[sb]);
    if (!I8) xgr = column_xsums<KQ>(E.X2, tc, lane);
  }
  {
    // chain of lane front f: symbols [64 wave, 64 wave + 64) of row l + 32 f, i.e. stream symbols 256 f + 64 wave..
    const int k = 4 * f + wave;
    uint32_t P = (uint32_t)M.split[((size_t)t * SPLITS + k * (SPLITS / 8)) * 32 + (uint32_t)l] - GUARD_BITS + 64u;
    const uint32_t tsel = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const uint32_t*)lut4;
    uint32_t tmask = 0x1FFCu;
    asm volatile("" : "+v"(tmask));
    uint32_t rlb = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint32_t*)(tw + l);
    asm volatile("" : "+v"(rlb));
    KU32* xcol = (KU32*)(E.X2 + (size_t)tc * (TW / 2));
    KU32* xq4 = (KU32*)(E.XQ + (size_t)__builtin_amdgcn_readfirstlane(tc) * TW);
    uint32_t slot = __builtin_amdgcn_ubfe(P, 5, 8);
    uint32_t A = *(LdsU32*)(rlb + ((slot - 2u) << 7));
    uint32_t B = *(LdsU32*)(rlb + ((slot - 1u) << 7));
    uint32_t C = *(LdsU32*)(rlb + (slot << 7));
    float* accrow = accb + (f * 32 + l) * NSUBT * MT;
    float acc = 0.f;
    int iacc = 0, iaccm[MT];
#pragma unroll
    for (int j = 0; j < MT; ++j) iaccm[j] = 0;
    constexpr int NW = SYMB == 4 ? 8 : 4;  // MT > 1: words of 4 grid bytes per group, as tile_gemv_i8
    uint32_t wprev = 0, wv[NW];
#pragma unroll 1
    for (int gi = 0; gi < 4; ++gi) {
      const int g = 4 * wave + gi;  // 16-symbol group within the row
#pragma unroll
      for (int p = 0; p < 8; ++p) {
        const uint32_t w1 = __builtin_amdgcn_alignbit(B, A, P);
        const uint32_t e1 = *(LdsU32*)table_addr(w1, tsel, tmask);
        const uint32_t w2 = w1 >> (e1 & 31u);
        const uint32_t e2 = *(LdsU32*)table_addr(w2, tsel, tmask);
        P = P + e1 + e2;
        const uint32_t nslot = __builtin_amdgcn_ubfe(P, 5, 8);
        const bool slide = nslot != slot;
        A = slide ? B : A;
        B = slide ? C : B;
        slot = nslot;
        C = *(LdsU32*)(rlb + (nslot << 7));
        if (I8 && MT > 1) {
          if (SYMB == 4) {
            wv[p] = __builtin_amdgcn_perm(e2, e1, 0x07060302u);
          } else {
            const uint32_t w2 = __builtin_amdgcn_perm(e2, e1, 0x0C0C0602u);
            if (p & 1) wv[p / 2] = wprev | (w2 << 16);
            else wprev = w2;
          }
        } else if (I8) {  // as tile_gemv_i8
          if (SYMB == 4) {
            iacc = __builtin_amdgcn_sdot4((int)__builtin_amdgcn_perm(e2, e1, 0x07060302u), (int)xq4[8 * g + p], iacc, false);
          } else {
            const uint32_t w2 = __builtin_amdgcn_perm(e2, e1, 0x0C0C0602u);
            if (p & 1) iacc = __builtin_amdgcn_sdot4((int)(wprev | (w2 << 16)), (int)xq4[4 * g + p / 2], iacc, false);
            else wprev = w2;
          }
        } else if (SYMB == 4) {
          const uint32_t v1 = __builtin_amdgcn_perm(e1, e1, 0x0C030C02u), v2 = __builtin_amdgcn_perm(e2, e2, 0x0C030C02u);
          const int c = 16 * g + 2 * p;
          acc = dot2(v2, xcol[c + 1], dot2(v1, xcol[c], acc));
        } else {
          const uint32_t w = __builtin_amdgcn_perm(e2, e1, 0x07060302u);
          acc = dot2(w, xcol[8 * g + p], acc);
        }
      }
      if (I8 && MT > 1) {
#pragma unroll
        for (int j = 0; j < MT; ++j)
          if (j < mt) {
            KU32* xj = xq4 + (size_t)j * (uint32_t)(__builtin_amdgcn_readfirstlane(M.K) / 4) + NW * g;
#pragma unroll
            for (int q = 0; q < NW; ++q) iaccm[j] = __builtin_amdgcn_sdot4((int)wv[q], (int)xj[q], iaccm[j], false);
          }
      }
      if (GPSUB == 1 || (gi & 1)) {
        if (I8 && MT > 1) {
#pragma unroll
          for (int j = 0; j < MT; ++j) {
            accrow[(g / GPSUB) * MT + j] = (float)iaccm[j];
            iaccm[j] = 0;
          }
        } else {
          accrow[g / GPSUB] = I8 ? (float)iacc : acc;  // |iacc| < 2^24: exact
        }
        acc = 0.f;
        iacc = 0;
      }
    }
  }
  __syncthreads();
  if (wave != 0) return;

  // row partials, as tile_gemv forms them: per super-block the min / bias term first, then d x the scaled sum of
  // the sub-block dot products in order
  const float* accrow = accb + lane * NSUBT * MT;
  float tot = 0.f;
  if (I8) {  // tile_gemv_i8's order: per sub-block s d_x acc, then - o s_x; token by token
    typedef __attribute__((address_space(4))) const float KF32;
#pragma unroll 1
    for (int j = 0; j < mt; ++j) {
      KF32* dx = (KF32*)(E.DX + (size_t)j * (M.K / 32) + (size_t)tc * (TW / 32));
      KF32* sx = (KF32*)(E.SX + (size_t)j * (M.K / 32) + (size_t)tc * (TW / 32));
      tot = 0.f;
#pragma unroll
      for (int sb = 0; sb < NSB; ++sb) {
        float dA, dB, mf[8];
        uint64_t scq, scq2;
        side_packed<KQ>(sw[sb], scq, scq2, dA, dB);
        if (KQ == KQ_Q4_K || KQ == KQ_Q5_K) side_mins(sw[sb], mf);
#pragma unroll
        for (int jj = 0; jj < NSUB; ++jj) {
          if (KQ == KQ_Q6_K && jj == 8) scq = scq2;
          const float scv = (KQ == KQ_Q6_K || KQ == KQ_IQ4_XS) ? (float)(int)(int8_t)(uint8_t)scq
                                                               : (float)(uint32_t)(scq & 255u);
          scq >>= 8;
          const int xb = (sb * 256 + jj * GW) / 32;
          tot = fmaf(dA * scv * dx[xb], accrow[(sb * NSUB + jj) * MT + (MT > 1 ? j : 0)], tot);
          if (KQ == KQ_Q4_K || KQ == KQ_Q5_K) tot = fmaf(-(dB * mf[jj]), sx[xb], tot);
        }
      }
      if (j + 1 < mt)
        __hip_atomic_store(E.P + ((size_t)tc * mt + j) * N + (size_t)tr * TN + (uint32_t)lane, tot, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    }
  }
#pragma unroll
  for (int sb = 0; !I8 && sb < NSB; ++sb) {
    float dA, dB;
    uint64_t scq, scq2;
    side_packed<KQ>(sw[sb], scq, scq2, dA, dB);
    if (KQ == KQ_Q4_K || KQ == KQ_Q5_K) {
      float mf[8], msum = 0.f;
      side_mins(sw[sb], mf);
#pragma unroll
      for (int jj = 0; jj < NSUB; ++jj) msum = fmaf(mf[jj], xgr(sb, jj, 0), msum);
      tot = fmaf(-dB, msum, tot);
    }
    if (KQ == KQ_IQ4_XS) {
      float csum = 0.f;
#pragma unroll
      for (int jj = 0; jj < NSUB; ++jj) csum = fmaf((float)(int)(int8_t)(uint8_t)(scq >> (8 * jj)), xgr(sb, jj, 0), csum);
      tot = fmaf(-128.f * dA, csum, tot);
    }
    float tsum = 0.f;
#pragma unroll
    for (int jj = 0; jj < NSUB; ++jj) {
      if (KQ == KQ_Q6_K && jj == 8) scq = scq2;
      const float scv = (KQ == KQ_Q6_K || KQ == KQ_IQ4_XS) ? (float)(int)(int8_t)(uint8_t)scq
                                                           : (float)(uint32_t)(scq & 255u);
      scq >>= 8;
      tsum = fmaf(scv, accrow[sb * NSUB + jj], tsum);
    }
    tot = fmaf(dA * VSCALE, tsum, tot);
  }
  float* out = E.P + ((size_t)tc * mt + (mt - 1)) * N + (size_t)tr * TN + (uint32_t)lane;  // the last token's
  __hip_atomic_store(out, tot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  row_reduce(E, tr, KT, N, lane, mt);
}

template <int KQ, bool I8, int MT = 1>
static hipError_t split_launch_t(const FlatPlan& p, int stage_rows, hipStream_t s) {
  const size_t smem = (size_t)stage_rows * 128;
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_fused_split<KQ, I8, MT>),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((k_fused_split<KQ, I8, MT>), dim3(p.ntiles), dim3(256), smem, s, p, stage_rows);
  return hipGetLastError();
}

template <int KQ>
static hipError_t split_launch(const FlatPlan& p, int stage_rows, hipStream_t s) {
  if (p.mt > 4) return split_launch_t<KQ, true, 8>(p, stage_rows, s);
  if (p.mt > 1) return split_launch_t<KQ, true, 4>(p, stage_rows, s);
  return p.i8 ? split_launch_t<KQ, true>(p, stage_rows, s) : split_launch_t<KQ, false>(p, stage_rows, s);
}

// the tokens of a flat plan: 0 / 1, or 2..8 with int8 activations (then every entry's Y needs ldy >= N)
static bool flat_tokens_ok(const FlatPlan& p) {
  if (p.mt < 0 || p.mt > 8 || (p.mt > 1 && !p.i8)) return false;
  for (int i = 0; p.mt > 1 && i < p.n; ++i)
    if (p.e[i].Y && p.e[i].ldy < p.e[i].M.N) return false;
  return true;
}

int split_stage_rows(const FlatPlan& p) {
  int r = 0;
  for (int i = 0; i < p.n; ++i) r = std::max(r, p.e[i].M.max_rows + 2);
  return r;
}

hipError_t launch_fused_split(const FlatPlan& p, hipStream_t s) {
  if (p.n < 1 || p.n > MAX_GROUP || p.ntiles < 1) return hipErrorInvalidValue;
  const int kqt = p.e[0].M.kqt;
  for (int i = 0; i < p.n; ++i) {
    const FlatEntry& e = p.e[i];
    const int end = i + 1 < p.n ? p.e[i + 1].tile0 : p.ntiles;
    if (e.M.kqt != kqt || !e.M.split || !e.M.lut4 || e.tile0 + e.ntile != end || e.ntile < 1 ||
        (!e.list && e.ntile != e.M.NT * e.M.KT) || (i == 0 && e.tile0 != 0) ||
        (p.i8 && (!e.M.luti8 || !e.XQ || !e.DX || !e.SX)))
      return hipErrorInvalidValue;
  }
  if (!flat_tokens_ok(p)) return hipErrorInvalidValue;
  const int rows = split_stage_rows(p);
  if (rows > 256 || rows * 128 + 4 * LUTN + TN * 16 * 4 * (p.mt > 1 ? 8 : 1) > 160 * 1024) return hipErrorInvalidValue;
  switch (kqt) {
    case KQ_Q4_K: return split_launch<KQ_Q4_K>(p, rows, s);
    case KQ_Q5_K: return split_launch<KQ_Q5_K>(p, rows, s);
    case KQ_Q6_K: return split_launch<KQ_Q6_K>(p, rows, s);
    case KQ_IQ4_XS: return split_launch<KQ_IQ4_XS>(p, rows, s);
    default: return hipErrorInvalidValue;
  }
}

// acc += dot2(x, w) with x = lane k of the lane's 16-lane row of xrow (DPP row_newbcast: x held the same in every
// row, so the broadcast costs no v_readlane). xrow comes from loads, so no VALU write precedes the DPP read; the
// compiler does not see the DPP inside the assembly, so the build disassembles its own code objects and refuses any
// DPP operation with fewer than the required wait states (lazyweights_amd/build.py, check_dpp_hazards). A form the
// compiler can see (update_dpp + fdot2) is not folded into one instruction: a v_mov_b32_dpp per product.
template <int K>
__device__ __forceinline__ void dot2_bcast(float& acc, uint32_t xrow, uint32_t w) {
  asm("v_dot2c_f32_f16_dpp %0, %1, %2 row_newbcast:%3 row_mask:0xf bank_mask:0xf bound_ctrl:1"
      : "+v"(acc)
      : "v"(xrow), "v"(w), "n"(K));
}
__device__ __forceinline__ void dot2_row(float& acc, uint32_t xrow, int k, uint32_t w) {
  switch (k) {  // k is a constant after unrolling
    case 0: dot2_bcast<0>(acc, xrow, w); break;
    case 1: dot2_bcast<1>(acc, xrow, w); break;
    case 2: dot2_bcast<2>(acc, xrow, w); break;
    case 3: dot2_bcast<3>(acc, xrow, w); break;
    case 4: dot2_bcast<4>(acc, xrow, w); break;
    case 5: dot2_bcast<5>(acc, xrow, w); break;
    case 6: dot2_bcast<6>(acc, xrow, w); break;
    case 7: dot2_bcast<7>(acc, xrow, w); break;
    case 8: dot2_bcast<8>(acc, xrow, w); break;
    case 9: dot2_bcast<9>(acc, xrow, w); break;
    case 10: dot2_bcast<10>(acc, xrow, w); break;
    case 11: dot2_bcast<11>(acc, xrow, w); break;
    case 12: dot2_bcast<12>(acc, xrow, w); break;
    case 13: dot2_bcast<13>(acc, xrow, w); break;
    case 14: dot2_bcast<14>(acc, xrow, w); break;
    default: dot2_bcast<15>(acc, xrow, w); break;
  }
}

// s_waitcnt vmcnt(n) for a wave-uniform n in [0, 63] (the count is an immediate: one wait per value; larger n wait
// for 63). The compiler does not see which value ran, so it still waits for every vector load whose result a later
// instruction reads; this is for loads whose results only LDS reads see (direct-to-LDS copies).
template <int N = 63>
__device__ __forceinline__ void wait_vmcnt_upto(int n) {
  if constexpr (N == 0) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  } else {
    if (n >= N) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
    else wait_vmcnt_upto<N - 1>(n);
  }
}

// The 8 chain starts (P form: bit position - GUARD_BITS + 64) of row f of lane stream s of tile t in the whole-tile
// kernels: the first at mid (f = 1) or the guard (f = 0), the others from the 9-bit deltas of dsplit.
template <class DevMatRef>
__device__ __forceinline__ void tile_chain_starts(const DevMatRef& M, int t, int f, int s, uint32_t* P) {
  const uint64_t d = M.dsplit[((size_t)t * 2 + f) * 32 + (uint32_t)s];
  const uint32_t mid = M.mid[(size_t)t * 32 + (uint32_t)s];
  P[0] = (f ? mid : (uint32_t)GUARD_BITS) - GUARD_BITS + 64u;
#pragma unroll
  for (int j = 1; j < 8; ++j) P[j] = P[j - 1] + 32u + (uint32_t)(d >> (9 * (j - 1)) & 511u);
}

// ── whole-tile kernel for flat launches (m = 1): a tile per wave, 8 chains per lane ───────────────────────
// the most tile copies a block of the whole-tile kernel keeps in flight (measured on config 2: 3-6 alike, 2-4 %
// faster than one per wave)
#ifndef LW_TILES_COPIES
#define LW_TILES_COPIES 4
#endif
constexpr int TILES_COPIES = LW_TILES_COPIES;
// Block = W waves sharing the decode tables; the block decodes tiles [T0, T0 + per) (spanning at most two
// matrices; a matrix's tiles in row-major order), wave w first tile T0 + w, then the next undecoded one from a
// counter in LDS, so each SIMD takes tiles at its own rate. The tables arrive by direct-to-LDS loads issued
// ahead of the waves' first tile copies, so a wave waits only for those before the block's barrier; at most
// TILES_COPIES copies are in flight per block. The next tile's copy is issued as soon as a decode ends, before
// the row partial is formed; the tiles' row counts and word offsets, read at that point, were brought into the
// scalar cache at the start (a wave's first copy of a fixed-stride matrix reads neither: it copies the tile's slot).
// A tile's word rows are copied whole into the wave's LDS buffer with direct-to-LDS loads (1 KB per instruction);
// lane l then decodes tile row l (lane stream l % 32, its row l / 32) as 8 chains of 32 symbols that start at the
// load-time split offsets and run interleaved instruction by instruction, so their LDS round trips overlap. A
// chain keeps its window rows in registers and reads one new row word per pair (per pair of symbols 2 table
// gathers, 1 row read and 14 VALU instructions; the gathers' bank conflicts and the VALU issue co-limit a tile).
// A tile row whose tiles are all the block's own is counted in LDS; the others in the entry's counter.
// There is no ring and no staging schedule: every tile of the matrices, exception tiles included, is decoded here.
// The lane keeps its row's sub-block dot products in registers and forms the row partial in tile_gemv's order
// (tile_gemv_i8's for int8 activations), the bits of the other kernels.
// (at most 16 waves per CU by the LDS of the tile buffers: 4 per SIMD, so the scheduler may spend up to 128 VGPRs on
// keeping the 8 chains' reads in flight)
// CANON (kernel mode 9, fp16 activations): codes are looked up by the comparator (canon_addr) in a 256-entry table
// of entries in canonical order instead of the 2048-entry table; the same entries, so the same bits. Its blocks have
// at most TILES_CANON_WAVES waves (3 per SIMD): the comparator's registers spill at 4.
// Diagnostic build only (-DLW_TIMELINE, lazyweights_amd.timeline): per-wave timestamps of the whole-tile kernel
// (s_memrealtime, 100 MHz) in g_timeline[block][wave][slot]: slot 0 the wave's start, 1 after the tables' barrier, 2
// its HW_ID register (SIMD and CU), 3 its end, and for its tile i < 8: 4 + 3 i the tile in LDS, 5 + 3 i its decode
// done, 6 + 3 i the next tile's copy issued. Lane 0 of each wave stores (vector stores); nothing else changes.
#ifdef LW_TIMELINE
constexpr int TL_BLOCKS = 1024, TL_WAVES = 16, TL_SLOTS = 32;
__device__ uint64_t g_timeline[TL_BLOCKS * TL_WAVES * TL_SLOTS];
__device__ __forceinline__ void tl_put(int k, uint64_t v) {
  if ((threadIdx.x & 63) == 0 && blockIdx.x < TL_BLOCKS && k < TL_SLOTS)
    g_timeline[((size_t)blockIdx.x * TL_WAVES + (threadIdx.x >> 6)) * TL_SLOTS + k] = v;
}
#define LW_TL(k) tl_put((k), __builtin_amdgcn_s_memrealtime())
#define LW_TL_HWID() tl_put(2, __builtin_amdgcn_s_getreg((4 << 0) | (0 << 6) | (31 << 11)))
#else
#define LW_TL(k) ((void)0)
#define LW_TL_HWID() ((void)0)
#endif

template <int V>
struct KqTag {
  static constexpr int value = V;
};
template <int KQA, int NTAB, bool I8, bool CANON = false, int KQB = KQA>
__global__ void __launch_bounds__(CANON ? 64 * TILES_CANON_WAVES : 1024, 1)
k_fused_tiles(FlatPlan plan, int per, int buf_rows) {
  constexpr int NC = 8;                                   // chains per lane (32 symbols each)
  constexpr int NG = 16 / NC;                             // 16-symbol groups per chain
  typedef __attribute__((address_space(3))) const uint32_t LdsU32;
  typedef __attribute__((address_space(4))) const char KChar;
  typedef __attribute__((address_space(4))) const FlatEntry KEntry;
  typedef __attribute__((address_space(4))) const uint32_t KU32;
  typedef __attribute__((address_space(4))) const float KF32;
  typedef __attribute__((address_space(4))) const uint16_t KU16;
  // one static LDS object at address 0, so the tables sit at 0 and 8 KB (table_addr ORs its base into the index);
  // the block's tile counter, copy counters and row counters after them
  __shared__ uint32_t lut4[NTAB * LUTN + 4 + TILES_ROWC];
  extern __shared__ __align__(16) uint32_t tbuf[];  // W x buf_rows word rows of 32 words

  KChar* kbase = (KChar*)__builtin_amdgcn_kernarg_segment_ptr();
  const int W = plan.W, T0 = (int)blockIdx.x * per, Tl = min(T0 + per, plan.ntiles) - 1;
  int ma = 0, mb = 0;
#pragma unroll
  for (int i = 1; i < MAX_GROUP; ++i) {
    if (i < plan.n && T0 >= plan.e[i].tile0) ma = i;
    if (i < plan.n && Tl >= plan.e[i].tile0) mb = i;
  }
  KEntry* ea = (KEntry*)(kbase + offsetof(FlatPlan, e) + (size_t)ma * sizeof(FlatEntry));
  KEntry* eb = (KEntry*)(kbase + offsetof(FlatPlan, e) + (size_t)mb * sizeof(FlatEntry));
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63, s = lane & 31, f = lane >> 5;
  LW_TL(0);
  LW_TL_HWID();
  int tl_i = 0;  // (the diagnostic timestamps' tile index)
  (void)tl_i;
  if (CANON) {  // the comparator tables' 256 entries: one 1 KB direct-to-LDS load per table, at the tables' places
    const uint4* ta = reinterpret_cast<const uint4*>(ea->M.canon + 32);
    const uint4* tb = reinterpret_cast<const uint4*>(eb->M.canon + 32);
    const int nchunk = (NTAB > 1 && mb != ma) ? 2 : 1;
    for (int c = wave; c < nchunk; c += W)
      __builtin_amdgcn_global_load_lds((c ? tb : ta) + lane, (__attribute__((address_space(3))) void*)(lut4 + LUTN * c),
                                       16, 0, 0);
  } else {  // the tables: 1 KB direct-to-LDS loads, chunk c (8 per table) by wave c mod W
    const uint4* ta = reinterpret_cast<const uint4*>(I8 ? ea->M.luti8 : ea->M.lut4);
    const uint4* tb = reinterpret_cast<const uint4*>(I8 ? eb->M.luti8 : eb->M.lut4);
    const int nchunk = (NTAB > 1 && mb != ma) ? 16 : 8;
    for (int c = wave; c < nchunk; c += W)
      __builtin_amdgcn_global_load_lds((c < 8 ? ta : tb) + 64 * (c & 7) + lane,
                                       (__attribute__((address_space(3))) void*)(lut4 + 256 * c), 16, 0, 0);
  }
  // Copies in flight are paced: copy k (in the order the waves ask) waits until copies 0 .. k - C have landed, so
  // the launch's first tiles land early instead of every wave's at the end of one burst over all CUs.
  uint32_t* next = lut4 + NTAB * LUTN;
  uint32_t* asked = next + 1;   // copies asked for (the first W: wave w's first tile is copy w)
  uint32_t* landed = next + 2;  // copies landed
  const int C = min(W, TILES_COPIES);
  uint32_t* rowc = next + 4;   // tile rows in the block's tiles: counter of the row whose first tile is T0 + r
  if (threadIdx.x == 0) {
    next[0] = (uint32_t)W;
    asked[0] = (uint32_t)W;
    landed[0] = 0u;
  }
  if (threadIdx.x < TILES_ROWC) rowc[threadIdx.x] = 0u;
  auto ask = [&](uint32_t k) {  // wait for copy k's turn
    while (k >= (uint32_t)C + __hip_atomic_load(landed, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP))
      __builtin_amdgcn_s_sleep(2);
  };
  uint32_t* buf = tbuf + (size_t)wave * buf_rows * 32;
  const uint32_t rlb = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint32_t*)(buf + s);
  uint32_t tmask = 0x1FFCu;
  asm volatile("" : "+v"(tmask));
  // tile n of the block: the second entry or not, and the tile index (wave-uniform values; row-major)
  auto tile_of = [&](int n, int& sec, int& t) {
    const int T = T0 + n;
    sec = __builtin_amdgcn_readfirstlane((NTAB > 1 && mb != ma && T >= eb->tile0) ? 1 : 0);
    KEntry* e = sec ? eb : ea;
    const int u = T - e->tile0;
    t = __builtin_amdgcn_readfirstlane(e->list ? (int)((KU32*)e->list)[u] : u);
  };
  // the tile's rows into the wave's buffer, 8 rows per copy instruction (lane l: row l / 8, words 4 (l % 8) ..),
  // the last one masked to the tile's own rows. The windows also read the 2 rows past the longest lane and the
  // table index takes up to 11 bits past a code's start: those rows keep whatever the buffer held, which no decoded
  // symbol depends on (every code lies within its lane's bits, a prefix code's entry ignores the bits after it).
  // The per-tile words are read through the scalar cache (read-only during the launch). A wave's first copy
  // (slot) of a matrix whose tiles lie at a fixed stride copies the whole slot (max_rows rows: the rows past the
  // tile's own are zeros) and reads no per-tile word, so it is issued as soon as the plan is read. Returns the
  // number of copy instructions.
  auto copy_tile = [&](KEntry* e, int t, bool slot) -> int {
    const int ts = e->M.tstride;
    const int nrow = (slot && ts > 0) ? ts : (int)((KU16*)e->M.rows)[t];
    const uint32_t* wt = e->M.words + (ts > 0 ? (size_t)32 * ts * t : (size_t)((KU32*)e->M.tbase)[t]);
    const uint4* src = reinterpret_cast<const uint4*>(wt) + lane;
    const int nc = (nrow + 7) / 8;
    for (int i = 0; i < nc; ++i)
      if (lane < 8 * (nrow - 8 * i))
        __builtin_amdgcn_global_load_lds(src + 64 * i, (__attribute__((address_space(3))) void*)(buf + 256 * i), 16, 0, 0);
    return nc;
  };
  // The in-launch reduction of a tile's row is deferred behind the next tile's copy and decode: its partial is
  // stored, and after the next copy's wait (which also covers the store) the row counter is incremented; the
  // counter's old value is read after the next decode (before the next copy is issued: a read after it would wait
  // for the copy), and the row's last tile sums the row once its own partial is stored.
  int pend = -1;  // the pending tile's entry: 0 = first, 1 = second, -1 = none
  int ptr = 0, pKT = 0, pN = 0;
  uint32_t pold = 0;
  auto finish_pending = [&]() {
    if (pend < 0) return;
    const uint32_t old = (uint32_t)__builtin_amdgcn_readlane((int)pold, 0);
    if (old == (uint32_t)(pKT - 1)) row_sum(*(pend ? eb : ea), ptr, pKT, pN, lane);
    pend = -1;
  };
  // Wave priority 3 - (tiles taken after the first), at least 0. Among waves of equal priority a SIMD favours the
  // oldest (lowest index), so the block's last waves, whose first copies are paced behind the others', would run
  // slowest and end the launch alone; waves that have decoded fewer tiles go first instead, and the waves end closer
  // together (config 2: 39.6 against 40.3 us per layer).
  int tdone = 0;
  __builtin_amdgcn_s_setprio(3);
  int n = wave;
  bool have = n < per && T0 + n < plan.ntiles;
  int sec = 0, t = 0, ncopy = 0;
  if (have) tile_of(n, sec, t);
  if (have && wave < C) ncopy = copy_tile(sec ? eb : ea, t, true);
  // this wave's table chunks, issued before its copy, are in LDS; the counters too; then every wave's
  // (a bare barrier: the copies stay in flight)
  wait_vmcnt_upto(ncopy);
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  LW_TL(1);
  if (have && wave >= C) {
    ask((uint32_t)wave);
    copy_tile(sec ? eb : ea, t, true);
  }
  if (wave == W - 1) {  // the block's row counts (and word offsets) into the scalar cache, read at each claim, by
                        // the wave whose first tile comes last
    uint32_t warm = 0;
    auto touch = [&](KEntry* e, int u0, int u1) {
      if (e->list) return;
      const bool tb = e->M.tstride == 0;
      for (int u = u0; u <= u1; u += 16) warm += (tb ? ((KU32*)e->M.tbase)[u] : 0u) + ((KU16*)e->M.rows)[u];
      warm += (tb ? ((KU32*)e->M.tbase)[u1] : 0u) + ((KU16*)e->M.rows)[u1];
    };
    touch(ea, T0 - ea->tile0, min(Tl, ea->tile0 + ea->ntile - 1) - ea->tile0);
    if (mb != ma) touch(eb, 0, Tl - eb->tile0);
    asm volatile("" ::"s"(warm));
  }
#pragma unroll 1
  while (have) {
    // one tile of format KQ (KQB: a tile of the plan's entries from nfa on)
    auto tile = [&](auto kq) __attribute__((always_inline)) {
      constexpr int KQ = decltype(kq)::value;
      constexpr int SYMB = kq_symbits(KQ);
      constexpr int TW = SYMB == 4 ? 2 * TK : TK;
      constexpr int GW = kq_gw(KQ), SB = kq_sbytes(KQ);
      constexpr int NSUBT = TW / GW;                          // sub-blocks per tile row
      constexpr int NSB = TW / 256;                           // super-blocks per tile row
      constexpr int NSUB = 256 / GW;                          // sub-blocks per super-block
      constexpr int GPSUB = (GW / (SYMB == 4 ? 2 : 1)) / 16;  // 16-symbol groups per sub-block (2 for Q5_K, else 1)
      constexpr float VSCALE = SYMB == 4 ? 16777216.f : 1.f;
      const int cur = sec;
      const bool second = sec != 0;
      KEntry* ep = second ? eb : ea;
      const auto& E = *ep;
      const auto& M = E.M;
      const int KT = M.KT, N = M.N;
      const int tc = t % KT, tr = t / KT;
      // side records, x sums and chain starts while the copy is in flight
      const uint8_t* srow = M.side + side_record(tr * TN, tc * NSB, KT, NSB) * SB + (uint32_t)(lane * SB);
      uint32_t sw[NSB][5];
  #pragma unroll
      for (int sb = 0; sb < NSB; ++sb) side_load<KQ>(srow + sb * (TN * SB), sw[sb]);
      XgRegs xgr;
      if (!I8) xgr = column_xsums<KQ>(E.X2, tc, lane);
      uint32_t P[NC];
      tile_chain_starts(M, t, f, s, P);
      const uint32_t tsel = second ? 4u * LUTN : 0u;
      uint32_t clim[10], cpk[11];  // the comparator's limits and length words (CANON), the table's place added
      if (CANON) {
        KU32* cz = (KU32*)M.canon;
  #pragma unroll
        for (int k = 0; k < 10; ++k) clim[k] = cz[k];
  #pragma unroll
        for (int k = 0; k < 11; ++k) cpk[k] = cz[10 + k] + (tsel << 16);
        // values in SGPRs (not a per-lane indexed load of the table words)
  #pragma unroll
        for (int k = 0; k < 10; ++k) asm volatile("" : "+s"(clim[k]));
  #pragma unroll
        for (int k = 0; k < 11; ++k) asm volatile("" : "+s"(cpk[k]));
      }
      // the tile column's activations in VGPRs, no scalar loads inside the decode loop (whose waits would drain every
      // chain's LDS reads): fp16 x as 16-dword rows repeated in each 16-lane row (xr[m] lane l = dword 16 m + l % 16,
      // used through DPP broadcasts), int8 x as dwords l, l + 64, .. read back with v_readlane
      constexpr int XV = I8 ? TW / 4 / 64 : 1, XR = I8 ? 1 : TW / 2 / 16;
      uint32_t xv[XV], xr[XR];
      if (I8) {
        const uint32_t* xs = reinterpret_cast<const uint32_t*>(E.XQ) + (size_t)tc * (TW / 4);
  #pragma unroll
        for (int k = 0; k < XV; ++k) xv[k] = xs[64 * k + lane];
      } else {
        const uint32_t* xs = E.X2 + (size_t)tc * (TW / 2) + (lane & 15);
  #pragma unroll
        for (int m = 0; m < XR; ++m) xr[m] = xs[16 * m];
      }
      auto xw = [&](int c) -> uint32_t { return (uint32_t)__builtin_amdgcn_readlane((int)xv[c >> 6], c & 63); };
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the tile is in LDS, the pending tile's partial stored
      LW_TL(4 + 3 * tl_i);
      if (lane == 0) __hip_atomic_fetch_add(landed, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      if (pend >= 0 && lane == 0)
        pold = __hip_atomic_fetch_add((pend ? eb : ea)->cnt + ptr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      // register windows: rows r, r + 1 (A, B) of each chain, row r + 2 (C) read after every pair (P = bit
      // position + 64: bits 5+ give the row C holds)
      uint32_t slot[NC], A[NC], B[NC], C[NC];
  #pragma unroll
      for (int j = 0; j < NC; ++j) {
        slot[j] = __builtin_amdgcn_ubfe(P[j], 5, 8);
        A[j] = *(LdsU32*)(rlb + ((slot[j] - 2u) << 7));
        B[j] = *(LdsU32*)(rlb + ((slot[j] - 1u) << 7));
        C[j] = *(LdsU32*)(rlb + (slot[j] << 7));
      }
      float sub[NSUBT];
      float acc[NC];
      int iacc[NC];
      uint32_t wprev[NC];
  #pragma unroll
      for (int j = 0; j < NC; ++j) {
        acc[j] = 0.f;
        iacc[j] = 0;
        wprev[j] = 0;
      }
      // one pair of symbols of every chain (group gi, pair p), then the end of a 16-symbol group
      auto pair_step = [&](const int gi, const int p) __attribute__((always_inline)) {
          // each step of the pair decode for all chains before the next step, so the chains' LDS round trips overlap
          // (the reads return in order: a chain waits only for its own)
          // (scheduling barriers keep the stages apart, so every chain's read is issued before the first result is
          // waited for; bits >= 16 of P carry table-entry payload and are ignored)
          uint32_t w1[NC], e1[NC], e2[NC];
  #pragma unroll
          for (int j = 0; j < NC; ++j) {
            w1[j] = __builtin_amdgcn_alignbit(B[j], A[j], P[j]);
            e1[j] = *(LdsU32*)(CANON ? canon_addr(w1[j], clim, cpk) : table_addr(w1[j], tsel, tmask));
          }
          __builtin_amdgcn_sched_barrier(0);
  #pragma unroll
          for (int j = 0; j < NC; ++j) {
            const uint32_t w2 = w1[j] >> (e1[j] & 31u);
            e2[j] = *(LdsU32*)(CANON ? canon_addr(w2, clim, cpk) : table_addr(w2, tsel, tmask));
          }
          __builtin_amdgcn_sched_barrier(0);
  #pragma unroll
          for (int j = 0; j < NC; ++j) {
            P[j] = P[j] + e1[j] + e2[j];
            const uint32_t nslot = __builtin_amdgcn_ubfe(P[j], 5, 8);
            const bool slide = nslot != slot[j];  // a pair advances at most 22 bits: at most one row
            A[j] = slide ? B[j] : A[j];
            B[j] = slide ? C[j] : B[j];
            slot[j] = nslot;
            C[j] = *(LdsU32*)(rlb + (nslot << 7));
          }
  #pragma unroll
          for (int j = 0; j < NC; ++j) {
            const int g = NG * j + gi;  // 16-symbol group within the row
            if (I8) {  // as tile_gemv_i8
              if (SYMB == 4) {
                iacc[j] = __builtin_amdgcn_sdot4((int)__builtin_amdgcn_perm(e2[j], e1[j], 0x07060302u),
                                                 (int)xw(8 * g + p), iacc[j], false);
              } else {
                const uint32_t v2 = __builtin_amdgcn_perm(e2[j], e1[j], 0x0C0C0602u);
                if (p & 1) iacc[j] = __builtin_amdgcn_sdot4((int)(wprev[j] | (v2 << 16)), (int)xw(4 * g + p / 2), iacc[j], false);
                else wprev[j] = v2;
              }
            } else if (SYMB == 4) {
              const uint32_t v1 = __builtin_amdgcn_perm(e1[j], e1[j], 0x0C030C02u);
              const uint32_t v2 = __builtin_amdgcn_perm(e2[j], e2[j], 0x0C030C02u);
              const int c = 16 * g + 2 * p;
              dot2_row(acc[j], xr[c >> 4], c & 15, v1);
              dot2_row(acc[j], xr[(c + 1) >> 4], (c + 1) & 15, v2);
            } else {
              const uint32_t v = __builtin_amdgcn_perm(e2[j], e1[j], 0x07060302u);
              const int c = 8 * g + p;
              dot2_row(acc[j], xr[c >> 4], c & 15, v);
            }
          }
      };
      auto group_end = [&](const int gi) __attribute__((always_inline)) {
        if (GPSUB == 1 || (gi & 1)) {
  #pragma unroll
          for (int j = 0; j < NC; ++j) {
            sub[(NG * j + gi) / GPSUB] = I8 ? (float)iacc[j] : acc[j];  // |iacc| < 2^24: exact
            acc[j] = 0.f;
            iacc[j] = 0;
          }
        }
      };
      if constexpr (CANON) {  // (the comparator's steps are past the unroller's size limit)
        static_for<NG>([&](auto gi) {
          static_for<8>([&](auto p) { pair_step(gi, p); });
          group_end(gi);
        });
      } else {
  #pragma unroll
        for (int gi = 0; gi < NG; ++gi) {
  #pragma unroll
          for (int p = 0; p < 8; ++p) pair_step(gi, p);
          group_end(gi);
        }
      }

      // the sub-block sums are formed here, not sunk past the claim and the copy below (the int8 products would be,
      // holding every table entry of the tile in scratch)
  #pragma unroll
      for (int k = 0; k < NSUBT; ++k) asm volatile("" : "+v"(sub[k]));
      LW_TL(5 + 3 * tl_i);
      // the next tile: claimed and its copy issued now (the claim's wait also covers every LDS read of the decode,
      // so the buffer is free); the pending row first
      {
        uint32_t nx = 0;
        if (lane == 0) nx = __hip_atomic_fetch_add(next, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        n = __builtin_amdgcn_readfirstlane((int)nx);
      }
      // the pending row's counter value (arrived during the decode)
      const uint32_t old = pend >= 0 ? (uint32_t)__builtin_amdgcn_readlane((int)pold, 0) : 0u;
      have = n < per && T0 + n < plan.ntiles;
      if (have) {
        tile_of(n, sec, t);
        uint32_t k = 0;
        if (lane == 0) k = __hip_atomic_fetch_add(asked, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        ask((uint32_t)__builtin_amdgcn_readfirstlane((int)k));
        copy_tile(sec ? eb : ea, t, false);
        LW_TL(6 + 3 * tl_i);
        ++tdone;  // the wave's priority falls with the tiles it has taken
        if (tdone == 1) __builtin_amdgcn_s_setprio(2);
        else if (tdone == 2) __builtin_amdgcn_s_setprio(1);
        else __builtin_amdgcn_s_setprio(0);
      }
      // the row partial in tile_gemv's order (tile_gemv_i8's for int8 activations)
      float tot = 0.f;
      if (I8) {
        KF32* dx = (KF32*)(E.DX + (size_t)tc * (TW / 32));
        KF32* sx = (KF32*)(E.SX + (size_t)tc * (TW / 32));
  #pragma unroll
        for (int sb = 0; sb < NSB; ++sb) {
          float dA, dB, mf[8];
          uint64_t scq, scq2;
          side_packed<KQ>(sw[sb], scq, scq2, dA, dB);
          if (KQ == KQ_Q4_K || KQ == KQ_Q5_K) side_mins(sw[sb], mf);
  #pragma unroll
          for (int jj = 0; jj < NSUB; ++jj) {
            if (KQ == KQ_Q6_K && jj == 8) scq = scq2;
            const float scv = (KQ == KQ_Q6_K || KQ == KQ_IQ4_XS) ? (float)(int)(int8_t)(uint8_t)scq
                                                                 : (float)(uint32_t)(scq & 255u);
            scq >>= 8;
            const int xb = (sb * 256 + jj * GW) / 32;
            tot = fmaf(dA * scv * dx[xb], sub[sb * NSUB + jj], tot);
            if (KQ == KQ_Q4_K || KQ == KQ_Q5_K) tot = fmaf(-(dB * mf[jj]), sx[xb], tot);
          }
        }
      } else {
  #pragma unroll
        for (int sb = 0; sb < NSB; ++sb) {
          float dA, dB;
          uint64_t scq, scq2;
          side_packed<KQ>(sw[sb], scq, scq2, dA, dB);
          if (KQ == KQ_Q4_K || KQ == KQ_Q5_K) {
            float mf[8], msum = 0.f;
            side_mins(sw[sb], mf);
  #pragma unroll
            for (int jj = 0; jj < NSUB; ++jj) msum = fmaf(mf[jj], xgr(sb, jj, 0), msum);
            tot = fmaf(-dB, msum, tot);
          }
          if (KQ == KQ_IQ4_XS) {
            float csum = 0.f;
  #pragma unroll
            for (int jj = 0; jj < NSUB; ++jj) csum = fmaf((float)(int)(int8_t)(uint8_t)(scq >> (8 * jj)), xgr(sb, jj, 0), csum);
            tot = fmaf(-128.f * dA, csum, tot);
          }
          float tsum = 0.f;
  #pragma unroll
          for (int jj = 0; jj < NSUB; ++jj) {
            if (KQ == KQ_Q6_K && jj == 8) scq = scq2;
            const float scv = (KQ == KQ_Q6_K || KQ == KQ_IQ4_XS) ? (float)(int)(int8_t)(uint8_t)scq
                                                                 : (float)(uint32_t)(scq & 255u);
            scq >>= 8;
            tsum = fmaf(scv, sub[sb * NSUB + jj], tsum);
          }
          tot = fmaf(dA * VSCALE, tsum, tot);
        }
      }
      float* out = E.P + (size_t)tc * N + (size_t)tr * TN + (uint32_t)lane;
      __hip_atomic_store(out, tot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (pend >= 0 && old == (uint32_t)(pKT - 1)) row_sum(*(pend ? eb : ea), ptr, pKT, pN, lane);
      pend = -1;
      if (E.Y) {
        // a tile row among the block's own tiles is counted in LDS at once (its global counter stays 0); a row
        // shared with other blocks in the entry's counter, one tile later
        const int r0 = E.tile0 + tr * KT - T0;
        if (!E.list && r0 >= 0 && r0 < TILES_ROWC && T0 + r0 + KT - 1 <= Tl) {
          uint32_t o = 0;
          if (lane == 0) o = __hip_atomic_fetch_add(rowc + r0, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
          if ((uint32_t)__builtin_amdgcn_readlane((int)o, 0) == (uint32_t)(KT - 1)) row_sum(E, tr, KT, N, lane, 1, false);
        } else {
          pend = cur;
          ptr = tr;
          pKT = KT;
          pN = N;
        }
      }
      ++tl_i;
    };
    if constexpr (KQB != KQA) {
      if (__builtin_amdgcn_readfirstlane((sec ? mb : ma) >= plan.nfa ? 1 : 0)) tile(KqTag<KQB>{});
      else tile(KqTag<KQA>{});
    } else {
      tile(KqTag<KQA>{});
    }
  }
  if (pend >= 0) {  // the last tile's reduction
    if (lane == 0)
      pold = __hip_atomic_fetch_add((pend ? eb : ea)->cnt + ptr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    finish_pending();
  }
  LW_TL(3);
}

// ── half-tile kernel for flat launches (m = 1, fp16 activations): a wave decodes half-tile units, two buffered ─────
// Unit (tile t, half f) = the tile's rows 32 f .. 32 f + 31 (lane stream s, its row f). Lane l decodes symbols
// 128 (l / 32) .. + 127 of row 32 f + (l % 32) as 4 chains of 32 symbols from the load-time split offsets; the two
// lanes of a row then hand their sub-block dot products to the lower one, which forms the row partial in
// tile_gemv's order (the bits of the other kernels).
// A unit's word rows are copied into one of the wave's two LDS buffers: rows [0, hrow & 0xFFFF) for f = 0, rows
// [hrow >> 16, rows[t]) for f = 1 (Layout::hrow). While a unit decodes, the next unit's copy and its loads (chain
// starts, x, the x words of the sub-block sums, side records) are in flight into the other buffer and a second
// register set: the wait at a unit's start is for data asked for one unit earlier. Values loaded for the next unit
// are only moved or computed on after that wait (an earlier use would make the compiler wait for the copy too).
// The block takes units [0, 2 n) of its tiles [T0, T0 + n) from a counter in LDS; the in-launch reduction is per
// tile row and half (counter 2 tr + f), its atomic issued one unit after the partial's store and its result read
// one unit later still. Tables as k_fused_tiles.
// The in-launch reduction of half a tile row (lanes 0..31: row 64 tr + 32 f + lane) in tile-column order, as
// row_sum; its counter (2 tr + f) is reset for the next launch.
template <class KEntryRef>
__device__ __forceinline__ void row_sum_half(const KEntryRef& E, int tr, int f, int KT, int N, int lane) {
  if (lane == 0) __hip_atomic_store(E.cnt + 2 * tr + f, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (lane >= 32) return;
  E.Y[(size_t)tr * TN + (uint32_t)(32 * f + lane)] =
      sum_partials(reinterpret_cast<uint32_t*>(E.P + (size_t)tr * TN + (uint32_t)(32 * f + lane)), (size_t)N, KT);
}

template <int KQ>
struct HalfRegs {
  static constexpr int SYMB = kq_symbits(KQ);
  static constexpr int XR = SYMB == 4 ? 8 : 4;  // x dwords of the lane's half row: 16 lanes x XR consecutive
  // the side record's words as loaded (Q6_K: the 5 aligned dwords holding the 2-byte aligned 18-byte record)
  static constexpr int SR = KQ == KQ_Q6_K ? 5 : (KQ == KQ_IQ4_XS ? 2 : 4);
  uint32_t sp[2];   // the lane's 4 chain starts (u16 pairs)
  uint32_t xr[XR];
  uint32_t xq[4];   // the x dwords of one quarter sub-block (lane 4 g + k: quarter k of sub-block g)
  uint32_t sr[SR];  // the side record of the lane's super-block (both lanes of a row: the row's only one)
  int t, sec, f;    // the unit (wave-uniform)
};

template <int KQ, int NTAB>
__global__ void __launch_bounds__(1024, 1)
k_fused_halves(FlatPlan plan, int per, int ubuf_rows) {
  typedef HalfRegs<KQ> R;
  constexpr int SYMB = kq_symbits(KQ);
  constexpr int TW = SYMB == 4 ? 2 * TK : TK;
  constexpr int GW = kq_gw(KQ), SB = kq_sbytes(KQ);
  constexpr int NSUBT = TW / GW;                          // sub-blocks per tile row
  constexpr int NSUBH = NSUBT / 2;                        // per lane (half a row)
  constexpr int NSB = TW / 256;                           // super-blocks per tile row (2: one per lane)
  constexpr int NSUB = 256 / GW;                          // sub-blocks per super-block
  constexpr int GPSUB = (GW / (SYMB == 4 ? 2 : 1)) / 16;  // 16-symbol groups per sub-block (2 for Q5_K, else 1)
  constexpr float VSCALE = SYMB == 4 ? 16777216.f : 1.f;
  constexpr int NC = 4;                                   // chains per lane (32 symbols each)
  constexpr int NG = 2;                                   // 16-symbol groups per chain
  constexpr int XR = R::XR, SR = R::SR;
  constexpr int Q = GW / 8;                               // x dwords per quarter sub-block (4)
  static_assert(KQ == KQ_Q6_K || Q == 4, "quarter sub-blocks of 4 dwords");
  typedef __attribute__((address_space(3))) const uint32_t LdsU32;
  typedef __attribute__((address_space(4))) const char KChar;
  typedef __attribute__((address_space(4))) const FlatEntry KEntry;
  typedef __attribute__((address_space(4))) const uint32_t KU32;
  __shared__ uint32_t lut4[NTAB * LUTN + 4];
  extern __shared__ __align__(16) uint32_t tbuf[];  // W x 2 x ubuf_rows word rows of 32 words

  KChar* kbase = (KChar*)__builtin_amdgcn_kernarg_segment_ptr();
  const int W = plan.W, T0 = (int)blockIdx.x * per, Tl = min(T0 + per, plan.ntiles) - 1;
  const int units = 2 * (Tl - T0 + 1);
  int ma = 0, mb = 0;
#pragma unroll
  for (int i = 1; i < MAX_GROUP; ++i) {
    if (i < plan.n && T0 >= plan.e[i].tile0) ma = i;
    if (i < plan.n && Tl >= plan.e[i].tile0) mb = i;
  }
  KEntry* ea = (KEntry*)(kbase + offsetof(FlatPlan, e) + (size_t)ma * sizeof(FlatEntry));
  KEntry* eb = (KEntry*)(kbase + offsetof(FlatPlan, e) + (size_t)mb * sizeof(FlatEntry));
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63, s = lane & 31, h = lane >> 5;
  {  // the tables: 1 KB direct-to-LDS loads, chunk c (8 per table) by wave c mod W, ahead of the first unit's
    const uint4* ta = reinterpret_cast<const uint4*>(ea->M.lut4);
    const uint4* tb = reinterpret_cast<const uint4*>(eb->M.lut4);
    const int nchunk = (NTAB > 1 && mb != ma) ? 16 : 8;
    for (int c = wave; c < nchunk; c += W)
      __builtin_amdgcn_global_load_lds((c < 8 ? ta : tb) + 64 * (c & 7) + lane,
                                       (__attribute__((address_space(3))) void*)(lut4 + 256 * c), 16, 0, 0);
  }
  uint32_t* next = lut4 + NTAB * LUTN;
  if (threadIdx.x == 0) *next = (uint32_t)W;
  uint32_t* const buf0 = tbuf + (size_t)(2 * wave) * ubuf_rows * 32;
  uint32_t* const buf1 = buf0 + (size_t)ubuf_rows * 32;
  uint32_t tmask = 0x1FFCu;
  asm volatile("" : "+v"(tmask));

  // unit v of the block: tile T0 + v / 2 (row-major in its matrix), half v % 2
  auto unit_of = [&](int v, R& U) {
    const int T = T0 + (v >> 1);
    U.sec = __builtin_amdgcn_readfirstlane((NTAB > 1 && mb != ma && T >= eb->tile0) ? 1 : 0);
    KEntry* e = U.sec ? eb : ea;
    const int u = T - e->tile0;
    U.t = __builtin_amdgcn_readfirstlane(e->list ? (int)((KU32*)e->list)[u] : u);
    U.f = v & 1;
  };
  // the unit's loads (kept as loaded); its rows' copy (8 rows per instruction, the last masked) is described in
  // (src, nrow) and issued two instructions per pair step of the decode that runs meanwhile (copy_part)
  // (buffer loads: the rows as a wave-uniform resource, instruction i at scalar offset 1 KB i, so the copy holds no
  // per-lane addresses through the decode)
  __amdgpu_buffer_rsrc_t crs = __builtin_amdgcn_make_buffer_rsrc(nullptr, 0, 0, kBufferRsrcWord3);
  int crow = 0;
  auto copy_part = [&](uint32_t* buf, int i0) {
#pragma unroll
    for (int i = i0; i < i0 + 2; ++i)
      if (8 * i < crow && lane < 8 * (crow - 8 * i))
        __builtin_amdgcn_raw_ptr_buffer_load_lds(crs, (__attribute__((address_space(3))) void*)(buf + 256 * i), 16,
                                                 lane * 16, 1024 * i, 0, 0);
  };
  auto ask = [&](R& U, uint32_t* buf) {
    KEntry* e = U.sec ? eb : ea;
    const auto& M = e->M;
    const int t = U.t, f = U.f, KT = M.KT, tc = t % KT, tr = t / KT;
    const uint2 sp = reinterpret_cast<const uint2*>(M.hsplit)[((size_t)t * 2 + f) * 64 + (uint32_t)lane];
    U.sp[0] = sp.x;
    U.sp[1] = sp.y;
    const uint32_t* xcol = e->X2 + (size_t)tc * (TW / 2);
    const uint4* xs = reinterpret_cast<const uint4*>(xcol + (uint32_t)(h * (TW / 4) + XR * (lane & 15)));
#pragma unroll
    for (int k = 0; k < XR / 4; ++k) {
      const uint4 v = xs[k];
      U.xr[4 * k] = v.x;
      U.xr[4 * k + 1] = v.y;
      U.xr[4 * k + 2] = v.z;
      U.xr[4 * k + 3] = v.w;
    }
    if (KQ != KQ_Q6_K) {  // lanes past the tile column's sub-blocks re-read its last quarter
      const uint4 v = reinterpret_cast<const uint4*>(xcol)[min(lane, 4 * NSUBT - 1)];
      U.xq[0] = v.x;
      U.xq[1] = v.y;
      U.xq[2] = v.z;
      U.xq[3] = v.w;
    }
    const uint8_t* p = M.side + (side_record(tr * TN, tc * NSB, KT, NSB) + (uint32_t)(NSB > 1 ? h * TN : 0) +
                                 (uint32_t)(32 * f + s)) * SB;
    if (KQ == KQ_Q6_K) {
      const uint32_t* a = reinterpret_cast<const uint32_t*>((uintptr_t)p & ~(uintptr_t)3);
#pragma unroll
      for (int i = 0; i < 5; ++i) U.sr[i] = a[i];
    } else if (KQ == KQ_IQ4_XS) {
      const uint2 v = *reinterpret_cast<const uint2*>(p);
      U.sr[0] = v.x;
      U.sr[1] = v.y;
    } else {
      const uint4 v = *reinterpret_cast<const uint4*>(p);
      U.sr[0] = v.x;
      U.sr[1] = v.y;
      U.sr[2] = v.z;
      U.sr[3] = v.w;
    }
    // (rows[t] through a scalar dword read: a 16-bit read would be a vector load waited for at once)
    const uint32_t hr = ((KU32*)M.hrow)[t];
    const uint32_t rw = ((KU32*)M.rows)[t >> 1] >> (16 * (t & 1)) & 0xFFFFu;
    const int r0 = f ? (int)(hr >> 16) : 0, nrow = f ? (int)rw - r0 : (int)(hr & 0xFFFFu);
    crs = __builtin_amdgcn_make_buffer_rsrc((void*)(M.words + ((KU32*)M.tbase)[t] + 32u * (uint32_t)r0), 0,
                                            nrow * 128, kBufferRsrcWord3);
    crow = nrow;
    for (int i = 8; 8 * i < crow; i += 2) copy_part(buf, i);  // rows past 64: up front
  };

  R RA;  // the unit asked for last
  const bool have = wave < units;
  if (have) {
    unit_of(wave, RA);
    ask(RA, buf0);
    for (int i = 0; i < 8; i += 2) copy_part(buf0, i);
  }
  // this wave's table chunks (issued before its first unit's loads and copy) are in LDS; the counter too; then
  // every wave's (a bare barrier: the copies stay in flight)
  wait_vmcnt_upto((crow + 7) / 8);
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  if (wave == 0) {  // the block's row counts, half rows and word offsets into the scalar cache (read at each ask)
    uint32_t warm = 0;
    auto touch = [&](KEntry* e, int u0, int u1) {
      if (e->list) return;
      for (int u = u0; u <= u1; u += 16)
        warm += ((KU32*)e->M.tbase)[u] + ((KU32*)e->M.hrow)[u] + ((KU32*)e->M.rows)[u >> 1];
      warm += ((KU32*)e->M.tbase)[u1] + ((KU32*)e->M.hrow)[u1] + ((KU32*)e->M.rows)[u1 >> 1];
    };
    touch(ea, T0 - ea->tile0, min(Tl, ea->tile0 + ea->ntile - 1) - ea->tile0);
    if (mb != ma) touch(eb, 0, Tl - eb->tile0);
    asm volatile("" ::"s"(warm));
  }

  // in-launch reduction state: pa = a stored partial whose counter is not yet incremented, pb = a counter increment
  // whose old value has not been read
  int pa_sec = -1, pa_tr = 0, pa_f = 0;
  int pb_sec = -1, pb_tr = 0, pb_f = 0;
  uint32_t pold = 0;
  auto reduce_pending = [&]() {  // after a vmcnt(0) wait
    if (pb_sec >= 0) {
      const auto& E = *(pb_sec ? eb : ea);
      const uint32_t old = (uint32_t)__builtin_amdgcn_readlane((int)pold, 0);
      if (old == (uint32_t)(E.M.KT - 1)) row_sum_half(E, pb_tr, pb_f, E.M.KT, E.M.N, lane);
      pb_sec = -1;
    }
    if (pa_sec >= 0) {
      const auto& E = *(pa_sec ? eb : ea);
      if (lane == 0)
        pold = __hip_atomic_fetch_add(E.cnt + 2 * pa_tr + pa_f, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      pb_sec = pa_sec;
      pb_tr = pa_tr;
      pb_f = pa_f;
      pa_sec = -1;
    }
  };

  // One unit per iteration: the unit asked for last (in Y, its rows in buffer `cur`) becomes X and decodes while the
  // next one is asked for into Y and the other buffer (X = Y only after the wait: moving values still being loaded
  // would wait for them).
  R X;
  int cur = 0;
#pragma unroll 1
  for (bool more = have; more;) {
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): X's rows and loads, the last partial's store
    X = RA;
    uint32_t* const bx = cur ? buf1 : buf0;
    uint32_t* const by = cur ? buf0 : buf1;
    R& Y = RA;
    reduce_pending();
    // the next unit is claimed ahead (its copy overlaps this decode) while more units are left than waves; the
    // last ones are claimed by whichever waves free up first, after their decode
    more = false;
    crow = 0;
    const bool ahead = (int)__hip_atomic_load(next, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) + W < units;
    if (ahead) {
      uint32_t nx = 0;
      if (lane == 0) nx = __hip_atomic_fetch_add(next, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      const int v = __builtin_amdgcn_readfirstlane((int)nx);
      more = v < units;
      if (more) {
        unit_of(v, Y);
        ask(Y, by);
      }
    }
    const bool second = X.sec != 0;
    const auto& E = *(second ? eb : ea);
    const auto& M = E.M;
    const int t = X.t, f = X.f, KT = M.KT, N = M.N;
    const int tc = t % KT, tr = t / KT;
    const uint32_t hr = ((KU32*)M.hrow)[t];
    const uint32_t r0 = f ? hr >> 16 : 0u;
    const uint32_t rlb = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint32_t*)(bx + s) - (r0 << 7);
    const uint32_t tsel = second ? 4u * LUTN : 0u;
    uint32_t P[NC], slot[NC], A[NC], B[NC], C[NC];
#pragma unroll
    for (int j = 0; j < NC; ++j) {
      P[j] = (X.sp[j >> 1] >> (16 * (j & 1)) & 0xFFFFu) - GUARD_BITS + 64u;
      slot[j] = __builtin_amdgcn_ubfe(P[j], 5, 8);
      A[j] = *(LdsU32*)(rlb + ((slot[j] - 2u) << 7));
      B[j] = *(LdsU32*)(rlb + ((slot[j] - 1u) << 7));
      C[j] = *(LdsU32*)(rlb + (slot[j] << 7));
    }
    float sub[NSUBH];
    float acc[NC];
#pragma unroll
    for (int j = 0; j < NC; ++j) acc[j] = 0.f;
#pragma unroll
    for (int gi = 0; gi < NG; ++gi) {
#pragma unroll
      for (int p = 0; p < 8; ++p) {
        if (gi == 0 && p < 4) copy_part(by, 2 * p);  // the next unit's first 64 rows, spread over the decode
        uint32_t w1[NC], e1[NC], e2[NC];
#pragma unroll
        for (int j = 0; j < NC; ++j) {
          w1[j] = __builtin_amdgcn_alignbit(B[j], A[j], P[j]);
          e1[j] = *(LdsU32*)table_addr(w1[j], tsel, tmask);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < NC; ++j) e2[j] = *(LdsU32*)table_addr(w1[j] >> (e1[j] & 31u), tsel, tmask);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < NC; ++j) {
          P[j] = P[j] + e1[j] + e2[j];
          const uint32_t nslot = __builtin_amdgcn_ubfe(P[j], 5, 8);
          const bool slide = nslot != slot[j];  // a pair advances at most 22 bits: at most one row
          A[j] = slide ? B[j] : A[j];
          B[j] = slide ? C[j] : B[j];
          slot[j] = nslot;
          C[j] = *(LdsU32*)(rlb + (nslot << 7));
        }
        // x dword c of the lane's half row is register c % XR of lane c / XR of its 16-lane row (DPP broadcast)
#pragma unroll
        for (int j = 0; j < NC; ++j) {
          const int g = NG * j + gi;  // 16-symbol group within the lane's half row
          if (SYMB == 4) {
            const uint32_t v1 = __builtin_amdgcn_perm(e1[j], e1[j], 0x0C030C02u);
            const uint32_t v2 = __builtin_amdgcn_perm(e2[j], e2[j], 0x0C030C02u);
            const int c = 16 * g + 2 * p;
            dot2_row(acc[j], X.xr[c % XR], c / XR, v1);
            dot2_row(acc[j], X.xr[(c + 1) % XR], (c + 1) / XR, v2);
          } else {
            const uint32_t v = __builtin_amdgcn_perm(e2[j], e1[j], 0x07060302u);
            const int c = 8 * g + p;
            dot2_row(acc[j], X.xr[c % XR], c / XR, v);
          }
        }
      }
      if (GPSUB == 1 || (gi & 1)) {
#pragma unroll
        for (int j = 0; j < NC; ++j) {
          sub[(NG * j + gi) / GPSUB] = acc[j];
          acc[j] = 0.f;
        }
      }
    }
    // x sums of the tile column's sub-blocks (as column_xsums, from the words asked for with X)
    // (xg[g]: the sum over sub-block g of the lane's super-block, or of the row's one super-block)
    float xg[8];
    if (KQ != KQ_Q6_K) {
      float a = 0.f;
#pragma unroll
      for (int c = 0; c < Q; ++c) a += h2f(X.xq[c]) + h2f(X.xq[c] >> 16);
      a += __shfl_xor(a, 1);
      a += __shfl_xor(a, 2);
#pragma unroll
      for (int g = 0; g < 8; ++g) {
        const float v0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, a), 4 * g));
        const float v1 = NSB == 2 ? __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, a), 4 * (g + 8)))
                                  : v0;
        xg[g] = h ? v1 : v0;
      }
    }
    // The row partial in tile_gemv's order, its terms split over the row's two lanes: with two super-blocks per row
    // each lane forms its super-block's terms and the upper lane applies them after the lower lane's partial; with
    // one, the lower lane runs the first half of the sub-block sum and the upper lane the rest and the total.
    uint32_t sw[5];
    if (KQ == KQ_Q6_K) {  // 18-byte records from a 256-byte aligned array: odd rows start 2 bytes into a dword
      const uint32_t sh = (s & 1) ? 16u : 0u;
#pragma unroll
      for (int i = 0; i < 4; ++i) sw[i] = __builtin_amdgcn_alignbit(X.sr[i + 1], X.sr[i], sh);
      sw[4] = X.sr[4] >> sh & 0xFFFFu;
    } else {
#pragma unroll
      for (int i = 0; i < SR; ++i) sw[i] = X.sr[i];
    }
    float dA, dB;
    uint64_t scq, scq2;
    side_packed<KQ>(sw, scq, scq2, dA, dB);
    float tot;
    if (NSB == 2) {  // Q4_K, IQ4_XS: lane h holds super-block h's sub-blocks
      float pre = 0.f;  // msum (Q4_K) or csum (IQ4_XS) of the lane's super-block
      if (KQ == KQ_Q4_K) {
        float mf[8];
        side_mins(sw, mf);
  #pragma unroll
        for (int jj = 0; jj < NSUB; ++jj) pre = fmaf(mf[jj], xg[jj], pre);
      }
      if (KQ == KQ_IQ4_XS) {
  #pragma unroll
        for (int jj = 0; jj < NSUB; ++jj)
          pre = fmaf((float)(int)(int8_t)(uint8_t)(scq >> (8 * jj)), xg[jj], pre);
      }
      float tsum = 0.f;
  #pragma unroll
      for (int jj = 0; jj < NSUB; ++jj) {
        const float scv = KQ == KQ_IQ4_XS ? (float)(int)(int8_t)(uint8_t)scq : (float)(uint32_t)(scq & 255u);
        scq >>= 8;
        tsum = fmaf(scv, sub[jj], tsum);
      }
      // super-block 0's terms from 0 (the lower lane's), then super-block 1's after them (the upper lane's)
      auto terms = [&](float t) {
        if (KQ == KQ_Q4_K) t = fmaf(-dB, pre, t);
        if (KQ == KQ_IQ4_XS) t = fmaf(-128.f * dA, pre, t);
        return fmaf(dA * VSCALE, tsum, t);
      };
      tot = terms(__shfl_xor(terms(0.f), 32));
    } else {  // Q5_K, Q6_K: one super-block per row, lane h holds its sub-blocks NSUBH h .. NSUBH h + NSUBH - 1
      uint64_t sq = h ? (KQ == KQ_Q6_K ? scq2 : scq >> (8 * NSUBH)) : scq;  // the lane's sub-blocks' scales
      auto half_sum = [&](float t) {
        uint64_t q = sq;
  #pragma unroll
        for (int jj = 0; jj < NSUBH; ++jj) {
          const float scv = KQ == KQ_Q6_K ? (float)(int)(int8_t)(uint8_t)q : (float)(uint32_t)(q & 255u);
          q >>= 8;
          t = fmaf(scv, sub[jj], t);
        }
        return t;
      };
      // the sum over the lower lane's sub-blocks from 0, continued over the upper lane's
      const float tsum = half_sum(__shfl_xor(half_sum(0.f), 32));
      tot = 0.f;
      if (KQ == KQ_Q5_K) {
        float mf[8], msum = 0.f;
        side_mins(sw, mf);
  #pragma unroll
        for (int jj = 0; jj < NSUB; ++jj) msum = fmaf(mf[jj], xg[jj], msum);
        tot = fmaf(-dB, msum, tot);
      }
      tot = fmaf(dA * VSCALE, tsum, tot);
    }
    if (lane >= 32) {
      float* out = E.P + (size_t)tc * N + (size_t)tr * TN + (uint32_t)(32 * f + s);
      __hip_atomic_store(out, tot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (E.Y) {
      pa_sec = X.sec;
      pa_tr = tr;
      pa_f = f;
    }
    if (!ahead) {
      uint32_t nx = 0;
      if (lane == 0) nx = __hip_atomic_fetch_add(next, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      const int v = __builtin_amdgcn_readfirstlane((int)nx);
      more = v < units;
      if (more) {
        unit_of(v, Y);
        ask(Y, by);
        for (int i = 0; i < 8; i += 2) copy_part(by, i);
      }
    }
    cur ^= 1;
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  reduce_pending();  // the last counter's old value read, the last partial's counter incremented
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  reduce_pending();
}

// ── whole-tile kernel on the matrix cores (2..8 tokens, fp16 activations, every format) ───────────────────
// The decode of k_fused_tiles (a tile per wave in LDS; 4 chains per lane), with the products of MT tokens on
// v_mfma_f32_4x4x4f16 (16 blocks of 4 lanes): block b computes D[i][j] = sum_k A[4 b' + i][k] B[4 b + j][k] into lane
// 4 b + j, register i, where b' is the block named by the instruction's broadcast field (cbsz 4, abid b'). B = the
// lane's own 4 weights of the pair (its row), A = the 4 x values of token i at those positions, broadcast from block
// b' of a register that holds 16 position blocks: x of a tile column fits 8 (4-bit formats) or 4 register pairs per
// 4 tokens, with no LDS traffic. The weights enter unscaled and exact in fp16: the 4-bit formats' grid bytes (Q4_K q,
// IQ4_XS kv[q] + 128) as denormals g 2^-24 from one byte permute per table entry, the 8-bit formats' fp16(f(q))
// (Q5_K q, Q6_K q - 32) from the entries; each chain keeps its current sub-block's sums of 4 tokens in one
// accumulator and folds them into fp32 with d s_j (2^24 d s_j for the denormal form; s_j signed for Q6_K and
// IQ4_XS) when the sub-block ends. The offset terms run on the same instruction with A = the sub-block sums of x as
// fp16 hi and lo (XS): Q4_K / Q5_K dmin sum_j m_j (sum x)_j with B = the row's mins, IQ4_XS 128 d sum_j s_j (sum x)_j
// (the grid's +128) with B = the row's signed scales; Q6_K has none. Each token's values agree with its own m = 1
// launch to fp32 rounding (another order of the same products). Partials [KT][mt][N], the in-launch reduction.
// The tile pipeline is k_fused_tiles': tables by direct-to-LDS loads, paced first copies, row-major tiles, the next
// tile's copy issued as soon as a decode ends.
// at most 16 waves per block (4 per SIMD: 128 VGPRs); 12 (3 per SIMD) for 8 tokens of the 4-bit formats, whose
// 8 tokens' x, the 4 chains' accumulators per token quad and the chains take more than 128 VGPRs
constexpr int TILES_MMA_WAVES = 16;
constexpr int tiles_mma_waves(int kqt, int mt) { return mt == 8 && kq_symbits(kqt) == 4 ? 12 : TILES_MMA_WAVES; }

// v_mfma_f32_4x4x4f16 over 16 blocks with A broadcast from block ABID
template <int ABID>
__device__ __forceinline__ f4v mfma4_from(h4v a, h4v b, f4v c) {
  return __builtin_amdgcn_mfma_f32_4x4x4f16(a, b, c, 4, ABID, 0);
}

template <int KQA, int NTAB, int MT, int KQB = KQA>
__global__ void __launch_bounds__(64 * (tiles_mma_waves(KQA, MT) < tiles_mma_waves(KQB, MT) ? tiles_mma_waves(KQA, MT)
                                                                                         : tiles_mma_waves(KQB, MT)),
                                  1)
k_fused_tiles_mma(FlatPlan plan, int per, int buf_rows) {
  static_assert(MT == 4 || MT == 8, "4 or 8 token slots");
  constexpr int NQ = MT / 4;      // token quads
  constexpr int NC = 4, NG = 16 / NC;  // chains per lane (64 symbols each: 8 tokens' x and accumulators leave no
                                       // registers for 8 chains at 4 waves per SIMD), 16-symbol groups per chain
  typedef __attribute__((address_space(3))) const uint32_t LdsU32;
  typedef __attribute__((address_space(4))) const char KChar;
  typedef __attribute__((address_space(4))) const FlatEntry KEntry;
  typedef __attribute__((address_space(4))) const uint32_t KU32;
  typedef __attribute__((address_space(4))) const uint16_t KU16;
  __shared__ uint32_t lut4[NTAB * LUTN + 4];
  extern __shared__ __align__(16) uint32_t tbuf[];

  KChar* kbase = (KChar*)__builtin_amdgcn_kernarg_segment_ptr();
  const int W = plan.W, T0 = (int)blockIdx.x * per, Tl = min(T0 + per, plan.ntiles) - 1, mt = plan.mt;
  int ma = 0, mb = 0;
#pragma unroll
  for (int i = 1; i < MAX_GROUP; ++i) {
    if (i < plan.n && T0 >= plan.e[i].tile0) ma = i;
    if (i < plan.n && Tl >= plan.e[i].tile0) mb = i;
  }
  KEntry* ea = (KEntry*)(kbase + offsetof(FlatPlan, e) + (size_t)ma * sizeof(FlatEntry));
  KEntry* eb = (KEntry*)(kbase + offsetof(FlatPlan, e) + (size_t)mb * sizeof(FlatEntry));
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63, s = lane & 31, f = lane >> 5;
  const int qb = lane >> 2, qi = lane & 3;  // 4-lane block and the lane's place in it
  {  // the tables: 1 KB direct-to-LDS loads, chunk c (8 per table) by wave c mod W
    const uint4* ta = reinterpret_cast<const uint4*>(ea->M.lut4);
    const uint4* tb = reinterpret_cast<const uint4*>(eb->M.lut4);
    const int nchunk = (NTAB > 1 && mb != ma) ? 16 : 8;
    for (int c = wave; c < nchunk; c += W)
      __builtin_amdgcn_global_load_lds((c < 8 ? ta : tb) + 64 * (c & 7) + lane,
                                       (__attribute__((address_space(3))) void*)(lut4 + 256 * c), 16, 0, 0);
  }
  // copies paced as in k_fused_tiles: copy k (in the order the waves ask) waits for copies 0 .. k - C to land
  uint32_t* next = lut4 + NTAB * LUTN;
  uint32_t* asked = next + 1;
  uint32_t* landed = next + 2;
  uint32_t* xs_done = next + 3;  // waves done with their share of the x sums
  const int C = min(W, TILES_COPIES);
  if (threadIdx.x == 0) {
    next[0] = (uint32_t)W;
    asked[0] = (uint32_t)W;
    landed[0] = 0u;
    xs_done[0] = 0u;
  }
  auto ask = [&](uint32_t k) {
    while (k >= (uint32_t)C + __hip_atomic_load(landed, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP))
      __builtin_amdgcn_s_sleep(2);
  };
  uint32_t* buf = tbuf + (size_t)wave * buf_rows * 32;
  const uint32_t rlb = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint32_t*)(buf + s);
  uint32_t tmask = 0x1FFCu;
  asm volatile("" : "+v"(tmask));
  auto tile_of = [&](int n, int& sec, int& t) {  // row-major, as k_fused_tiles
    const int T = T0 + n;
    sec = __builtin_amdgcn_readfirstlane((NTAB > 1 && mb != ma && T >= eb->tile0) ? 1 : 0);
    KEntry* e = sec ? eb : ea;
    const int u = T - e->tile0;
    t = __builtin_amdgcn_readfirstlane(e->list ? (int)((KU32*)e->list)[u] : u);
  };
  auto copy_tile = [&](KEntry* e, int t, bool slot) -> int {  // as k_fused_tiles (a first copy takes the slot)
    const int ts = e->M.tstride;
    const int nrow = (slot && ts > 0) ? ts : (int)((KU16*)e->M.rows)[t];
    const uint32_t* wt = e->M.words + (ts > 0 ? (size_t)32 * ts * t : (size_t)((KU32*)e->M.tbase)[t]);
    const uint4* src = reinterpret_cast<const uint4*>(wt) + lane;
    const int nc = (nrow + 7) / 8;
    for (int i = 0; i < nc; ++i)
      if (lane < 8 * (nrow - 8 * i))
        __builtin_amdgcn_global_load_lds(src + 64 * i, (__attribute__((address_space(3))) void*)(buf + 256 * i), 16, 0, 0);
    return nc;
  };
  int pend = -1;
  int ptr = 0, pKT = 0, pN = 0;
  uint32_t pold = 0;
  auto finish_pending = [&]() {
    if (pend < 0) return;
    const uint32_t old = (uint32_t)__builtin_amdgcn_readlane((int)pold, 0);
    if (old == (uint32_t)(pKT - 1)) row_sum(*(pend ? eb : ea), ptr, pKT, pN, lane, mt);
    pend = -1;
  };
  int n = wave;
  bool have = n < per && T0 + n < plan.ntiles;
  int sec = 0, t = 0, ncopy = 0;
  if (have) tile_of(n, sec, t);
  if (have && wave < C) ncopy = copy_tile(sec ? eb : ea, t, true);
  // this wave's table chunks and the counters are in place; then every wave's (a bare barrier: copies stay in flight)
  wait_vmcnt_upto(ncopy);
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  // The x sums of every tile column the block decodes, in LDS after the tile buffers (tiles_mma_xs_bytes): per
  // column slot, token and group of 4 sub-blocks their sums in xsum_sub's order as 4 fp16 hi halves, then 4 fp16 lo
  // halves. Column slots: the first entry's columns from ca0 (mod KT), then the second entry's from cb0. Formed by
  // the waves that wait for their first copy's turn (all waves when none waits) before they ask for it; read once
  // the block's counter shows every share stored.
  // (groups of 4 sub-blocks per tile column: TW / 128 of the entry's type; Q6_K has no x sums)
  auto gpc_of = [&](KEntry* e) { return e->M.symbits == 4 ? 4 : 2; };
  auto cols = [&](KEntry* e, int u0, int u1, int& c0) {  // the columns of the entry's tiles u0 .. u1 (row-major)
    const int KT = e->M.KT;
    c0 = u1 - u0 + 1 >= KT ? 0 : u0 % KT;
    return min(KT, u1 - u0 + 1);
  };
  int ca0 = 0, cb0 = 0;
  const int nca = cols(ea, T0 - ea->tile0, min(Tl, ea->tile0 + ea->ntile - 1) - ea->tile0, ca0);
  const int ncb = (NTAB > 1 && mb != ma) ? cols(eb, 0, Tl - eb->tile0, cb0) : 0;
  const int gpa = gpc_of(ea), gpb = gpc_of(eb);
  const bool xsa = ea->M.kqt != KQ_Q6_K, xsbe = ncb > 0 && eb->M.kqt != KQ_Q6_K;
  uint64_t* xsb = reinterpret_cast<uint64_t*>(tbuf + (size_t)W * buf_rows * 32);
  const size_t xsb_b = (size_t)nca * mt * gpa * 2;  // the second entry's sums after the first's
  const int xw0 = W > C ? C : 0, xnw = W - xw0;
  if ((xsa || xsbe) && wave >= xw0) {
    const int na = xsa ? nca * mt * gpa : 0, ntot = na + (xsbe ? ncb * mt * gpb : 0);
    for (int i = (wave - xw0) * 64 + lane; i < ntot; i += xnw * 64) {
      const bool second = i >= na;
      KEntry* e = second ? eb : ea;
      const int ii = second ? i - na : i, GPC = second ? gpb : gpa, TW = 128 * GPC;
      const int gq = ii % GPC, r = ii / GPC, tok = r % mt, lc = r / mt;
      const int KT = e->M.KT, K = e->M.K;
      int c = (second ? cb0 : ca0) + lc;
      if (c >= KT) c -= KT;
      const uint4* x4 = reinterpret_cast<const uint4*>(e->X2 + (size_t)tok * (K / 2) + (size_t)c * (TW / 2) + 64 * gq);
      uint64_t hi4 = 0, lo4 = 0;
#pragma unroll
      for (int k = 0; k < 4; ++k) {  // sub-block 4 gq + k: 32 fp16 = 4 uint4
        uint4 v[4];
#pragma unroll
        for (int w = 0; w < 4; ++w) v[w] = x4[4 * k + w];
        const float sum = xsum_sub<32>([&](int d) {
          const uint4& u = v[d >> 2];
          return (d & 3) == 0 ? u.x : (d & 3) == 1 ? u.y : (d & 3) == 2 ? u.z : u.w;
        });
        const _Float16 hi = (_Float16)sum;
        hi4 |= (uint64_t)__builtin_bit_cast(uint16_t, hi) << (16 * k);
        lo4 |= (uint64_t)__builtin_bit_cast(uint16_t, (_Float16)(sum - (float)hi)) << (16 * k);
      }
      uint64_t* xs = xsb + (second ? xsb_b : 0) + ((size_t)lc * mt + tok) * (GPC * 2) + 2 * gq;
      xs[0] = hi4;
      xs[1] = lo4;
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the stores are done
    if (lane == 0) __hip_atomic_fetch_add(xs_done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  }
  if (have && wave >= C) {
    ask((uint32_t)wave);
    copy_tile(sec ? eb : ea, t, true);
  }
  if (wave == W - 1) {  // the block's row counts (and word offsets) into the scalar cache, read at each claim, by
                        // the wave whose first tile comes last
    uint32_t warm = 0;
    auto touch = [&](KEntry* e, int u0, int u1) {
      if (e->list) return;
      const bool tb = e->M.tstride == 0;
      for (int u = u0; u <= u1; u += 16) warm += (tb ? ((KU32*)e->M.tbase)[u] : 0u) + ((KU16*)e->M.rows)[u];
      warm += (tb ? ((KU32*)e->M.tbase)[u1] : 0u) + ((KU16*)e->M.rows)[u1];
    };
    touch(ea, T0 - ea->tile0, min(Tl, ea->tile0 + ea->ntile - 1) - ea->tile0);
    if (mb != ma) touch(eb, 0, Tl - eb->tile0);
    asm volatile("" ::"s"(warm));
  }
  // every share of the x sums stored: checked at each tile start until it holds; a tile that starts earlier (a
  // first tile) reads its sums after its decode instead
  bool xs_ready = !(xsa || xsbe);
#pragma unroll 1
  while (have) {
    if (!xs_ready)
      xs_ready = __builtin_amdgcn_readfirstlane((int)__hip_atomic_load(xs_done, __ATOMIC_RELAXED,
                                                                        __HIP_MEMORY_SCOPE_WORKGROUP)) >= xnw;
    asm volatile("" ::: "memory");
    // one tile of format KQ (KQB: a tile of the plan's entries from nfa on)
    auto tile = [&](auto kq) __attribute__((always_inline)) {
      constexpr int KQ = decltype(kq)::value;
      constexpr int SYMB = kq_symbits(KQ);
      constexpr int TW = SYMB == 4 ? 2 * TK : TK;
      constexpr int SB = kq_sbytes(KQ);
      constexpr int NSB = TW / 256;   // super-blocks per tile row
      constexpr int NPR = TW / 64;    // x register pairs per quad (16 position blocks of 4 weights each)
      constexpr int GW = kq_gw(KQ), NSUB = 256 / GW;          // weights per sub-block, sub-blocks per super-block
      constexpr int GPSUB = (GW / (SYMB == 4 ? 2 : 1)) / 16;  // 16-symbol groups per sub-block
      constexpr int GPC = TW / 128;                           // groups of 4 sub-blocks per tile column
      constexpr bool XSUMS = KQ != KQ_Q6_K;                   // an offset term over the sub-blocks' x sums
      // the weights enter unscaled: 4-bit codes as fp16 denormals q 2^-24 (one byte permute per entry), 8-bit formats
      // as fp16(q) from the table; each chain's sums per sub-block are scaled by dA s_j (2^24 s_j) when it ends
      constexpr float WSCALE = SYMB == 4 ? 16777216.f : 1.f;
      const bool xs_late = !xs_ready;
      const int cur = sec;
      const bool second = sec != 0;
      KEntry* ep = second ? eb : ea;
      const auto& E = *ep;
      const auto& M = E.M;
      const int KT = M.KT, N = M.N, K = M.K;
      const int tc = t % KT, tr = t / KT;
      const uint8_t* srow = M.side + side_record(tr * TN, tc * NSB, KT, NSB) * SB + (uint32_t)(lane * SB);
      uint32_t sw[NSB][5];
  #pragma unroll
      for (int sb = 0; sb < NSB; ++sb) side_load<KQ>(srow + sb * (TN * SB), sw[sb]);
      uint32_t P[NC];
      {
        uint32_t P8[8];
        tile_chain_starts(M, t, f, s, P8);
  #pragma unroll
        for (int j = 0; j < NC; ++j) P[j] = P8[j * (8 / NC)];
      }
      const uint32_t tsel = second ? 4u * LUTN : 0u;
      // x of the tile column: register pair m of quad q, lane 4 b + i = token 4 q + i's weights 4 (16 m + b) .. + 3
      // (zero for tokens >= mt)
      h4v xa[NQ][NPR], xs[NQ];
  #pragma unroll
      for (int q = 0; q < NQ; ++q) {
        const int tok = 4 * q + qi;
        const bool ok = tok < mt;
        const uint32_t* xrow = E.X2 + (size_t)(ok ? tok : 0) * (K / 2) + (size_t)tc * (TW / 2);
  #pragma unroll
        for (int m = 0; m < NPR; ++m) {
          const uint2 v = ok ? *reinterpret_cast<const uint2*>(xrow + 2 * (16 * m + qb)) : make_uint2(0u, 0u);
          xa[q][m] = __builtin_bit_cast(h4v, v);
        }
      }
      // XS: lane 4 b + i = token 4 q + i's sums of 4 sub-blocks (hi or lo halves), block b = 2 (2 sb + half) + (lo)
      auto load_xs = [&]() {
  #pragma unroll
        for (int q = 0; q < NQ; ++q) {
          const int tok = 4 * q + qi, cb = qb & 7, lo = cb & 1, sh = cb >> 1;  // sh = 2 sb + half
          uint64_t sv = 0;
          if (XSUMS && tok < mt && qb < 4 * NSB) {
            const int lc = (tc - (second ? cb0 : ca0) + KT) % KT;  // the column's slot
            sv = xsb[(second ? xsb_b : 0) + ((size_t)lc * mt + tok) * (GPC * 2) + 2 * sh + lo];
          }
          xs[q] = __builtin_bit_cast(h4v, sv);
        }
      };
      if (!xs_late) load_xs();
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the tile is in LDS, the pending tile's partials stored
      if (lane == 0) __hip_atomic_fetch_add(landed, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      if (pend >= 0 && lane == 0)
        pold = __hip_atomic_fetch_add((pend ? eb : ea)->cnt + ptr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      uint32_t slot[NC], A[NC], B[NC], C[NC];
  #pragma unroll
      for (int j = 0; j < NC; ++j) {
        slot[j] = __builtin_amdgcn_ubfe(P[j], 5, 8);
        A[j] = *(LdsU32*)(rlb + ((slot[j] - 2u) << 7));
        B[j] = *(LdsU32*)(rlb + ((slot[j] - 1u) << 7));
        C[j] = *(LdsU32*)(rlb + (slot[j] << 7));
      }
      // the lane's sub-block scales (bytes, low first) per super-block
      uint64_t scq[NSB], scq2[NSB];  // scales of sub-blocks 0..7 and (Q6_K) 8..15
      float dA[NSB], dB[NSB];
  #pragma unroll
      for (int sb = 0; sb < NSB; ++sb) side_packed<KQ>(sw[sb], scq[sb], scq2[sb], dA[sb], dB[sb]);
      // s_j of sub-block js of the tile row (a constant after unrolling), extracted where it is used: the scale words
      // are opaque here, so the compiler does not hold every converted scale through the decode (8 tokens of IQ4_XS
      // spilled)
      auto scale_of = [&](int js) -> float {
        const int jsb = js / NSUB, jj = js % NSUB;
        uint32_t w = (uint32_t)((jj >= 8 ? scq2[jsb] : scq[jsb]) >> (32 * ((jj % 8) / 4)));
        asm("" : "+v"(w));
        const uint32_t b = (w >> (8 * (jj % 4))) & 255u;
        return (KQ == KQ_Q6_K || KQ == KQ_IQ4_XS) ? (float)(int)(int8_t)(uint8_t)b : (float)b;
      };
      f4v acc[NC][NQ];  // per chain: its current sub-block's sums, 4 tokens per register quad
      float fa[NQ][4];  // scaled sums of the finished sub-blocks
  #pragma unroll
      for (int q = 0; q < NQ; ++q) {
  #pragma unroll
        for (int i = 0; i < 4; ++i) fa[q][i] = 0.f;
  #pragma unroll
        for (int j = 0; j < NC; ++j) acc[j][q] = f4v{0.f, 0.f, 0.f, 0.f};
      }
      uint32_t wprev[NC];
  #pragma unroll
      for (int j = 0; j < NC; ++j) wprev[j] = 0;
      static_for<NG>([&](auto gic) {
        constexpr int gi = decltype(gic)::value;
        static_for<8>([&](auto pc) {
          constexpr int p = decltype(pc)::value;
          uint32_t w1[NC], e1[NC], e2[NC];
  #pragma unroll
          for (int j = 0; j < NC; ++j) {
            w1[j] = __builtin_amdgcn_alignbit(B[j], A[j], P[j]);
            e1[j] = *(LdsU32*)table_addr(w1[j], tsel, tmask);
          }
          __builtin_amdgcn_sched_barrier(0);
  #pragma unroll
          for (int j = 0; j < NC; ++j) e2[j] = *(LdsU32*)table_addr(w1[j] >> (e1[j] & 31u), tsel, tmask);
          __builtin_amdgcn_sched_barrier(0);
  #pragma unroll
          for (int j = 0; j < NC; ++j) {
            P[j] = P[j] + e1[j] + e2[j];
            const uint32_t nslot = __builtin_amdgcn_ubfe(P[j], 5, 8);
            const bool slide = nslot != slot[j];
            A[j] = slide ? B[j] : A[j];
            B[j] = slide ? C[j] : B[j];
            slot[j] = nslot;
            C[j] = *(LdsU32*)(rlb + (nslot << 7));
          }
          static_for<NC>([&](auto jc) {
            constexpr int j = decltype(jc)::value;
            if constexpr (SYMB == 4) {  // 4 codes as fp16 denormals q 2^-24, in weight order
              const uint2 wv = make_uint2(__builtin_amdgcn_perm(e1[j], e1[j], 0x0C030C02u),
                                          __builtin_amdgcn_perm(e2[j], e2[j], 0x0C030C02u));
              constexpr int g = NG * j + gi;           // 16-symbol group within the tile row
              constexpr int pb = 8 * g + p;            // position block of the 4 weights within the tile row
  #pragma unroll
              for (int q = 0; q < NQ; ++q)
                acc[j][q] = mfma4_from<pb & 15>(xa[q][pb >> 4], __builtin_bit_cast(h4v, wv), acc[j][q]);
            } else {  // 2 codes per pair (fp16(q) in the entries' upper halves), 4 per product
              const uint32_t v = __builtin_amdgcn_perm(e2[j], e1[j], 0x07060302u);
              if constexpr (p & 1) {
                constexpr int pb = 4 * (NG * j + gi) + p / 2;
  #pragma unroll
                for (int q = 0; q < NQ; ++q)
                  acc[j][q] = mfma4_from<pb & 15>(xa[q][pb >> 4], __builtin_bit_cast(h4v, make_uint2(wprev[j], v)), acc[j][q]);
              } else {
                wprev[j] = v;
              }
            }
          });
        });
        // sub-blocks ending with this group: y += dA s_j acc (2^24 s_j for the denormal form), then acc = 0
        if constexpr ((gi + 1) % GPSUB == 0) {
          static_for<NC>([&](auto jc) {
            constexpr int j = decltype(jc)::value;
            constexpr int js = (NG * j + gi) / GPSUB;  // sub-block within the tile row
            const float sa = dA[js / NSUB] * WSCALE * scale_of(js);
  #pragma unroll
            for (int q = 0; q < NQ; ++q) {
  #pragma unroll
              for (int i = 0; i < 4; ++i) fa[q][i] = fmaf(acc[j][q][i], sa, fa[q][i]);
              acc[j][q] = f4v{0.f, 0.f, 0.f, 0.f};
            }
          });
        }
      });
      // the products are formed here, not sunk past the claim and the copy below
  #pragma unroll
      for (int q = 0; q < NQ; ++q)
  #pragma unroll
        for (int i = 0; i < 4; ++i) asm volatile("" : "+v"(fa[q][i]));
      if (xs_late) {  // this tile's sums, now that every share is stored
        while (__hip_atomic_load(xs_done, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < (uint32_t)xnw)
          __builtin_amdgcn_s_sleep(2);
        asm volatile("" ::: "memory");
        load_xs();
        xs_ready = true;
      }
      // the next tile: claimed and its copy issued now (the claim's wait also covers every LDS read of the decode,
      // so the buffer is free); the pending row's counter value arrived during the decode
      {
        uint32_t nx = 0;
        if (lane == 0) nx = __hip_atomic_fetch_add(next, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        n = __builtin_amdgcn_readfirstlane((int)nx);
      }
      const uint32_t old = pend >= 0 ? (uint32_t)__builtin_amdgcn_readlane((int)pold, 0) : 0u;
      have = n < per && T0 + n < plan.ntiles;
      if (have) {
        tile_of(n, sec, t);
        uint32_t k = 0;
        if (lane == 0) k = __hip_atomic_fetch_add(asked, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        ask((uint32_t)__builtin_amdgcn_readfirstlane((int)k));
        copy_tile(sec ? eb : ea, t, false);
      }
      // offset terms: per super-block and token, sum_j c_j (sum x)_j from the hi and lo halves of the sums, c_j = the
      // mins m_j (Q4_K / Q5_K) or the signed scales s_j (IQ4_XS)
      f4v mac[NSB][NQ];
  #pragma unroll
      for (int sb = 0; sb < NSB; ++sb) {
        if constexpr (!XSUMS) break;
        float mf[8];
        if constexpr (KQ == KQ_IQ4_XS) {
  #pragma unroll
          for (int jj = 0; jj < 8; ++jj) mf[jj] = scale_of(8 * sb + jj);
        } else {
          side_mins(sw[sb], mf);
        }
        const h4v m0 = h4v{(_Float16)mf[0], (_Float16)mf[1], (_Float16)mf[2], (_Float16)mf[3]};
        const h4v m1 = h4v{(_Float16)mf[4], (_Float16)mf[5], (_Float16)mf[6], (_Float16)mf[7]};
  #pragma unroll
        for (int q = 0; q < NQ; ++q) {
          f4v r = {0.f, 0.f, 0.f, 0.f};
          if (sb == 0) {
            r = mfma4_from<0>(xs[q], m0, r);
            r = mfma4_from<1>(xs[q], m0, r);
            r = mfma4_from<2>(xs[q], m1, r);
            r = mfma4_from<3>(xs[q], m1, r);
          } else {
            r = mfma4_from<4>(xs[q], m0, r);
            r = mfma4_from<5>(xs[q], m0, r);
            r = mfma4_from<6>(xs[q], m1, r);
            r = mfma4_from<7>(xs[q], m1, r);
          }
          mac[sb][q] = r;
        }
      }
      float* out = E.P + (size_t)tc * mt * N + (size_t)tr * TN + (uint32_t)lane;
  #pragma unroll
      for (int q = 0; q < NQ; ++q)
  #pragma unroll
        for (int i = 0; i < 4; ++i) {
          float tot = fa[q][i];
          if constexpr (XSUMS) {
  #pragma unroll
            for (int sb = 0; sb < NSB; ++sb)
              tot = fmaf(KQ == KQ_IQ4_XS ? -128.f * dA[sb] : -dB[sb], mac[sb][q][i], tot);
          }
          if (4 * q + i < mt) __hip_atomic_store(out + (size_t)(4 * q + i) * N, tot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      if (pend >= 0 && old == (uint32_t)(pKT - 1)) row_sum(*(pend ? eb : ea), ptr, pKT, pN, lane, mt);
      pend = -1;
      if (E.Y) {
        pend = cur;
        ptr = tr;
        pKT = KT;
        pN = N;
      }
    };
    if constexpr (KQB != KQA) {
      if (__builtin_amdgcn_readfirstlane((sec ? mb : ma) >= plan.nfa ? 1 : 0)) tile(KqTag<KQB>{});
      else tile(KqTag<KQA>{});
    } else {
      tile(KqTag<KQA>{});
    }
  }
  if (pend >= 0) {
    if (lane == 0)
      pold = __hip_atomic_fetch_add((pend ? eb : ea)->cnt + ptr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    finish_pending();
  }
}

template <int KQ, int NTAB, int MT, int KQB = KQ>
static hipError_t tiles_mma_launch_t(const FlatPlan& p, int per, int buf_rows, hipStream_t s) {
  const size_t smem = (size_t)p.W * buf_rows * 128 + tiles_mma_xs_bytes(p, per);
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_fused_tiles_mma<KQ, NTAB, MT, KQB>),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
  if (e != hipSuccess) return e;
  const int blocks = (p.ntiles + per - 1) / per;
  hipLaunchKernelGGL((k_fused_tiles_mma<KQ, NTAB, MT, KQB>), dim3(blocks), dim3(p.W * 64), smem, s, p, per,
                     buf_rows);
  return hipGetLastError();
}

// two K-quant types in one launch: entries [0, nfa) of type KQA < KQB, the rest of KQB
template <int KQA, int KQB>
static hipError_t tiles_mma_launch_mixed_t(const FlatPlan& p, int per, int buf_rows, hipStream_t s) {
  return p.mt <= 4 ? tiles_mma_launch_t<KQA, 2, 4, KQB>(p, per, buf_rows, s)
                   : tiles_mma_launch_t<KQA, 2, 8, KQB>(p, per, buf_rows, s);
}
static hipError_t tiles_mma_launch_mixed(int kqa, int kqb, const FlatPlan& p, int per, int buf_rows, hipStream_t s) {
  switch (kqa * 8 + kqb) {
    case KQ_Q4_K * 8 + KQ_Q5_K: return tiles_mma_launch_mixed_t<KQ_Q4_K, KQ_Q5_K>(p, per, buf_rows, s);
    case KQ_Q4_K * 8 + KQ_Q6_K: return tiles_mma_launch_mixed_t<KQ_Q4_K, KQ_Q6_K>(p, per, buf_rows, s);
    case KQ_Q4_K * 8 + KQ_IQ4_XS: return tiles_mma_launch_mixed_t<KQ_Q4_K, KQ_IQ4_XS>(p, per, buf_rows, s);
    case KQ_Q5_K * 8 + KQ_Q6_K: return tiles_mma_launch_mixed_t<KQ_Q5_K, KQ_Q6_K>(p, per, buf_rows, s);
    case KQ_Q5_K * 8 + KQ_IQ4_XS: return tiles_mma_launch_mixed_t<KQ_Q5_K, KQ_IQ4_XS>(p, per, buf_rows, s);
    case KQ_Q6_K * 8 + KQ_IQ4_XS: return tiles_mma_launch_mixed_t<KQ_Q6_K, KQ_IQ4_XS>(p, per, buf_rows, s);
    default: return hipErrorInvalidValue;
  }
}

template <int KQ>
static hipError_t tiles_mma_launch(const FlatPlan& p, int per, int buf_rows, hipStream_t s) {
  const bool one = p.n == 1;
  if (p.mt <= 4) return one ? tiles_mma_launch_t<KQ, 1, 4>(p, per, buf_rows, s) : tiles_mma_launch_t<KQ, 2, 4>(p, per, buf_rows, s);
  return one ? tiles_mma_launch_t<KQ, 1, 8>(p, per, buf_rows, s) : tiles_mma_launch_t<KQ, 2, 8>(p, per, buf_rows, s);
}

// ── whole-tile kernel on the matrix cores for int8 activations (2..8 tokens, every format) ─────────────────
// The decode and tile pipeline of k_fused_tiles_mma; the products on v_mfma_i32_4x4x4i8 over the int8 grid values
// of the load-time int8 table (Q4_K q, Q5_K q, Q6_K q - 32, IQ4_XS kv[q]) and x quantized per block of 32
// (launch_quant_x8: XQ, and per block DX = d, SX = d sum q). Block b of the instruction computes
// D[i][j] = sum_k A[4 b' + i][k] B[4 b + j][k] into lane 4 b + j, register i (checked on the GPU): B = the lane's own
// 4 weights of a position block, A = 4 tokens' int8 x there, broadcast from block b' of a register that holds 16
// position blocks (one dword per lane). Each chain's integer sums per sub-block (exact) are folded into fp32 when
// the sub-block ends: y_t += dA s_j d_x(t, block) acc; the Q4_K / Q5_K offset term dB sum_j m_j SX(t, j) runs on
// v_mfma_f32_4x4x4f16 with SX split into fp16 hi and lo, as the fp16 kernel's mins term. Each token's values agree
// with its own m = 1 int8 launch to fp32 rounding (another order of the same exact sub-block sums).
template <int KQ, int NTAB, int MT>
__global__ void __launch_bounds__(64 * tiles_mma_waves(KQ, MT), 1)
k_fused_tiles_mma8(FlatPlan plan, int per, int buf_rows) {
  static_assert(MT == 4 || MT == 8, "4 or 8 token slots");
  constexpr int SYMB = kq_symbits(KQ);
  constexpr int TW = SYMB == 4 ? 2 * TK : TK;
  constexpr int SB = kq_sbytes(KQ), GW = kq_gw(KQ);
  constexpr int NSB = TW / 256;                          // super-blocks per tile row
  constexpr int NSUB = 256 / GW;                         // sub-blocks per super-block
  constexpr int GPSUB = (GW / (SYMB == 4 ? 2 : 1)) / 16;  // 16-symbol groups per sub-block (2 for Q5_K, else 1)
  constexpr bool MINS = KQ == KQ_Q4_K || KQ == KQ_Q5_K;
  constexpr bool SIGNED = KQ == KQ_Q6_K || KQ == KQ_IQ4_XS;  // signed sub-block scales
  constexpr int XB = TW / 32;                            // x blocks of 32 per tile column
  constexpr int NQ = MT / 4;                             // token quads
  constexpr int NPR = TW / 64;                           // x registers per quad (16 position blocks of 4 each)
  constexpr int NC = 4, NG = 16 / NC;                    // chains per lane (64 symbols each), groups per chain
  typedef __attribute__((address_space(3))) const uint32_t LdsU32;
  typedef __attribute__((address_space(4))) const char KChar;
  typedef __attribute__((address_space(4))) const FlatEntry KEntry;
  typedef __attribute__((address_space(4))) const uint32_t KU32;
  typedef __attribute__((address_space(4))) const uint16_t KU16;
  __shared__ uint32_t lut4[NTAB * LUTN + 4];
  extern __shared__ __align__(16) uint32_t tbuf[];

  KChar* kbase = (KChar*)__builtin_amdgcn_kernarg_segment_ptr();
  const int W = plan.W, T0 = (int)blockIdx.x * per, Tl = min(T0 + per, plan.ntiles) - 1, mt = plan.mt;
  int ma = 0, mb = 0;
#pragma unroll
  for (int i = 1; i < MAX_GROUP; ++i) {
    if (i < plan.n && T0 >= plan.e[i].tile0) ma = i;
    if (i < plan.n && Tl >= plan.e[i].tile0) mb = i;
  }
  KEntry* ea = (KEntry*)(kbase + offsetof(FlatPlan, e) + (size_t)ma * sizeof(FlatEntry));
  KEntry* eb = (KEntry*)(kbase + offsetof(FlatPlan, e) + (size_t)mb * sizeof(FlatEntry));
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63, s = lane & 31, f = lane >> 5;
  const int qb = lane >> 2, qi = lane & 3;  // 4-lane block and the lane's place in it
  {  // the int8 tables: 1 KB direct-to-LDS loads, chunk c (8 per table) by wave c mod W
    const uint4* ta = reinterpret_cast<const uint4*>(ea->M.luti8);
    const uint4* tb = reinterpret_cast<const uint4*>(eb->M.luti8);
    const int nchunk = (NTAB > 1 && mb != ma) ? 16 : 8;
    for (int c = wave; c < nchunk; c += W)
      __builtin_amdgcn_global_load_lds((c < 8 ? ta : tb) + 64 * (c & 7) + lane,
                                       (__attribute__((address_space(3))) void*)(lut4 + 256 * c), 16, 0, 0);
  }
  // copies paced as in k_fused_tiles
  uint32_t* next = lut4 + NTAB * LUTN;
  uint32_t* asked = next + 1;
  uint32_t* landed = next + 2;
  const int C = min(W, TILES_COPIES);
  if (threadIdx.x == 0) {
    next[0] = (uint32_t)W;
    asked[0] = (uint32_t)W;
    landed[0] = 0u;
  }
  auto ask = [&](uint32_t k) {
    while (k >= (uint32_t)C + __hip_atomic_load(landed, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP))
      __builtin_amdgcn_s_sleep(2);
  };
  uint32_t* buf = tbuf + (size_t)wave * buf_rows * 32;
  const uint32_t rlb = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint32_t*)(buf + s);
  uint32_t tmask = 0x1FFCu;
  asm volatile("" : "+v"(tmask));
  auto tile_of = [&](int n, int& sec, int& t) {  // row-major, as k_fused_tiles
    const int T = T0 + n;
    sec = __builtin_amdgcn_readfirstlane((NTAB > 1 && mb != ma && T >= eb->tile0) ? 1 : 0);
    KEntry* e = sec ? eb : ea;
    const int u = T - e->tile0;
    t = __builtin_amdgcn_readfirstlane(e->list ? (int)((KU32*)e->list)[u] : u);
  };
  auto copy_tile = [&](KEntry* e, int t, bool slot) -> int {  // as k_fused_tiles (a first copy takes the slot)
    const int ts = e->M.tstride;
    const int nrow = (slot && ts > 0) ? ts : (int)((KU16*)e->M.rows)[t];
    const uint32_t* wt = e->M.words + (ts > 0 ? (size_t)32 * ts * t : (size_t)((KU32*)e->M.tbase)[t]);
    const uint4* src = reinterpret_cast<const uint4*>(wt) + lane;
    const int nc = (nrow + 7) / 8;
    for (int i = 0; i < nc; ++i)
      if (lane < 8 * (nrow - 8 * i))
        __builtin_amdgcn_global_load_lds(src + 64 * i, (__attribute__((address_space(3))) void*)(buf + 256 * i), 16, 0, 0);
    return nc;
  };
  int pend = -1;
  int ptr = 0, pKT = 0, pN = 0;
  uint32_t pold = 0;
  auto finish_pending = [&]() {
    if (pend < 0) return;
    const uint32_t old = (uint32_t)__builtin_amdgcn_readlane((int)pold, 0);
    if (old == (uint32_t)(pKT - 1)) row_sum(*(pend ? eb : ea), ptr, pKT, pN, lane, mt);
    pend = -1;
  };
  int n = wave;
  bool have = n < per && T0 + n < plan.ntiles;
  int sec = 0, t = 0, ncopy = 0;
  if (have) tile_of(n, sec, t);
  if (have && wave < C) ncopy = copy_tile(sec ? eb : ea, t, true);
  wait_vmcnt_upto(ncopy);
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  if (have && wave >= C) {
    ask((uint32_t)wave);
    copy_tile(sec ? eb : ea, t, true);
  }
  if (wave == W - 1) {  // the block's row counts (and word offsets) into the scalar cache, read at each claim, by
                        // the wave whose first tile comes last
    uint32_t warm = 0;
    auto touch = [&](KEntry* e, int u0, int u1) {
      if (e->list) return;
      const bool tb = e->M.tstride == 0;
      for (int u = u0; u <= u1; u += 16) warm += (tb ? ((KU32*)e->M.tbase)[u] : 0u) + ((KU16*)e->M.rows)[u];
      warm += (tb ? ((KU32*)e->M.tbase)[u1] : 0u) + ((KU16*)e->M.rows)[u1];
    };
    touch(ea, T0 - ea->tile0, min(Tl, ea->tile0 + ea->ntile - 1) - ea->tile0);
    if (mb != ma) touch(eb, 0, Tl - eb->tile0);
    asm volatile("" ::"s"(warm));
  }
#pragma unroll 1
  while (have) {
    const int cur = sec;
    const bool second = sec != 0;
    KEntry* ep = second ? eb : ea;
    const auto& E = *ep;
    const auto& M = E.M;
    const int KT = M.KT, N = M.N, K = M.K;
    const int tc = t % KT, tr = t / KT;
    const uint8_t* srow = M.side + side_record(tr * TN, tc * NSB, KT, NSB) * SB + (uint32_t)(lane * SB);
    uint32_t sw[NSB][5];
#pragma unroll
    for (int sb = 0; sb < NSB; ++sb) side_load<KQ>(srow + sb * (TN * SB), sw[sb]);
    uint32_t P[NC];
    {
      uint32_t P8[8];
      tile_chain_starts(M, t, f, s, P8);
#pragma unroll
      for (int j = 0; j < NC; ++j) P[j] = P8[j * (8 / NC)];
    }
    const uint32_t tsel = second ? 4u * LUTN : 0u;
    // x of the tile column: register m of quad q, lane 4 b + i = token 4 q + i's int8 x at positions 4 (16 m + b) ..
    // + 3 (zero for tokens >= mt); its block scales d as two lane-distributed registers (value i = token i / XB,
    // block i % XB: read back with v_readlane)
    uint32_t xa[NQ][NPR];
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const int tok = 4 * q + qi;
      const bool ok = tok < mt;
      const uint32_t* xrow = reinterpret_cast<const uint32_t*>(E.XQ + (size_t)(ok ? tok : 0) * K + (size_t)tc * TW);
#pragma unroll
      for (int m = 0; m < NPR; ++m) xa[q][m] = ok ? xrow[16 * m + qb] : 0u;
    }
    float dxv[2];
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int v = 64 * r + lane, tok = v / XB;
      dxv[r] = tok < mt ? E.DX[(size_t)tok * (K / 32) + (size_t)tc * XB + v % XB] : 0.f;
    }
    // the offset term's A operand: lane 4 b + i = token 4 q + i's SX of 4 sub-blocks as fp16 hi or lo halves,
    // block b = 2 (2 sb + half) + (lo) (Q4_K / Q5_K: a sub-block is one x block)
    h4v xs[NQ];
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const int tok = 4 * q + qi, cb = qb & 7, lo = cb & 1, sh = cb >> 1;
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      if (MINS && tok < mt && qb < 4 * NSB) v = *reinterpret_cast<const float4*>(E.SX + (size_t)tok * (K / 32) + (size_t)tc * XB + 4 * sh);
      xs[q] = h4v{(_Float16)v.x, (_Float16)v.y, (_Float16)v.z, (_Float16)v.w};
      if (lo)
        xs[q] = h4v{(_Float16)(v.x - (float)xs[q][0]), (_Float16)(v.y - (float)xs[q][1]),
                    (_Float16)(v.z - (float)xs[q][2]), (_Float16)(v.w - (float)xs[q][3])};
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the tile is in LDS, the pending tile's partials stored
    if (lane == 0) __hip_atomic_fetch_add(landed, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    if (pend >= 0 && lane == 0)
      pold = __hip_atomic_fetch_add((pend ? eb : ea)->cnt + ptr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    uint32_t slot[NC], A[NC], B[NC], Cw[NC];
#pragma unroll
    for (int j = 0; j < NC; ++j) {
      slot[j] = __builtin_amdgcn_ubfe(P[j], 5, 8);
      A[j] = *(LdsU32*)(rlb + ((slot[j] - 2u) << 7));
      B[j] = *(LdsU32*)(rlb + ((slot[j] - 1u) << 7));
      Cw[j] = *(LdsU32*)(rlb + (slot[j] << 7));
    }
    uint64_t scq[NSB], scq2[NSB];
    float dA[NSB], dB[NSB];
#pragma unroll
    for (int sb = 0; sb < NSB; ++sb) side_packed<KQ>(sw[sb], scq[sb], scq2[sb], dA[sb], dB[sb]);
    v4i32 ia[NC][NQ];
    float fa[NQ][4];
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
#pragma unroll
      for (int i = 0; i < 4; ++i) fa[q][i] = 0.f;
#pragma unroll
      for (int j = 0; j < NC; ++j) ia[j][q] = v4i32{0, 0, 0, 0};
    }
    uint32_t wprev[NC];
#pragma unroll
    for (int j = 0; j < NC; ++j) wprev[j] = 0;
    static_for<NG>([&](auto gic) {
      constexpr int gi = decltype(gic)::value;
      static_for<8>([&](auto pc) {
        constexpr int p = decltype(pc)::value;
        uint32_t w1[NC], e1[NC], e2[NC];
#pragma unroll
        for (int j = 0; j < NC; ++j) {
          w1[j] = __builtin_amdgcn_alignbit(B[j], A[j], P[j]);
          e1[j] = *(LdsU32*)table_addr(w1[j], tsel, tmask);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < NC; ++j) e2[j] = *(LdsU32*)table_addr(w1[j] >> (e1[j] & 31u), tsel, tmask);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < NC; ++j) {
          P[j] = P[j] + e1[j] + e2[j];
          const uint32_t nslot = __builtin_amdgcn_ubfe(P[j], 5, 8);
          const bool slide = nslot != slot[j];
          A[j] = slide ? B[j] : A[j];
          B[j] = slide ? Cw[j] : B[j];
          slot[j] = nslot;
          Cw[j] = *(LdsU32*)(rlb + (nslot << 7));
        }
        static_for<NC>([&](auto jc) {
          constexpr int j = decltype(jc)::value;
          constexpr int g = NG * j + gi;  // 16-symbol group within the tile row
          if constexpr (SYMB == 4) {      // 4 weights: the grid bytes of both entries, in weight order
            constexpr int pb = 8 * g + p;
            const int w = (int)__builtin_amdgcn_perm(e2[j], e1[j], 0x07060302u);
#pragma unroll
            for (int q = 0; q < NQ; ++q)
              ia[j][q] = __builtin_amdgcn_mfma_i32_4x4x4i8((int)xa[q][pb >> 4], w, ia[j][q], 4, pb & 15, 0);
          } else {  // 2 weights per pair, 4 per product
            const uint32_t v = __builtin_amdgcn_perm(e2[j], e1[j], 0x0C0C0602u);
            if constexpr (p & 1) {
              constexpr int pb = 4 * g + p / 2;
#pragma unroll
              for (int q = 0; q < NQ; ++q)
                ia[j][q] = __builtin_amdgcn_mfma_i32_4x4x4i8((int)xa[q][pb >> 4], (int)(wprev[j] | v << 16), ia[j][q],
                                                              4, pb & 15, 0);
            } else {
              wprev[j] = v;
            }
          }
        });
      });
      // sub-blocks ending with this group: y_t += dA s_j d_x(t, block) acc, then acc = 0
      if constexpr ((gi + 1) % GPSUB == 0) {
        static_for<NC>([&](auto jc) {
          constexpr int j = decltype(jc)::value;
          constexpr int js = (NG * j + gi) / GPSUB;  // sub-block within the tile row
          constexpr int sb = js / NSUB, jj = js % NSUB, xb = js * GW / 32;
          const uint64_t sq = jj < 8 ? scq[sb] : scq2[sb];
          const uint32_t byte = (uint32_t)(sq >> (8 * (jj % 8))) & 255u;
          const float sa = dA[sb] * (SIGNED ? (float)(int)(int8_t)(uint8_t)byte : (float)byte);
#pragma unroll
          for (int q = 0; q < NQ; ++q)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int v = (4 * q + i) * XB + xb;  // a constant after unrolling
              const float dx = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, dxv[v >> 6]), v & 63));
              fa[q][i] = fmaf((float)ia[j][q][i], sa * dx, fa[q][i]);
              ia[j][q][i] = 0;
            }
        });
      }
    });
#pragma unroll
    for (int q = 0; q < NQ; ++q)
#pragma unroll
      for (int i = 0; i < 4; ++i) asm volatile("" : "+v"(fa[q][i]));
    // the next tile: claimed and its copy issued now (the claim's wait also covers every LDS read of the decode)
    {
      uint32_t nx = 0;
      if (lane == 0) nx = __hip_atomic_fetch_add(next, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      n = __builtin_amdgcn_readfirstlane((int)nx);
    }
    const uint32_t old = pend >= 0 ? (uint32_t)__builtin_amdgcn_readlane((int)pold, 0) : 0u;
    have = n < per && T0 + n < plan.ntiles;
    if (have) {
      tile_of(n, sec, t);
      uint32_t k = 0;
      if (lane == 0) k = __hip_atomic_fetch_add(asked, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      ask((uint32_t)__builtin_amdgcn_readfirstlane((int)k));
      copy_tile(sec ? eb : ea, t, false);
    }
    float* out = E.P + (size_t)tc * mt * N + (size_t)tr * TN + (uint32_t)lane;
    f4v mac[NSB][NQ];
    if constexpr (MINS) {  // per super-block and token, sum_j m_j SX_j from the hi and lo halves
#pragma unroll
      for (int sb = 0; sb < NSB; ++sb) {
        float mf[8];
        side_mins(sw[sb], mf);
        const h4v m0 = h4v{(_Float16)mf[0], (_Float16)mf[1], (_Float16)mf[2], (_Float16)mf[3]};
        const h4v m1 = h4v{(_Float16)mf[4], (_Float16)mf[5], (_Float16)mf[6], (_Float16)mf[7]};
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
          f4v r = {0.f, 0.f, 0.f, 0.f};
          if (sb == 0) {
            r = mfma4_from<0>(xs[q], m0, r);
            r = mfma4_from<1>(xs[q], m0, r);
            r = mfma4_from<2>(xs[q], m1, r);
            r = mfma4_from<3>(xs[q], m1, r);
          } else {
            r = mfma4_from<4>(xs[q], m0, r);
            r = mfma4_from<5>(xs[q], m0, r);
            r = mfma4_from<6>(xs[q], m1, r);
            r = mfma4_from<7>(xs[q], m1, r);
          }
          mac[sb][q] = r;
        }
      }
    }
#pragma unroll
    for (int q = 0; q < NQ; ++q)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float tot = fa[q][i];
        if constexpr (MINS) {
#pragma unroll
          for (int sb = 0; sb < NSB; ++sb) tot = fmaf(-dB[sb], mac[sb][q][i], tot);
        }
        if (4 * q + i < mt) __hip_atomic_store(out + (size_t)(4 * q + i) * N, tot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    if (pend >= 0 && old == (uint32_t)(pKT - 1)) row_sum(*(pend ? eb : ea), ptr, pKT, pN, lane, mt);
    pend = -1;
    if (E.Y) {
      pend = cur;
      ptr = tr;
      pKT = KT;
      pN = N;
    }
  }
  if (pend >= 0) {
    if (lane == 0)
      pold = __hip_atomic_fetch_add((pend ? eb : ea)->cnt + ptr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    finish_pending();
  }
}

template <int KQ, int NTAB, int MT>
static hipError_t tiles_mma8_launch_t(const FlatPlan& p, int per, int buf_rows, hipStream_t s) {
  const size_t smem = (size_t)p.W * buf_rows * 128;
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_fused_tiles_mma8<KQ, NTAB, MT>),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
  if (e != hipSuccess) return e;
  const int blocks = (p.ntiles + per - 1) / per;
  hipLaunchKernelGGL((k_fused_tiles_mma8<KQ, NTAB, MT>), dim3(blocks), dim3(p.W * 64), smem, s, p, per, buf_rows);
  return hipGetLastError();
}

template <int KQ>
static hipError_t tiles_mma8_launch(const FlatPlan& p, int per, int buf_rows, hipStream_t s) {
  const bool one = p.n == 1;
  if (p.mt <= 4) return one ? tiles_mma8_launch_t<KQ, 1, 4>(p, per, buf_rows, s) : tiles_mma8_launch_t<KQ, 2, 4>(p, per, buf_rows, s);
  return one ? tiles_mma8_launch_t<KQ, 1, 8>(p, per, buf_rows, s) : tiles_mma8_launch_t<KQ, 2, 8>(p, per, buf_rows, s);
}

template <int KQ, int NTAB, bool I8, bool CANON = false, int KQB = KQ>
static hipError_t tiles_launch_t(const FlatPlan& p, int per, int buf_rows, hipStream_t s) {
  const size_t smem = (size_t)p.W * buf_rows * 128;
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_fused_tiles<KQ, NTAB, I8, CANON, KQB>),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
  if (e != hipSuccess) return e;
  const int blocks = (p.ntiles + per - 1) / per;
  hipLaunchKernelGGL((k_fused_tiles<KQ, NTAB, I8, CANON, KQB>), dim3(blocks), dim3(p.W * 64), smem, s, p, per,
                     buf_rows);
  return hipGetLastError();
}

// two K-quant types in one launch (fp16 activations): entries [0, nfa) of type KQA < KQB, the rest of KQB
static hipError_t tiles_launch_mixed(int kqa, int kqb, const FlatPlan& p, int per, int buf_rows, hipStream_t s) {
  switch (kqa * 8 + kqb) {
    case KQ_Q4_K * 8 + KQ_Q5_K: return tiles_launch_t<KQ_Q4_K, 2, false, false, KQ_Q5_K>(p, per, buf_rows, s);
    case KQ_Q4_K * 8 + KQ_Q6_K: return tiles_launch_t<KQ_Q4_K, 2, false, false, KQ_Q6_K>(p, per, buf_rows, s);
    case KQ_Q4_K * 8 + KQ_IQ4_XS: return tiles_launch_t<KQ_Q4_K, 2, false, false, KQ_IQ4_XS>(p, per, buf_rows, s);
    case KQ_Q5_K * 8 + KQ_Q6_K: return tiles_launch_t<KQ_Q5_K, 2, false, false, KQ_Q6_K>(p, per, buf_rows, s);
    case KQ_Q5_K * 8 + KQ_IQ4_XS: return tiles_launch_t<KQ_Q5_K, 2, false, false, KQ_IQ4_XS>(p, per, buf_rows, s);
    case KQ_Q6_K * 8 + KQ_IQ4_XS: return tiles_launch_t<KQ_Q6_K, 2, false, false, KQ_IQ4_XS>(p, per, buf_rows, s);
    default: return hipErrorInvalidValue;
  }
}

template <int KQ>
static hipError_t tiles_launch(const FlatPlan& p, int per, int buf_rows, hipStream_t s) {
  const bool one = p.n == 1;  // one matrix: one table
  if (p.i8) return one ? tiles_launch_t<KQ, 1, true>(p, per, buf_rows, s) : tiles_launch_t<KQ, 2, true>(p, per, buf_rows, s);
  if (p.canon)
    return one ? tiles_launch_t<KQ, 1, false, true>(p, per, buf_rows, s) : tiles_launch_t<KQ, 2, false, true>(p, per, buf_rows, s);
  return one ? tiles_launch_t<KQ, 1, false>(p, per, buf_rows, s) : tiles_launch_t<KQ, 2, false>(p, per, buf_rows, s);
}

// word rows of a whole-tile kernel's tile buffer: the longest tile of the plan and the 2 rows its windows read past
// a lane's end (copies are masked to a tile's own rows, so no rounding to whole 1 KB copies is needed)
int tiles_buf_rows(const FlatPlan& p) {
  int r = 0;
  for (int i = 0; i < p.n; ++i) r = std::max(r, p.e[i].M.max_rows + 2);
  return r;
}

hipError_t launch_fused_tiles(const FlatPlan& p, int per, hipStream_t s) {
  if (p.n < 1 || p.n > MAX_GROUP || p.W < 1 || p.W > (p.canon ? TILES_CANON_WAVES : 16) || per < p.W ||
      p.ntiles < 1 || p.mt > 1)
    return hipErrorInvalidValue;
  // two K-quant types: entries [0, nfa) of the first (the smaller type code), the rest of the second
  const bool mixed = p.nfa > 0 && p.nfa < p.n;
  const int kqt = p.e[0].M.kqt, kqb = mixed ? p.e[p.nfa].M.kqt : kqt;
  if (mixed && (p.i8 || p.canon || kqb <= kqt)) return hipErrorInvalidValue;
  for (int i = 0; i < p.n; ++i) {
    const FlatEntry& e = p.e[i];
    const int end = i + 1 < p.n ? p.e[i + 1].tile0 : p.ntiles;
    // a block (`per` consecutive tiles) spans at most two matrices
    if (e.M.kqt != (mixed && i >= p.nfa ? kqb : kqt) || !e.M.dsplit || !e.M.mid || !e.M.lut4 || !e.M.rows || e.M.packed || e.tile0 + e.ntile != end ||
        e.ntile < 1 || (p.n > 1 && e.ntile < per) || (!e.list && e.ntile != e.M.NT * e.M.KT) ||
        (i == 0 && e.tile0 != 0) || (p.i8 && (!e.M.luti8 || !e.XQ || !e.DX || !e.SX)) ||
        (p.canon && (p.i8 || !e.M.canon)))
      return hipErrorInvalidValue;
  }
  const int rows = tiles_buf_rows(p);
  if (rows > 256 || (size_t)p.W * rows * 128 + (p.n > 1 ? 2 : 1) * 4 * LUTN + 4 * (4 + TILES_ROWC) > 160 * 1024)
    return hipErrorInvalidValue;
  if (mixed) return tiles_launch_mixed(kqt, kqb, p, per, rows, s);
  switch (kqt) {
    case KQ_Q4_K: return tiles_launch<KQ_Q4_K>(p, per, rows, s);
    case KQ_Q5_K: return tiles_launch<KQ_Q5_K>(p, per, rows, s);
    case KQ_Q6_K: return tiles_launch<KQ_Q6_K>(p, per, rows, s);
    case KQ_IQ4_XS: return tiles_launch<KQ_IQ4_XS>(p, per, rows, s);
    default: return hipErrorInvalidValue;
  }
}

template <int KQ, int NTAB>
static hipError_t halves_launch_t(const FlatPlan& p, int per, int ubuf_rows, hipStream_t s) {
  const size_t smem = (size_t)p.W * 2 * ubuf_rows * 128;
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_fused_halves<KQ, NTAB>),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
  if (e != hipSuccess) return e;
  const int blocks = (p.ntiles + per - 1) / per;
  hipLaunchKernelGGL((k_fused_halves<KQ, NTAB>), dim3(blocks), dim3(p.W * 64), smem, s, p, per, ubuf_rows);
  return hipGetLastError();
}

template <int KQ>
static hipError_t halves_launch(const FlatPlan& p, int per, int ubuf_rows, hipStream_t s) {
  return p.n == 1 ? halves_launch_t<KQ, 1>(p, per, ubuf_rows, s) : halves_launch_t<KQ, 2>(p, per, ubuf_rows, s);
}

int halves_buf_rows(const FlatPlan& p) {
  int r = 0;
  for (int i = 0; i < p.n; ++i) r = std::max(r, p.e[i].M.max_hrows + 2);
  return r;
}

hipError_t launch_fused_halves(const FlatPlan& p, int per, hipStream_t s) {
  if (p.n < 1 || p.n > MAX_GROUP || p.W < 1 || p.W > 16 || 2 * per < p.W || p.ntiles < 1 || p.mt > 1 || p.i8)
    return hipErrorInvalidValue;
  const int kqt = p.e[0].M.kqt;
  for (int i = 0; i < p.n; ++i) {
    const FlatEntry& e = p.e[i];
    const int end = i + 1 < p.n ? p.e[i + 1].tile0 : p.ntiles;
    // a block (`per` consecutive tiles) spans at most two matrices
    if (e.M.kqt != kqt || !e.M.split || !e.M.lut4 || !e.M.rows || !e.M.hrow || e.M.packed || !e.X2 || !e.P ||
        (e.Y && !e.cnt) || e.tile0 + e.ntile != end || e.ntile < 1 || (p.n > 1 && e.ntile < per) ||
        (!e.list && e.ntile != e.M.NT * e.M.KT) || (i == 0 && e.tile0 != 0))
      return hipErrorInvalidValue;
  }
  const int rows = halves_buf_rows(p);
  if (rows > 256 || (size_t)p.W * 2 * rows * 128 + (p.n > 1 ? 2 : 1) * 4 * LUTN > 160 * 1024)
    return hipErrorInvalidValue;
  switch (kqt) {
    case KQ_Q4_K: return halves_launch<KQ_Q4_K>(p, per, rows, s);
    case KQ_Q5_K: return halves_launch<KQ_Q5_K>(p, per, rows, s);
    case KQ_Q6_K: return halves_launch<KQ_Q6_K>(p, per, rows, s);
    case KQ_IQ4_XS: return halves_launch<KQ_IQ4_XS>(p, per, rows, s);
    default: return hipErrorInvalidValue;
  }
}

size_t tiles_mma_xs_bytes(const FlatPlan& p, int per) {
  // a block's tiles lie in at most per tile columns; per column and token 4 bytes per sub-block (int8 activations
  // bring their block sums: none)
  if (p.i8) return 0;
  int tw = 0;
  for (int i = 0; i < p.n; ++i) tw = std::max(tw, kq_symbits(p.e[i].M.kqt) == 4 ? 2 * TK : TK);
  return (size_t)std::max(per, 0) * std::max(p.mt, 0) * tw / 32 * 4;
}

int tiles_mma_max_waves(int kqt, int mt) { return tiles_mma_waves(kqt, mt <= 4 ? 4 : 8); }

hipError_t launch_fused_tiles_mma8(const FlatPlan& p, int per, hipStream_t s) {
  if (p.n < 1 || p.n > MAX_GROUP || p.W < 1 || per < p.W || p.ntiles < 1 || p.mt < 1 || p.mt > 8 || !p.i8 ||
      p.W > tiles_mma_max_waves(p.e[0].M.kqt, p.mt))
    return hipErrorInvalidValue;
  const int kqt = p.e[0].M.kqt;
  for (int i = 0; i < p.n; ++i) {
    const FlatEntry& e = p.e[i];
    const int end = i + 1 < p.n ? p.e[i + 1].tile0 : p.ntiles;
    if (e.M.kqt != kqt || !e.M.dsplit || !e.M.mid || !e.M.luti8 || !e.M.rows || e.M.packed || !e.XQ || !e.DX ||
        !e.SX || e.tile0 + e.ntile != end || e.ntile < 1 || (p.n > 1 && e.ntile < per) || e.list ||
        e.ntile != e.M.NT * e.M.KT || (i == 0 && e.tile0 != 0))
      return hipErrorInvalidValue;
  }
  const int rows = tiles_buf_rows(p);
  if (rows > 256 || (size_t)p.W * rows * 128 + (p.n > 1 ? 2 : 1) * 4 * LUTN + 16 > 160 * 1024)
    return hipErrorInvalidValue;
  switch (kqt) {
    case KQ_Q4_K: return tiles_mma8_launch<KQ_Q4_K>(p, per, rows, s);
    case KQ_Q5_K: return tiles_mma8_launch<KQ_Q5_K>(p, per, rows, s);
    case KQ_Q6_K: return tiles_mma8_launch<KQ_Q6_K>(p, per, rows, s);
    case KQ_IQ4_XS: return tiles_mma8_launch<KQ_IQ4_XS>(p, per, rows, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_fused_tiles_mma(const FlatPlan& p, int per, hipStream_t s) {
  if (p.n < 1 || p.n > MAX_GROUP || p.W < 1 || per < p.W || p.ntiles < 1 || p.mt < 1 || p.mt > 8 || p.i8)
    return hipErrorInvalidValue;
  // two K-quant types: entries [0, nfa) of the first (the smaller type code), the rest of the second
  const bool mixed = p.nfa > 0 && p.nfa < p.n;
  const int kqt = p.e[0].M.kqt, kqb = mixed ? p.e[p.nfa].M.kqt : kqt;
  if ((mixed && kqb <= kqt) || p.W > tiles_mma_max_waves(kqt, p.mt) || p.W > tiles_mma_max_waves(kqb, p.mt))
    return hipErrorInvalidValue;
  for (int i = 0; i < p.n; ++i) {
    const FlatEntry& e = p.e[i];
    const int end = i + 1 < p.n ? p.e[i + 1].tile0 : p.ntiles;
    if (e.M.kqt != (mixed && i >= p.nfa ? kqb : kqt) || !e.M.dsplit || !e.M.mid || !e.M.lut4 || !e.M.rows || e.M.packed || e.tile0 + e.ntile != end ||
        e.ntile < 1 || (p.n > 1 && e.ntile < per) || e.list || e.ntile != e.M.NT * e.M.KT ||
        (i == 0 && e.tile0 != 0))
      return hipErrorInvalidValue;
  }
  const int rows = tiles_buf_rows(p);
  if (rows > 256 ||
      (size_t)p.W * rows * 128 + tiles_mma_xs_bytes(p, per) + (p.n > 1 ? 2 : 1) * 4 * LUTN + 16 > 160 * 1024)
    return hipErrorInvalidValue;
  if (mixed) return tiles_mma_launch_mixed(kqt, kqb, p, per, rows, s);
  switch (kqt) {
    case KQ_Q4_K: return tiles_mma_launch<KQ_Q4_K>(p, per, rows, s);
    case KQ_Q5_K: return tiles_mma_launch<KQ_Q5_K>(p, per, rows, s);
    case KQ_Q6_K: return tiles_mma_launch<KQ_Q6_K>(p, per, rows, s);
    case KQ_IQ4_XS: return tiles_mma_launch<KQ_IQ4_XS>(p, per, rows, s);
    default: return hipErrorInvalidValue;
  }
}

template <int KQ, int RS, int NTAB, bool I8, int MT = 1>
static hipError_t flat_launch_t(const FlatPlan& p, hipStream_t s) {
  const size_t smem = (size_t)(p.W + p.nspare) * 2 * RS * 128;
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_fused_flat<KQ, RS, NTAB, I8, MT>),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
  if (e != hipSuccess) return e;
  const int blocks = (p.ntiles + p.W - 1) / p.W;
  hipLaunchKernelGGL((k_fused_flat<KQ, RS, NTAB, I8, MT>), dim3(blocks), dim3(p.W * 64), smem, s, p);
  return hipGetLastError();
}

// one-wave blocks never span two matrices: one table
template <int KQ, int RS>
static hipError_t flat_launch(const FlatPlan& p, hipStream_t s) {
  if (p.mt > 4) return p.W == 1 ? flat_launch_t<KQ, RS, 1, true, 8>(p, s) : flat_launch_t<KQ, RS, 2, true, 8>(p, s);
  if (p.mt > 1) return p.W == 1 ? flat_launch_t<KQ, RS, 1, true, 4>(p, s) : flat_launch_t<KQ, RS, 2, true, 4>(p, s);
  if (p.i8) return p.W == 1 ? flat_launch_t<KQ, RS, 1, true>(p, s) : flat_launch_t<KQ, RS, 2, true>(p, s);
  return p.W == 1 ? flat_launch_t<KQ, RS, 1, false>(p, s) : flat_launch_t<KQ, RS, 2, false>(p, s);
}

// Waves of the flat kernel for (kqt, rs, i8 tokens mt) one CU holds at once by its register use (4 SIMDs x 512
// VGPRs, allocated in 8s; at most 8 waves per SIMD), 0 for an unknown configuration.
template <int KQ, int RS>
static int flat_waves_t(int mt) {
  hipFuncAttributes a{};
  const void* f = mt > 4   ? reinterpret_cast<const void*>(&k_fused_flat<KQ, RS, 2, true, 8>)
                  : mt > 1 ? reinterpret_cast<const void*>(&k_fused_flat<KQ, RS, 2, true, 4>)
                           : reinterpret_cast<const void*>(&k_fused_flat<KQ, RS, 2, true>);
  if (hipFuncGetAttributes(&a, f) != hipSuccess || a.numRegs < 1) return 0;
  return 4 * std::min(8, 512 / ((a.numRegs + 7) / 8 * 8));
}

int flat_waves_per_cu(int kqt, int rs, int mt) {
  if ((rs != 16 && rs != 32) || kqt < KQ_Q4_K || kqt > KQ_IQ4_XS) return 0;
  // per (format, ring, 1 / 4 / 8 tokens): the attribute query once, its answer kept (one device per process)
  static int cache[5][2][3] = {};
  int& c = cache[kqt][rs == 32][mt > 4 ? 2 : (mt > 1 ? 1 : 0)];
  if (c) return c;
  switch (kqt) {
    case KQ_Q4_K: c = rs == 16 ? flat_waves_t<KQ_Q4_K, 16>(mt) : flat_waves_t<KQ_Q4_K, 32>(mt); break;
    case KQ_Q5_K: c = rs == 16 ? flat_waves_t<KQ_Q5_K, 16>(mt) : flat_waves_t<KQ_Q5_K, 32>(mt); break;
    case KQ_Q6_K: c = rs == 16 ? flat_waves_t<KQ_Q6_K, 16>(mt) : flat_waves_t<KQ_Q6_K, 32>(mt); break;
    default: c = rs == 16 ? flat_waves_t<KQ_IQ4_XS, 16>(mt) : flat_waves_t<KQ_IQ4_XS, 32>(mt); break;
  }
  return c;
}

hipError_t launch_fused_flat(const FlatPlan& p, hipStream_t s) {
  if (p.n < 1 || p.n > MAX_GROUP || p.W < 1 || p.W > 16 || p.ntiles < 1) return hipErrorInvalidValue;
  const int kqt = p.e[0].M.kqt, rs = p.e[0].M.ring_rows;
  for (int i = 0; i < p.n; ++i) {
    const FlatEntry& e = p.e[i];
    const DevMat& M = e.M;
    const int end = i + 1 < p.n ? p.e[i + 1].tile0 : p.ntiles;
    if (M.kqt != kqt || M.ring_rows != rs || !M.sched || !M.lut4 || e.tile0 + e.ntile != end || e.ntile < p.W ||
        (!e.list && e.ntile != M.NT * M.KT) || (i == 0 && e.tile0 != 0) ||
        (p.i8 && (!M.luti8 || !e.XQ || !e.DX || !e.SX)))
      return hipErrorInvalidValue;
  }
  if (rs != 16 && rs != 32) return hipErrorInvalidValue;
  if (!flat_tokens_ok(p)) return hipErrorInvalidValue;
  if (rs == 32 && p.W > 8) return hipErrorInvalidValue;  // LDS: 16 KB of tables + W x 8 KB of rings
  // spare rings: 16-row launches only, within the LDS of one CU (160 KB: 16 KB of tables + 32 x 4 KB of rings)
  if (p.nspare < 0 || (p.nspare && (rs != 16 || p.W + p.nspare > 32))) return hipErrorInvalidValue;
  switch (kqt) {
    case KQ_Q4_K: return rs == 16 ? flat_launch<KQ_Q4_K, 16>(p, s) : flat_launch<KQ_Q4_K, 32>(p, s);
    case KQ_Q5_K: return rs == 16 ? flat_launch<KQ_Q5_K, 16>(p, s) : flat_launch<KQ_Q5_K, 32>(p, s);
    case KQ_Q6_K: return rs == 16 ? flat_launch<KQ_Q6_K, 16>(p, s) : flat_launch<KQ_Q6_K, 32>(p, s);
    case KQ_IQ4_XS: return rs == 16 ? flat_launch<KQ_IQ4_XS, 16>(p, s) : flat_launch<KQ_IQ4_XS, 32>(p, s);
    default: return hipErrorInvalidValue;
  }
}

template <int KQ, int MT>
static hipError_t packed_launch(const GroupPlan& p, hipStream_t s) {
  constexpr int TW = kq_symbits(KQ) == 4 ? 2 * TK : TK;
  const size_t smem = ((size_t)((TW / 2) + TW / kq_gw(KQ)) * MT + 3) / 4 * 16 + (size_t)16 * PK_SLOTS * 1024 +
                      (MT == 1 ? (size_t)16 * (TW / 2) * 4 : 0);
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_fused_packed<KQ, MT>),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((k_fused_packed<KQ, MT>), dim3(p.blocks), dim3(1024), smem, s, p);
  return hipGetLastError();
}

template <int KQ>
static hipError_t packed_mt(const GroupPlan& p, hipStream_t s) {
  if (p.mt <= 1) return packed_launch<KQ, 1>(p, s);
  if (p.mt <= 2) return packed_launch<KQ, 2>(p, s);
  if (p.mt <= 4) return packed_launch<KQ, 4>(p, s);
  if (p.mt <= 8) return packed_launch<KQ, 8>(p, s);
  return packed_launch<KQ, 16>(p, s);
}

hipError_t launch_fused_packed(const GroupPlan& p, hipStream_t s) {
  if (p.n < 1 || p.n > MAX_GROUP || p.mt < 1 || p.mt > 16 || p.blocks < 1) return hipErrorInvalidValue;
  const int kqt = p.e[0].M.kqt;
  for (int i = 0; i < p.n; ++i)
    if (p.e[i].M.kqt != kqt || !p.e[i].M.packed || !p.e[i].M.lut4) return hipErrorInvalidValue;
  switch (kqt) {
    case KQ_Q4_K: return packed_mt<KQ_Q4_K>(p, s);
    case KQ_Q5_K: return packed_mt<KQ_Q5_K>(p, s);
    case KQ_Q6_K: return packed_mt<KQ_Q6_K>(p, s);
    case KQ_IQ4_XS: return packed_mt<KQ_IQ4_XS>(p, s);
    default: return hipErrorInvalidValue;
  }
}

template <int KQ, bool I8>
static hipError_t packed_flat_launch_t(const FlatPlan& p, int blocks, size_t smem, hipStream_t s) {
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_fused_packed_flat<KQ, I8>),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((k_fused_packed_flat<KQ, I8>), dim3(blocks), dim3(p.W * 64), smem, s, p);
  return hipGetLastError();
}

template <int KQ>
static hipError_t packed_flat_launch(const FlatPlan& p, int blocks, size_t smem, hipStream_t s) {
  return p.i8 ? packed_flat_launch_t<KQ, true>(p, blocks, smem, s) : packed_flat_launch_t<KQ, false>(p, blocks, smem, s);
}

hipError_t launch_fused_packed_flat(const FlatPlan& p, hipStream_t s) {
  if (p.n < 1 || p.n > MAX_GROUP || p.W < 1 || p.W > 16 || p.ntiles < 1 || p.mt > 1) return hipErrorInvalidValue;
  const int kqt = p.e[0].M.kqt;
  for (int i = 0; i < p.n; ++i) {
    const FlatEntry& e = p.e[i];
    const int end = i + 1 < p.n ? p.e[i + 1].tile0 : p.ntiles;
    if (e.M.kqt != kqt || !e.M.packed || !e.M.lut4 || e.list || e.tile0 + e.ntile != end || e.ntile < p.W ||
        e.ntile != e.M.NT * e.M.KT || (i == 0 && e.tile0 != 0) || (p.i8 && (!e.M.luti8 || !e.XQ || !e.DX || !e.SX)))
      return hipErrorInvalidValue;
  }
  const int blocks = (p.ntiles + p.W - 1) / p.W;
  const size_t smem = (size_t)p.W * PK_SLOTS * 1024 + (size_t)p.W * (kq_symbits(kqt) == 4 ? TK : TK / 2) * 4;
  switch (kqt) {
    case KQ_Q4_K: return packed_flat_launch<KQ_Q4_K>(p, blocks, smem, s);
    case KQ_Q5_K: return packed_flat_launch<KQ_Q5_K>(p, blocks, smem, s);
    case KQ_Q6_K: return packed_flat_launch<KQ_Q6_K>(p, blocks, smem, s);
    case KQ_IQ4_XS: return packed_flat_launch<KQ_IQ4_XS>(p, blocks, smem, s);
    default: return hipErrorInvalidValue;
  }
}

int group_waves_per_block(int ring_rows) { return ring_rows == 16 ? 16 : 8; }

// dynamic LDS of the ring kernel (the 8 KB decode table is static)
static size_t ring_smem(int symbits, int kqt, int MT, int WPB, int RS) {
  const int TW = symbits == 4 ? 2 * TK : TK, GW = kq_gw(kqt);
  return (size_t)(TW / 2) * MT * 4 + (size_t)(TW / GW) * MT * 4 + (size_t)WPB * 2 * RS * 128;
}

template <int KQ, int MT, int RS>
static hipError_t ring_launch(const GroupPlan& p, hipStream_t s) {
  constexpr int WPB = RS == 16 ? 16 : 8;
  const size_t smem = ring_smem(kq_symbits(KQ), KQ, MT, WPB, RS);
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_fused_ring<KQ, MT, WPB, RS>),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((k_fused_ring<KQ, MT, WPB, RS>), dim3(p.blocks), dim3(WPB * 64), smem, s, p);
  return hipGetLastError();
}

template <int KQ, int RS>
static hipError_t ring_mt(const GroupPlan& p, hipStream_t s) {
  if (p.mt <= 1) return ring_launch<KQ, 1, RS>(p, s);
  if (p.mt <= 2) return ring_launch<KQ, 2, RS>(p, s);
  if (p.mt <= 4) return ring_launch<KQ, 4, RS>(p, s);
  if (p.mt <= 8) return ring_launch<KQ, 8, RS>(p, s);
  return ring_launch<KQ, 16, RS>(p, s);
}

template <int KQ>
static hipError_t ring_kq(const GroupPlan& p, hipStream_t s) {
  return p.e[0].M.ring_rows == 16 ? ring_mt<KQ, 16>(p, s) : ring_mt<KQ, 32>(p, s);
}

hipError_t launch_fused_group(const GroupPlan& p, hipStream_t s) {
  if (p.n < 1 || p.n > MAX_GROUP || p.mt < 1 || p.mt > 16 || p.blocks < 1) return hipErrorInvalidValue;
  const int kqt = p.e[0].M.kqt, rs = p.e[0].M.ring_rows;
  for (int i = 0; i < p.n; ++i)
    if (p.e[i].M.kqt != kqt || p.e[i].M.ring_rows != rs || !p.e[i].M.sched || !p.e[i].M.lut4) return hipErrorInvalidValue;
  if (rs != 16 && rs != 32) return hipErrorInvalidValue;
  switch (kqt) {
    case KQ_Q4_K: return ring_kq<KQ_Q4_K>(p, s);
    case KQ_Q5_K: return ring_kq<KQ_Q5_K>(p, s);
    case KQ_Q6_K: return ring_kq<KQ_Q6_K>(p, s);
    case KQ_IQ4_XS: return ring_kq<KQ_IQ4_XS>(p, s);
    default: return hipErrorInvalidValue;
  }
}

template <int PER>
__global__ void k_reduce_group(ReducePlan plan) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= plan.total) return;
  ReduceEntry E = plan.e[0];
#pragma unroll
  for (int k = 1; k < MAX_GROUP; ++k)
    if (k < plan.n && i >= plan.e[k].out0) E = plan.e[k];
  const int o = i - E.out0, j = o / E.N, n = o - j * E.N;
  const uint32_t o0 = (uint32_t)(j * PER * E.N + n), step = (uint32_t)(plan.m * PER * E.N);
  // partials summed in tile-column order (a column's pseudo-tokens in order), the loads of up to 32 / PER columns
  // in flight
  // (the partials are a previous launch's, complete; their slots go back to kNoPartial for the in-launch reductions)
  constexpr int B = 32 / PER;
  float a = 0.f;
  for (int tc = 0; tc < E.KT; tc += B) {
    float v[B][PER];
#pragma unroll
    for (int u = 0; u < B; ++u)
#pragma unroll
      for (int q = 0; q < PER; ++q)
        v[u][q] = tc + u < E.KT ? E.P[o0 + (uint32_t)(tc + u) * step + (uint32_t)(q * E.N)] : 0.f;
#pragma unroll
    for (int u = 0; u < B; ++u)
      if (tc + u < E.KT)
#pragma unroll
        for (int q = 0; q < PER; ++q) {
          a += v[u][q];
          reinterpret_cast<uint32_t*>(E.P)[o0 + (uint32_t)(tc + u) * step + (uint32_t)(q * E.N)] = kNoPartial;
        }
  }
  E.Y[(size_t)j * E.ldy + n] = a;
}

hipError_t launch_reduce_group(const ReducePlan& p, hipStream_t s) {
  if (p.n < 1 || p.n > MAX_GROUP || p.total < 1 || p.per < 1 || p.per > 2) return hipErrorInvalidValue;
  if (p.per == 1) hipLaunchKernelGGL(k_reduce_group<1>, dim3((p.total + 255) / 256), dim3(256), 0, s, p);
  else hipLaunchKernelGGL(k_reduce_group<2>, dim3((p.total + 255) / 256), dim3(256), 0, s, p);
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
  uint32_t pos = half ? (uint32_t)M.mid[(size_t)t * 32 + l] : (uint32_t)GUARD_BITS;
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

// codes of a packed matrix for tile rows [tr0, tr1): one thread per 16-symbol chunk (pk4: two codes per symbol,
// low nibble first; pk8: one), rows relative to tr0
template <int SYMB, bool TILED>
__global__ void __launch_bounds__(256) k_unpack(DevMat M, uint8_t* __restrict__ out, int tr0, int tr1) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;  // chunk within the row range
  const size_t n = (size_t)(tr1 - tr0) * M.KT * 16 * 64;
  if (i >= n) return;
  const int L = (int)(i & 63), g = (int)((i >> 6) & 15);
  const size_t tt = i >> 10;  // tile within the range
  const int tc = (int)(tt % M.KT), trr = (int)(tt / M.KT);
  const uint4 c = reinterpret_cast<const uint4*>(M.words)[((size_t)(tr0 + trr) * M.KT + tc) * 1024 + (size_t)(g * 64 + L)];
  const uint32_t w[4] = {c.x, c.y, c.z, c.w};
  if (TILED) {  // the prefill GEMM's layout (launch_decode_tiled): 16 codes (IQ4_XS: grid bytes) per 16-byte piece
    const int row = trr * TN + L, KC = M.K / 32;
    uint8_t* o = out + ((size_t)(row >> 5) * KC * 64 + (row & 31)) * 16;
    if (SYMB == 4) {  // 32 codes = one chunk: symbols 0..7 -> piece h = 0, 8..15 -> h = 1
      const size_t kc = (size_t)(tc * TK + 16 * g) / 16;
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        uint32_t v[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint32_t sy = (w[2 * hh + (q >> 1)] >> (16 * (q & 1))) & 0xFFFFu;
          if (M.kqt == KQ_IQ4_XS)  // grid bytes kv[q] + 128 from the symbol table (lut4 bytes 2, 3)
            v[q] = (M.lut4[sy & 255u] >> 16) | (M.lut4[sy >> 8] >> 16) << 16;
          else
            v[q] = (sy & 15u) | ((sy >> 4) & 15u) << 8 | ((sy >> 8) & 15u) << 16 | (sy >> 12) << 24;
        }
        *reinterpret_cast<uint4*>(o + (kc * 64 + 32 * hh) * 16) = make_uint4(v[0], v[1], v[2], v[3]);
      }
    } else {  // 16 codes = half a chunk
      const int k = tc * TK + 16 * g;
      *reinterpret_cast<uint4*>(o + ((size_t)(k >> 5) * 64 + 32 * ((k >> 4) & 1)) * 16) = c;
    }
    return;
  }
  uint8_t* o = out + (size_t)(trr * TN + L) * M.K + (size_t)(tc * TK + 16 * g) * (SYMB == 4 ? 2 : 1);
#pragma unroll
  for (int b = 0; b < 16; ++b) {
    const uint32_t sym = (w[b >> 2] >> (8 * (b & 3))) & 255u;
    if (SYMB == 4) {
      o[2 * b] = (uint8_t)(sym & 15u);
      o[2 * b + 1] = (uint8_t)(sym >> 4);
    } else {
      o[b] = (uint8_t)sym;
    }
  }
}

// Codes of a coded matrix with split offsets (the decode bench, rt_test_decode, path 2's codes): one block of 4 waves
// per tile, the tile staged in LDS, 8 chains per lane (wave w: symbols [64 w, 64 w + 64) of row l and row l + 32,
// as k_fused_split). The table entries are rebuilt per block as len | sym << 16 from the reference layout's u16
// LUT. Each wave collects its 64 rows x CW code bytes in LDS (rows 136 B apart: 8-byte aligned, 2-way bank
// conflicts at most) and then stores them row by row, whole 64- or 128-byte segments, so the rows' lines are written
// at once instead of 4 bytes per row and store.
template <int SYMB, bool TILED>
__global__ void __launch_bounds__(256) k_decode_split(DevMat M, uint8_t* __restrict__ out, int tr0, int tr1,
                                                      int stage_rows) {
  constexpr int CW = SYMB == 4 ? 128 : 64;  // code bytes per row and wave
  constexpr int RSTR = 136;                 // LDS row stride of the code rows
  typedef __attribute__((address_space(3))) const uint32_t LdsU32;
  // one static LDS object, the table first, so that the table sits at LDS address 0 (table_addr ORs its base into
  // the index bits), then the 4 waves' code rows
  __shared__ __align__(16) uint32_t lds_static[LUTN + 4 * 64 * RSTR / 4];
  uint32_t* lut4 = lds_static;
  uint8_t* rowbuf = reinterpret_cast<uint8_t*>(lds_static + LUTN);
  extern __shared__ __align__(16) uint32_t tw[];
  const int KT = M.KT, K = M.K;
  const int t = tr0 * KT + (int)blockIdx.x;
  if (t >= tr1 * KT) return;
  const int tc = t % KT, tr = t / KT;
  const int R = min((int)M.rows[t] + 2, stage_rows);
  for (int i = threadIdx.x; i < LUTN; i += 256) {
    const uint32_t e = M.lut[i];
    lut4[i] = (e >> 8) | (e & 255u) << 16;
  }
  const uint4* src = reinterpret_cast<const uint4*>(M.words + M.tbase[t]);
  for (int i = threadIdx.x; i < 8 * R; i += 256) reinterpret_cast<uint4*>(tw)[i] = src[i];
  __syncthreads();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63, l = lane & 31, f = lane >> 5;
  // the lane decodes symbols 64 k .. 64 k + 63 of its lane stream as two chains of 32 from the split offsets
  // 2 k and 2 k + 1, interleaved step by step so that their LDS round trips overlap
  const int k = 4 * f + wave;
  const uint32_t tsel = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const uint32_t*)lut4;
  uint32_t tmask = 0x1FFCu;
  asm volatile("" : "+v"(tmask));
  const uint32_t rlb = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint32_t*)(tw + l);
  uint32_t P[2], slot[2], A[2], B[2], C[2];
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    P[c] = (uint32_t)M.split[((size_t)t * SPLITS + 2 * k + c) * 32 + (uint32_t)l] - GUARD_BITS + 64u;
    slot[c] = __builtin_amdgcn_ubfe(P[c], 5, 8);
    A[c] = *(LdsU32*)(rlb + ((slot[c] - 2u) << 7));
    B[c] = *(LdsU32*)(rlb + ((slot[c] - 1u) << 7));
    C[c] = *(LdsU32*)(rlb + (slot[c] << 7));
  }
  uint8_t* const wbuf = rowbuf + wave * 64 * RSTR;     // the wave's 64 code rows
  uint8_t* rb = wbuf + (f * 32 + l) * RSTR;              // the lane's row
#pragma unroll 4
  for (int p = 0; p < 16; ++p) {
    uint32_t w1[2], e1[2], e2[2];
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      w1[c] = __builtin_amdgcn_alignbit(B[c], A[c], P[c]);
      e1[c] = *(LdsU32*)table_addr(w1[c], tsel, tmask);
    }
#pragma unroll
    for (int c = 0; c < 2; ++c) e2[c] = *(LdsU32*)table_addr(w1[c] >> (e1[c] & 31u), tsel, tmask);
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      P[c] = P[c] + e1[c] + e2[c];
      const uint32_t nslot = __builtin_amdgcn_ubfe(P[c], 5, 8);
      const bool slide = nslot != slot[c];
      A[c] = slide ? B[c] : A[c];
      B[c] = slide ? C[c] : B[c];
      slot[c] = nslot;
      C[c] = *(LdsU32*)(rlb + (nslot << 7));
      const uint32_t s1 = e1[c] >> 16, s2 = e2[c] >> 16;
      if (SYMB == 4)  // codes low nibble first: 4 bytes per pair
        *reinterpret_cast<uint32_t*>(rb + 64 * c + 4 * p) =
            (s1 & 15u) | (s1 >> 4) << 8 | (s2 & 15u) << 16 | (s2 >> 4) << 24;
      else
        *reinterpret_cast<uint16_t*>(rb + 32 * c + 2 * p) = (uint16_t)(s1 | s2 << 8);
    }
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  if (TILED) {  // the prefill GEMM's layout: per 32-row tile and 32-code chunk one 1 KB piece, lane-linear
    const int KC = K / 32, kc0 = (tc * (SYMB == 4 ? 2 * TK : TK) + wave * CW) / 32;
#pragma unroll
    for (int f2 = 0; f2 < 2; ++f2) {
      const size_t rt = (size_t)(tr - tr0) * 2 + f2;
#pragma unroll
      for (int cc = 0; cc < CW / 32; ++cc) {
        const uint8_t* src = wbuf + (f2 * 32 + l) * RSTR + cc * 32 + 16 * f;  // row c = l, half h = f
        const uint2 a = *reinterpret_cast<const uint2*>(src), b = *reinterpret_cast<const uint2*>(src + 8);
        *reinterpret_cast<uint4*>(out + ((rt * KC + kc0 + cc) * 64 + lane) * 16) = make_uint4(a.x, a.y, b.x, b.y);
      }
    }
    return;
  }
  // the wave's 64 rows: 8-byte pieces, CW / 8 lanes per row
  constexpr int LPR = CW / 8, RPI = 64 / LPR;  // lanes per row, rows per store instruction
  const int pr = lane / LPR, pc = lane % LPR;
  uint8_t* orow = out + (size_t)((tr - tr0) * TN) * K + (size_t)tc * (SYMB == 4 ? 2 * TK : TK) + wave * CW + pc * 8;
#pragma unroll
  for (int r0 = 0; r0 < 64; r0 += RPI) {
    const int r = r0 + pr;
    *reinterpret_cast<uint2*>(orow + (size_t)r * K) = *reinterpret_cast<const uint2*>(wbuf + r * RSTR + pc * 8);
  }
}

// Codes in the prefill GEMM's tiled layout (launch_decode_tiled): one block of 4 waves per tile as k_decode_split,
// but each lane runs the two 32-symbol chains of its 64-symbol segment (split starts 2k and 2k + 1) interleaved, and
// stores its codes straight from registers: 16 codes make one lane's piece of the tiled layout, and the 32 lanes of a
// row half write 32 consecutive pieces (512 B) per store. No code rows in LDS: the block holds the table and the tile.
template <int SYMB, bool GRID>
__global__ void __launch_bounds__(256) k_decode_tiled(DevMat M, uint8_t* __restrict__ out, int tr0, int tr1,
                                                      int stage_rows) {
  typedef __attribute__((address_space(3))) const uint32_t LdsU32;
  __shared__ __align__(16) uint32_t lut4[LUTN];  // the only static LDS object: at LDS address 0 (table_addr ORs it in)
  extern __shared__ __align__(16) uint32_t tw[];
  const int KT = M.KT, KC = M.K / 32;
  const int t = tr0 * KT + (int)blockIdx.x;
  if (t >= tr1 * KT) return;
  const int tc = t % KT, tr = t / KT;
  const int R = min((int)M.rows[t] + 2, stage_rows);
  if (GRID) {  // entries len | grid byte of the pair's first code << 16 | second << 24 (decode_table4)
    for (int i = threadIdx.x; i < LUTN / 4; i += 256)
      reinterpret_cast<uint4*>(lut4)[i] = reinterpret_cast<const uint4*>(M.lut4)[i];
  } else {
    for (int i = threadIdx.x; i < LUTN; i += 256) {
      const uint32_t e = M.lut[i];
      lut4[i] = (e >> 8) | (e & 255u) << 16;
    }
  }
  const uint4* src = reinterpret_cast<const uint4*>(M.words + M.tbase[t]);
  for (int i = threadIdx.x; i < 8 * R; i += 256) reinterpret_cast<uint4*>(tw)[i] = src[i];
  __syncthreads();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63, l = lane & 31, f = lane >> 5;
  const int k = 4 * f + wave;  // segment of bit-lane l: row f * 32 + l, symbols 64 wave .. 64 wave + 63
  const uint32_t tsel = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const uint32_t*)lut4;
  uint32_t tmask = 0x1FFCu;
  asm volatile("" : "+v"(tmask));
  const uint32_t rlb = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint32_t*)(tw + l);
  uint32_t P[2], slot[2], A[2], B[2], C[2];
#pragma unroll
  for (int ch = 0; ch < 2; ++ch) {
    P[ch] = (uint32_t)M.split[((size_t)t * SPLITS + 2 * k + ch) * 32 + (uint32_t)l] - GUARD_BITS + 64u;
    slot[ch] = __builtin_amdgcn_ubfe(P[ch], 5, 8);
    A[ch] = *(LdsU32*)(rlb + ((slot[ch] - 2u) << 7));
    B[ch] = *(LdsU32*)(rlb + ((slot[ch] - 1u) << 7));
    C[ch] = *(LdsU32*)(rlb + (slot[ch] << 7));
  }
  // chain ch holds codes [2 (64 wave + 32 ch), + 64) (SYMB 4) or [64 wave + 32 ch, + 32) (SYMB 8) of the row
  const size_t rt = (size_t)(tr - tr0) * 2 + f;
  uint8_t* const obase = out + (rt * KC * 64 + l) * 16;
  const int kc0 = SYMB == 4 ? tc * (2 * TK / 32) + 4 * wave : tc * (TK / 32) + 2 * wave;
  uint32_t acc[2][4];
#pragma unroll
  for (int p = 0; p < 16; ++p) {
#pragma unroll
    for (int ch = 0; ch < 2; ++ch) {
      const uint32_t w1 = __builtin_amdgcn_alignbit(B[ch], A[ch], P[ch]);
      const uint32_t e1 = *(LdsU32*)table_addr(w1, tsel, tmask);
      const uint32_t w2 = w1 >> (e1 & 31u);
      const uint32_t e2 = *(LdsU32*)table_addr(w2, tsel, tmask);
      P[ch] = P[ch] + e1 + e2;
      const uint32_t nslot = __builtin_amdgcn_ubfe(P[ch], 5, 8);
      const bool slide = nslot != slot[ch];
      A[ch] = slide ? B[ch] : A[ch];
      B[ch] = slide ? C[ch] : B[ch];
      slot[ch] = nslot;
      C[ch] = *(LdsU32*)(rlb + (nslot << 7));
      const uint32_t s1 = e1 >> 16, s2 = e2 >> 16;
      if (SYMB == 4) {  // 4 codes per pair, low nibble first (GRID: their grid bytes); a piece every 4 pairs
        acc[ch][p & 3] = GRID ? s1 | s2 << 16 : (s1 & 15u) | (s1 >> 4) << 8 | (s2 & 15u) << 16 | (s2 >> 4) << 24;
        if ((p & 3) == 3) {
          const int q = p >> 2;  // piece q of the chain's 64 codes: chunk kc0 + 2 ch + q / 2, half q % 2
          *reinterpret_cast<uint4*>(obase + ((size_t)(kc0 + 2 * ch + (q >> 1)) * 64 + 32 * (q & 1)) * 16) =
              make_uint4(acc[ch][0], acc[ch][1], acc[ch][2], acc[ch][3]);
        }
      } else {  // 2 codes per pair; a piece every 8 pairs
        const uint32_t v = s1 | s2 << 8;
        if (p & 1) acc[ch][(p >> 1) & 3] |= v << 16;
        else acc[ch][(p >> 1) & 3] = v;
        if ((p & 7) == 7)
          *reinterpret_cast<uint4*>(obase + ((size_t)(kc0 + ch) * 64 + 32 * (p >> 3)) * 16) =
              make_uint4(acc[ch][0], acc[ch][1], acc[ch][2], acc[ch][3]);
      }
    }
  }
}

template <bool TILED>
static hipError_t decode_fast(const DevMat& M, uint8_t* out, int tr0, int tr1, hipStream_t s) {
  if (M.packed) {
    const size_t n = (size_t)(tr1 - tr0) * M.KT * 16 * 64;
    if (!n) return hipSuccess;
    if (M.symbits == 4) hipLaunchKernelGGL((k_unpack<4, TILED>), dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, M, out, tr0, tr1);
    else hipLaunchKernelGGL((k_unpack<8, TILED>), dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, M, out, tr0, tr1);
    return hipGetLastError();
  }
  if (tr0 >= tr1) return hipSuccess;
  const int rows = M.max_rows + 2;
  const size_t sm = (size_t)rows * 128;
  const void* f = M.symbits == 4 ? reinterpret_cast<const void*>(&k_decode_split<4, TILED>)
                                 : reinterpret_cast<const void*>(&k_decode_split<8, TILED>);
  hipError_t e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)sm);
  if (e != hipSuccess) return e;
  const dim3 grid((unsigned)((tr1 - tr0) * M.KT));
  if (M.symbits == 4) hipLaunchKernelGGL((k_decode_split<4, TILED>), grid, dim3(256), sm, s, M, out, tr0, tr1, rows);
  else hipLaunchKernelGGL((k_decode_split<8, TILED>), grid, dim3(256), sm, s, M, out, tr0, tr1, rows);
  return hipGetLastError();
}

bool decode_tiled_ok(const DevMat& M) {
  return M.K % 32 == 0 && (M.kqt != KQ_IQ4_XS || M.lut4) &&
         (M.packed || (M.split && M.rows && M.lut && M.max_rows + 2 <= 256));
}

hipError_t launch_decode_tiled(const DevMat& M, uint8_t* out, int tr0, int tr1, hipStream_t s) {
  if (!decode_tiled_ok(M)) return hipErrorNotSupported;
  if (M.packed || tr0 >= tr1) return decode_fast<true>(M, out, tr0, tr1, s);
  const int rows = M.max_rows + 2;
  const size_t sm = (size_t)rows * 128;
  const bool grid_bytes = M.kqt == KQ_IQ4_XS;
  const void* f = M.symbits != 4 ? reinterpret_cast<const void*>(&k_decode_tiled<8, false>)
                  : grid_bytes   ? reinterpret_cast<const void*>(&k_decode_tiled<4, true>)
                                 : reinterpret_cast<const void*>(&k_decode_tiled<4, false>);
  hipError_t e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)sm);
  if (e != hipSuccess) return e;
  const dim3 grid((unsigned)((tr1 - tr0) * M.KT));
  if (M.symbits != 4) hipLaunchKernelGGL((k_decode_tiled<8, false>), grid, dim3(256), sm, s, M, out, tr0, tr1, rows);
  else if (grid_bytes) hipLaunchKernelGGL((k_decode_tiled<4, true>), grid, dim3(256), sm, s, M, out, tr0, tr1, rows);
  else hipLaunchKernelGGL((k_decode_tiled<4, false>), grid, dim3(256), sm, s, M, out, tr0, tr1, rows);
  return hipGetLastError();
}

hipError_t launch_decode(const DevMat& M, uint8_t* out, int tr0, int tr1, hipStream_t s) {
  if (M.packed || (M.split && M.rows && M.lut && M.max_rows + 2 <= 256))  // the unpack / 8-chain kernels
    return decode_fast<false>(M, out, tr0, tr1, s);
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
    side_load<KQ>(M.side + side_record(n, b, M.KT, M.symbits == 4 ? 2 : 1) * SB, sw);
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

// ── prefill GEMM on the matrix cores (path 2, m > 16): decoded codes x fp16 hi + lo activations ──────────
// Y[t][n] = sum over sub-blocks of s_n (x_t . f(q_n)) - o_n (sum x_t), as k_gemm_codes, with both sums on
// v_mfma_f32_32x32x8f16. Block = 4 waves = 64 rows x 64 tokens, wave = 32 x 32. In a block of 32 lanes the MFMA
// takes A[i][k] (token i, 8 weights) from lane i + 32 (k / 4) and B[k][j] (row j) from lane j + 32 (k / 4), and
// leaves D[i][j] in lane j + 32 h, register r, i = 8 (r / 4) + 4 h + r % 4 (checked on the GPU): every lane holds
// one row (its scales) and 16 tokens. Products are exact (f(q) and the hi / lo halves of x are fp16, fp32 sums);
// the activation sums come from a second MFMA with B = 1.
template <int KQ>
__global__ void __launch_bounds__(256) k_gemm_codes_mfma(DevMat M, const uint8_t* __restrict__ codes, int row0,
                                                         int nrows, const uint16_t* __restrict__ X16, int m,
                                                         float* __restrict__ Y, int ldy) {
  constexpr int GW = kq_gw(KQ), SB = kq_sbytes(KQ);
  constexpr bool MINS = KQ == KQ_Q4_K || KQ == KQ_Q5_K;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, c = lane & 31, h = lane >> 5;
  const int nl = blockIdx.x * 64 + (wave & 1) * 32 + c;   // the lane's row (relative to row0)
  const int t0 = blockIdx.y * 64 + (wave >> 1) * 32;       // the wave's first token
  const int K = M.K;
  const int nls = min(nl, nrows - 1);                      // rows past the end compute row nrows - 1, unstored
  const int ta = min(t0 + c, m - 1);                       // the lane's token for A (clamped likewise)
  const uint8_t* cr = codes + (size_t)nls * K + 4 * h;
  const uint16_t* xh = X16 + (size_t)(2 * ta) * K + 4 * h;
  const uint16_t* xl = X16 + (size_t)(2 * ta + 1) * K + 4 * h;
  const h4v ones = {(_Float16)1.f, (_Float16)1.f, (_Float16)1.f, (_Float16)1.f};
  f16x16 tot = {};
  for (int b = 0; b < K / 256; ++b) {
    uint32_t sw[5];
    side_load<KQ>(M.side + side_record(row0 + nls, b, M.KT, M.symbits == 4 ? 2 : 1) * SB, sw);
    for (int jj = 0; jj < 256 / GW; ++jj) {
      float sc, o;
      side_scale<KQ>(sw, jj, sc, o);
      f16x16 d1 = {}, d2 = {};
#pragma unroll
      for (int ks = 0; ks < GW / 8; ++ks) {
        const int k = b * 256 + jj * GW + ks * 8;
        const uint32_t q = *reinterpret_cast<const uint32_t*>(cr + k);
        float w0 = (float)(q & 255u), w1 = (float)((q >> 8) & 255u);  // v_cvt_f32_ubyte0..3
        float w2 = (float)((q >> 16) & 255u), w3 = (float)(q >> 24);
        if (KQ == KQ_Q6_K) {
          w0 -= 32.f;
          w1 -= 32.f;
          w2 -= 32.f;
          w3 -= 32.f;
        } else if (KQ == KQ_IQ4_XS) {
          w0 = (float)IQ4_GRID[q & 15u];
          w1 = (float)IQ4_GRID[(q >> 8) & 15u];
          w2 = (float)IQ4_GRID[(q >> 16) & 15u];
          w3 = (float)IQ4_GRID[(q >> 24) & 15u];
        }
        const h4v wv = {(_Float16)w0, (_Float16)w1, (_Float16)w2, (_Float16)w3};
        const h4v ah = __builtin_bit_cast(h4v, *reinterpret_cast<const uint2*>(xh + k));
        const h4v al = __builtin_bit_cast(h4v, *reinterpret_cast<const uint2*>(xl + k));
        d1 = __builtin_amdgcn_mfma_f32_32x32x8f16(ah, wv, d1, 0, 0, 0);
        d1 = __builtin_amdgcn_mfma_f32_32x32x8f16(al, wv, d1, 0, 0, 0);
        if (MINS) {
          d2 = __builtin_amdgcn_mfma_f32_32x32x8f16(ah, ones, d2, 0, 0, 0);
          d2 = __builtin_amdgcn_mfma_f32_32x32x8f16(al, ones, d2, 0, 0, 0);
        }
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) tot[r] = MINS ? tot[r] + (sc * d1[r] - o * d2[r]) : tot[r] + sc * d1[r];
    }
  }
  if (nl >= nrows) return;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int t = t0 + 8 * (r / 4) + 4 * h + (r % 4);
    if (t < m) Y[(size_t)t * ldy + row0 + nl] = tot[r];
  }
}

hipError_t launch_gemm_codes_mfma(const DevMat& M, const uint8_t* codes, int row0, int nrows, const void* X16, int m,
                                  float* Y, int ldy, hipStream_t s) {
  if (nrows < 1 || m < 1) return hipErrorInvalidValue;
  const dim3 grid((nrows + 63) / 64, (m + 63) / 64);
  const uint16_t* x = static_cast<const uint16_t*>(X16);
  switch (M.kqt) {
    case KQ_Q4_K: hipLaunchKernelGGL(k_gemm_codes_mfma<KQ_Q4_K>, grid, dim3(256), 0, s, M, codes, row0, nrows, x, m, Y, ldy); break;
    case KQ_Q5_K: hipLaunchKernelGGL(k_gemm_codes_mfma<KQ_Q5_K>, grid, dim3(256), 0, s, M, codes, row0, nrows, x, m, Y, ldy); break;
    case KQ_Q6_K: hipLaunchKernelGGL(k_gemm_codes_mfma<KQ_Q6_K>, grid, dim3(256), 0, s, M, codes, row0, nrows, x, m, Y, ldy); break;
    case KQ_IQ4_XS: hipLaunchKernelGGL(k_gemm_codes_mfma<KQ_IQ4_XS>, grid, dim3(256), 0, s, M, codes, row0, nrows, x, m, Y, ldy); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// ── prefill GEMM on the matrix cores, Q4_K / Q5_K (path 2 and m > 8, the default for these formats) ─────────
// Y[t][n] = sum over super-blocks of d_n (x_t . w'_n) - dmin_n (Sx_t . m_n), where w'_k = sc_j q_k is the code scaled
// by its sub-block's 6-bit scale (at most 63 x 31 = 1953) and Sx_t,j the sum of x_t over sub-block j, m_n,j the
// sub-block's 6-bit min. Both dot products run on v_mfma_f32_32x32x16_f16 with x split into fp16 hi + lo (two
// products per weight, fp32 accumulation), the mins term as one K = 16 product per super-block (8 sub-blocks,
// zero-padded) with Sx split likewise; d and dmin applied once per super-block.
// Weights enter the products as w'/16, exact in fp16: a byte permute against 0x54 bytes makes fp16(64 + q/16) of each
// code, and one fma with sc and -64 sc leaves sc q / 16 (every intermediate exact); the 16 goes into d.
// Operand layout (32x32x16): lane l holds A[i = l % 32][k = 8 (l / 32) + 0..7] (token i) and B[k = 8 (l / 32) + 0..7]
// [j = l % 32] (weight row j), and receives D[i = 8 (r / 4) + 4 (l / 32) + r % 4][j = l % 32] in register r: a lane owns
// one weight row (one set of scales) per row tile and 16 tokens of the token tile.
// Block = GEMM_WAVES waves over 64 weight rows (two row tiles) x 32 tokens; the waves split K by super-block (wave w
// takes super-blocks w, w + GEMM_WAVES, ...) and their partial tiles are summed through LDS in wave order, so the
// result does not depend on timing. A skinny prefill (m = 128, N = 4096) gives 256 blocks.
constexpr int GEMM_WAVES = 8;
typedef _Float16 h8v __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// codes q0..q3 (bytes of qw) -> sc q / 16 as 4 fp16 in two words (nsc = -64 sc)
__device__ __forceinline__ uint2 scaled_codes16(uint32_t qw, h2v sc, h2v nsc) {
  const h2v a = __builtin_bit_cast(h2v, __builtin_amdgcn_perm(0x54545454u, qw, 0x04010400u));
  const h2v b = __builtin_bit_cast(h2v, __builtin_amdgcn_perm(0x54545454u, qw, 0x04030402u));
  return make_uint2(__builtin_bit_cast(uint32_t, __builtin_elementwise_fma(a, sc, nsc)),
                    __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(b, sc, nsc)));
}

// a row's Q4_K / Q5_K super-block record, compacted: the 8 scales and the 8 mins as bytes, d x 16 and dmin
struct KSide {
  uint32_t sc_lo, sc_hi, m_lo, m_hi;
  float d16, dmin;
};
__device__ __forceinline__ KSide kside(const uint32_t* w) {
  KSide k;
  k.sc_lo = w[1] & 0x3F3F3F3Fu;
  k.sc_hi = (w[3] & 0x0F0F0F0Fu) | ((w[1] >> 2) & 0x30303030u);
  k.m_lo = w[2] & 0x3F3F3F3Fu;
  k.m_hi = ((w[3] >> 4) & 0x0F0F0F0Fu) | ((w[2] >> 2) & 0x30303030u);
  k.d16 = 16.f * h2f(w[0]);
  k.dmin = h2f(w[0] >> 16);
  return k;
}
// sub-block j's scale as an fp16 pair
__device__ __forceinline__ h2v kside_sc(const KSide& k, int j) {
  const _Float16 v = (_Float16)(float)((((j < 4) ? k.sc_lo : k.sc_hi) >> (8 * (j & 3))) & 255u);
  return h2v{v, v};
}
// the 8 mins as the B operand of the mins product (k 0..7; lanes h = 1 pass zeros)
__device__ __forceinline__ h8v kside_mins(const KSide& k) {
  h8v v;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[i] = (_Float16)(float)((k.m_lo >> (8 * i)) & 255u);
    v[4 + i] = (_Float16)(float)((k.m_hi >> (8 * i)) & 255u);
  }
  return v;
}

// Layouts (all lane-linear: one wave's load of a piece is one contiguous 1 KB read):
//   codes CT: per 32-row tile rt and 32-code chunk kc (the weights of one sub-block) a 1 KB piece at
//     (rt KC + kc) 1024, lane (h, c) = 32 h + c holding row c's codes 16 h .. 16 h + 15 of the chunk;
//   x XT: per 32-token tile tt, chunk kc, half (hi / lo) and step s a 1 KB piece at (((tt KC + kc) 2 + half) 2 + s)
//     1024, lane (h, c) holding x[token c][32 kc + 16 h + 8 s + 0..7] as fp16;
//   SXT: per token tile tt, super-block sb and half a 512-byte piece, lane c (< 32) holding Sx[token c][8 sb + 0..7].
// Step s of chunk kc gives lane (h, c) the weights 32 kc + 16 h + 8 s + 0..7 in both operands: the products of the
// 32 weights of the chunk are all taken once, in a different order than k, which a dot product does not see.
template <int KQ>
__global__ void __launch_bounds__(64 * GEMM_WAVES) k_gemm_prefill(DevMat M, const uint8_t* __restrict__ CT, int row0,
                                                               const uint16_t* __restrict__ XT,
                                                               const uint16_t* __restrict__ SXT, int m,
                                                               float* __restrict__ Y, int ldy) {
  static_assert(KQ == KQ_Q4_K || KQ == KQ_Q5_K, "scaled weights are exact in fp16 for Q4_K / Q5_K only");
  constexpr int SB = kq_sbytes(KQ), NSB = kq_symbits(KQ) == 4 ? 2 : 1;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63, c = lane & 31, h = lane >> 5;
  const int rp = blockIdx.x, tt = blockIdx.y;            // pair of 32-row tiles of the chunk, 32-token tile
  const int K = M.K, KC = K / 32, NB = K / 256;
  const int nA = rp * 64 + c, nB = nA + 32;              // the lane's weight rows within the chunk
  // buffer resources over the block's codes (its two row tiles) and x (its token tile): the lane's byte offset is
  // the only per-lane address, the chunk offset a scalar
  const __amdgpu_buffer_rsrc_t rc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t*>(CT + (size_t)rp * 2 * KC * 1024), (short)0, 2 * KC * 1024, kBufferRsrcWord3);
  const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(XT + (size_t)tt * KC * 2048), (short)0, KC * 4096, kBufferRsrcWord3);
  const uint16_t* sxw = SXT + (size_t)tt * NB * 512 + c * 8;
  const uint32_t vo = (uint32_t)lane * 16;
  // operands in flight: codes and x three chunks ahead on 4-slot rings (one depth for both: the load counter
  // completes in issue order); 8 chunks per super-block keep the rings aligned
  auto load_q = [&](int kc, u32x4& qa, u32x4& qb) {
    qa = __builtin_amdgcn_raw_buffer_load_b128(rc, vo, kc * 1024, 0);
    qb = __builtin_amdgcn_raw_buffer_load_b128(rc, vo, (KC + kc) * 1024, 0);
  };
  auto load_x = [&](int kc, u32x4* x) {
#pragma unroll
    for (int i = 0; i < 4; ++i) x[i] = __builtin_amdgcn_raw_buffer_load_b128(rx, vo + i * 1024, kc * 4096, 0);
  };
  f16x16 totA = {}, totB = {};
  uint32_t swa[5] = {}, swb[5] = {};
  u32x4 qa[4] = {}, qb[4] = {}, xr[4][4] = {};
  if (wave < NB) {
    side_load<KQ>(M.side + side_record(row0 + nA, wave, M.KT, NSB) * SB, swa);
    side_load<KQ>(M.side + side_record(row0 + nB, wave, M.KT, NSB) * SB, swb);
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      load_q(wave * 8 + i, qa[i], qb[i]);
      load_x(wave * 8 + i, xr[i]);
    }
  }
  for (int sb = wave; sb < NB; sb += GEMM_WAVES) {
    const KSide ka = kside(swa), kb = kside(swb);
    const int nsb = sb + GEMM_WAVES;
    if (nsb < NB) {
      side_load<KQ>(M.side + side_record(row0 + nA, nsb, M.KT, NSB) * SB, swa);
      side_load<KQ>(M.side + side_record(row0 + nB, nsb, M.KT, NSB) * SB, swb);
    }
    uint4 sxh = {}, sxl = {};  // Sx of this super-block, loaded at chunk 5
    f16x16 dA = {}, dB = {};
#pragma unroll
    for (int j = 0; j < 8; ++j) {  // the super-block's 8 chunks (sub-blocks)
      if (j < 5 || nsb < NB) {
        const int kn = j < 5 ? sb * 8 + j + 3 : nsb * 8 + j - 5;
        load_q(kn, qa[(j + 3) & 3], qb[(j + 3) & 3]);
        load_x(kn, xr[(j + 3) & 3]);
      }
      if (j == 5 && h == 0) {  // lanes h = 0 hold the mins product's k 0..7; k 8..15 stay zero
        sxh = *reinterpret_cast<const uint4*>(sxw + (size_t)sb * 512);
        sxl = *reinterpret_cast<const uint4*>(sxw + (size_t)sb * 512 + 256);
      }
      __builtin_amdgcn_sched_barrier(0);  // keep the loads issued here, ahead of this chunk's products
      const u32x4 ca = qa[j & 3], cb = qb[j & 3];
      const u32x4* xc = xr[j & 3];
      const h2v sca = kside_sc(ka, j), scb = kside_sc(kb, j);
      const h2v n64 = {(_Float16)-64.f, (_Float16)-64.f};
      const h2v nsa = sca * n64, nsb2 = scb * n64;
#pragma unroll
      for (int st = 0; st < 2; ++st) {
        const uint2 a0 = scaled_codes16(ca[2 * st], sca, nsa), a1 = scaled_codes16(ca[2 * st + 1], sca, nsa);
        const uint2 b0 = scaled_codes16(cb[2 * st], scb, nsb2), b1 = scaled_codes16(cb[2 * st + 1], scb, nsb2);
        const h8v wa = __builtin_bit_cast(h8v, make_uint4(a0.x, a0.y, a1.x, a1.y));
        const h8v wb = __builtin_bit_cast(h8v, make_uint4(b0.x, b0.y, b1.x, b1.y));
        const h8v xh = __builtin_bit_cast(h8v, xc[st]), xl = __builtin_bit_cast(h8v, xc[2 + st]);
        dA = __builtin_amdgcn_mfma_f32_32x32x16_f16(xh, wa, dA, 0, 0, 0);
        dB = __builtin_amdgcn_mfma_f32_32x32x16_f16(xh, wb, dB, 0, 0, 0);
        dA = __builtin_amdgcn_mfma_f32_32x32x16_f16(xl, wa, dA, 0, 0, 0);
        dB = __builtin_amdgcn_mfma_f32_32x32x16_f16(xl, wb, dB, 0, 0, 0);
      }
    }
    // mins: A2 = the tokens' Sx over the super-block's 8 sub-blocks, B2 = the row's 8 mins
    h8v ma = {}, mb = {};
    if (h == 0) {
      ma = kside_mins(ka);
      mb = kside_mins(kb);
    }
    f16x16 mA = {}, mB = {};
    mA = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(h8v, sxh), ma, mA, 0, 0, 0);
    mB = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(h8v, sxh), mb, mB, 0, 0, 0);
    mA = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(h8v, sxl), ma, mA, 0, 0, 0);
    mB = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(h8v, sxl), mb, mB, 0, 0, 0);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      totA[r] = fmaf(ka.d16, dA[r], fmaf(-ka.dmin, mA[r], totA[r]));
      totB[r] = fmaf(kb.d16, dB[r], fmaf(-kb.dmin, mB[r], totB[r]));
    }
  }
  // partial tiles -> LDS as part[wave][row tile][r][lane] (lane-contiguous, no bank conflicts), then each thread
  // sums its outputs over the waves in order; consecutive threads take consecutive lanes = consecutive weight rows
  __shared__ float part[GEMM_WAVES][2][16][64];
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    part[wave][0][r][lane] = totA[r];
    part[wave][1][r][lane] = totB[r];
  }
  __syncthreads();
  for (int e = threadIdx.x; e < 2 * 16 * 64; e += 64 * GEMM_WAVES) {
    const int half = e >> 10, r = (e >> 6) & 15, l = e & 63;
    float acc = 0.f;
#pragma unroll
    for (int w = 0; w < GEMM_WAVES; ++w) acc += part[w][half][r][l];
    const int t = tt * 32 + 8 * (r / 4) + 4 * (l >> 5) + (r % 4);
    if (t < m) Y[(size_t)t * ldy + row0 + rp * 64 + 32 * half + (l & 31)] = acc;
  }
}

// ── prefill GEMM on the matrix cores, Q6_K / IQ4_XS: unscaled grid weights, folded per sub-block ─────────────
// Y[t][n] = sum over sub-blocks j of d_n s_n,j (x_t . f(q_n)) with f(q) = q - 32 (Q6_K) or kv[q] (IQ4_XS): integers of
// at most 8 bits, exact in fp16, where the scaled s f(q) (up to 128 x 32 or 32 x 127) is not. Each sub-block's
// products go to a fresh accumulator tile (x split into fp16 hi + lo, as k_gemm_prefill), folded into the fp32 total
// with d s_j (exact in fp32) once the sub-block is in. No offsets: neither format has mins.
// The block, the waves' split of K, the rings and the wave-order LDS sum are those of k_gemm_prefill. A step's K = 16
// must lie in one sub-block:
//   IQ4_XS (32-weight sub-blocks) takes k_gemm_prefill's steps (a chunk = a sub-block) over the grid bytes kv[q] + 128
//   of the tiled codes; weights fp16(1024 + g) from a byte permute against 0x64, minus 1152.
//   Q6_K (16-weight sub-blocks) takes weights 16 s + 8 h + 0..7 of the chunk in step s for lane (h, c), so that step s
//   is sub-block 2 kc + s: 8 bytes of the codes piece at lane slot 32 s + c, byte 8 h, and the x piece of step h at
//   lane slot 32 s + c (the products of a chunk are still each taken once); weights fp16(1024 + q) minus 1056.
template <int KQ>
__global__ void __launch_bounds__(64 * GEMM_WAVES) k_gemm_prefill_sub(DevMat M, const uint8_t* __restrict__ CT, int row0,
                                                                   const uint16_t* __restrict__ XT, int m,
                                                                   float* __restrict__ Y, int ldy) {
  static_assert(KQ == KQ_Q6_K || KQ == KQ_IQ4_XS, "per-sub-block folding: Q6_K and IQ4_XS");
  constexpr bool Q6 = KQ == KQ_Q6_K;
  constexpr int SB = kq_sbytes(KQ), NSB = kq_symbits(KQ) == 4 ? 2 : 1;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63, c = lane & 31, h = lane >> 5;
  const int rp = blockIdx.x, tt = blockIdx.y;
  const int K = M.K, KC = K / 32, NB = K / 256;
  const int nA = rp * 64 + c, nB = nA + 32;
  const __amdgpu_buffer_rsrc_t rc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t*>(CT + (size_t)rp * 2 * KC * 1024), (short)0, 2 * KC * 1024, kBufferRsrcWord3);
  const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(XT + (size_t)tt * KC * 2048), (short)0, KC * 4096, kBufferRsrcWord3);
  // the lane's byte offsets of step s's operands in a chunk's codes piece and in its x pieces (hi, then lo 2 KB on)
  uint32_t vq[2], vx[2];
#pragma unroll
  for (int st = 0; st < 2; ++st) {
    vq[st] = Q6 ? (uint32_t)(32 * st + c) * 16 + 8 * h : (uint32_t)lane * 16;
    vx[st] = Q6 ? (uint32_t)h * 1024 + (uint32_t)(32 * st + c) * 16 : (uint32_t)st * 1024 + (uint32_t)lane * 16;
  }
  // a chunk's codes as 4 words per row tile, words 2 s and 2 s + 1 = the 8 weights of step s
  auto load_q = [&](int kc, u32x4& qa, u32x4& qb) {
    if (Q6) {
#pragma unroll
      for (int st = 0; st < 2; ++st) {
        const auto a = __builtin_amdgcn_raw_buffer_load_b64(rc, vq[st], kc * 1024, 0);
        const auto b = __builtin_amdgcn_raw_buffer_load_b64(rc, vq[st], (KC + kc) * 1024, 0);
        qa[2 * st] = a[0];
        qa[2 * st + 1] = a[1];
        qb[2 * st] = b[0];
        qb[2 * st + 1] = b[1];
      }
    } else {
      qa = __builtin_amdgcn_raw_buffer_load_b128(rc, vq[0], kc * 1024, 0);
      qb = __builtin_amdgcn_raw_buffer_load_b128(rc, vq[0], (KC + kc) * 1024, 0);
    }
  };
  auto load_x = [&](int kc, u32x4* x) {  // x[2 half + s]
#pragma unroll
    for (int i = 0; i < 4; ++i) x[i] = __builtin_amdgcn_raw_buffer_load_b128(rx, vx[i & 1] + (i >> 1) * 2048, kc * 4096, 0);
  };
  // 4 weights (bytes of qw) -> fp16 f(q) in two words
  const h2v bias = Q6 ? h2v{(_Float16)-1056.f, (_Float16)-1056.f} : h2v{(_Float16)-1152.f, (_Float16)-1152.f};
  auto grid16 = [&](uint32_t qw) -> uint2 {
    const h2v a = __builtin_bit_cast(h2v, __builtin_amdgcn_perm(0x64646464u, qw, 0x04010400u));
    const h2v b = __builtin_bit_cast(h2v, __builtin_amdgcn_perm(0x64646464u, qw, 0x04030402u));
    return make_uint2(__builtin_bit_cast(uint32_t, a + bias), __builtin_bit_cast(uint32_t, b + bias));
  };
  // d s_j of sub-block j of a super-block record (words as side_load)
  auto sub_scale = [&](const uint32_t* w, int j) -> float {
    if (Q6) return h2f(w[4]) * (float)(int)(int8_t)(uint8_t)(w[j >> 2] >> (8 * (j & 3)));
    const uint32_t ls = ((w[1] >> (4 * j)) & 15u) | ((w[0] >> (16 + 2 * j)) & 3u) << 4;
    return h2f(w[0]) * (float)((int)ls - 32);
  };
  f16x16 totA = {}, totB = {};
  uint32_t swa[5] = {}, swb[5] = {};
  u32x4 qa[4] = {}, qb[4] = {}, xr[4][4] = {};
  if (wave < NB) {
    side_load<KQ>(M.side + side_record(row0 + nA, wave, M.KT, NSB) * SB, swa);
    side_load<KQ>(M.side + side_record(row0 + nB, wave, M.KT, NSB) * SB, swb);
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      load_q(wave * 8 + i, qa[i], qb[i]);
      load_x(wave * 8 + i, xr[i]);
    }
  }
  for (int sb = wave; sb < NB; sb += GEMM_WAVES) {
    uint32_t wa[5], wb[5];
#pragma unroll
    for (int i = 0; i < 5; ++i) {
      wa[i] = swa[i];
      wb[i] = swb[i];
    }
    const int nsb = sb + GEMM_WAVES;
    if (nsb < NB) {
      side_load<KQ>(M.side + side_record(row0 + nA, nsb, M.KT, NSB) * SB, swa);
      side_load<KQ>(M.side + side_record(row0 + nB, nsb, M.KT, NSB) * SB, swb);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {  // the super-block's 8 chunks
      if (j < 5 || nsb < NB) {
        const int kn = j < 5 ? sb * 8 + j + 3 : nsb * 8 + j - 5;
        load_q(kn, qa[(j + 3) & 3], qb[(j + 3) & 3]);
        load_x(kn, xr[(j + 3) & 3]);
      }
      __builtin_amdgcn_sched_barrier(0);  // keep the loads issued here, ahead of this chunk's products
      const u32x4 ca = qa[j & 3], cb = qb[j & 3];
      const u32x4* xc = xr[j & 3];
      f16x16 dA = {}, dB = {};
#pragma unroll
      for (int st = 0; st < 2; ++st) {
        if (Q6 && st == 1) {
          dA = f16x16{};
          dB = f16x16{};
        }
        const uint2 a0 = grid16(ca[2 * st]), a1 = grid16(ca[2 * st + 1]);
        const uint2 b0 = grid16(cb[2 * st]), b1 = grid16(cb[2 * st + 1]);
        const h8v wva = __builtin_bit_cast(h8v, make_uint4(a0.x, a0.y, a1.x, a1.y));
        const h8v wvb = __builtin_bit_cast(h8v, make_uint4(b0.x, b0.y, b1.x, b1.y));
        const h8v xh = __builtin_bit_cast(h8v, xc[st]), xl = __builtin_bit_cast(h8v, xc[2 + st]);
        dA = __builtin_amdgcn_mfma_f32_32x32x16_f16(xh, wva, dA, 0, 0, 0);
        dB = __builtin_amdgcn_mfma_f32_32x32x16_f16(xh, wvb, dB, 0, 0, 0);
        dA = __builtin_amdgcn_mfma_f32_32x32x16_f16(xl, wva, dA, 0, 0, 0);
        dB = __builtin_amdgcn_mfma_f32_32x32x16_f16(xl, wvb, dB, 0, 0, 0);
        if (Q6 || st == 1) {  // the sub-block is in: fold it
          const int js = Q6 ? 2 * j + st : j;
          const float sa = sub_scale(wa, js), sbb = sub_scale(wb, js);
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            totA[r] = fmaf(sa, dA[r], totA[r]);
            totB[r] = fmaf(sbb, dB[r], totB[r]);
          }
          // keep the fold here: sunk below the chunk loop's branches it would hold every chunk's tiles live (spills)
          asm volatile("" : "+v"(totA), "+v"(totB));
        }
      }
    }
  }
  __shared__ float part[GEMM_WAVES][2][16][64];
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    part[wave][0][r][lane] = totA[r];
    part[wave][1][r][lane] = totB[r];
  }
  __syncthreads();
  for (int e = threadIdx.x; e < 2 * 16 * 64; e += 64 * GEMM_WAVES) {
    const int half = e >> 10, r = (e >> 6) & 15, l = e & 63;
    float acc = 0.f;
#pragma unroll
    for (int w = 0; w < GEMM_WAVES; ++w) acc += part[w][half][r][l];
    const int t = tt * 32 + 8 * (r / 4) + 4 * (l >> 5) + (r % 4);
    if (t < m) Y[(size_t)t * ldy + row0 + rp * 64 + 32 * half + (l & 31)] = acc;
  }
}

// x of the prefill GEMM: fp32 X [m][K] -> XT (fp16 hi = fp16(x), lo = fp16(x - hi)) and SXT (per sub-block of 32
// weights s = ((a0 + a1) + (a2 + a3)), a_q the in-order fp32 sum of its q-th 8 values, as fp16 hi / lo), tokens
// padded with zeros to a multiple of 64. Thread = (chunk, q, token c of the tile): the 32 threads of one q write one
// lane-linear 512-byte run of a piece; the chunk's four a_q meet in LDS.
__global__ void __launch_bounds__(256) k_prefill_x(const float* __restrict__ X, uint16_t* __restrict__ XT,
                                                   uint16_t* __restrict__ SXT, int m, int K) {
  const int KC = K / 32, NB = K / 256;
  const int i = (int)blockIdx.x * 256 + threadIdx.x;     // the grid covers the padded tokens exactly
  const int c = i & 31, q = (i >> 5) & 3, ci = i >> 7;
  const int tt = ci / KC, kc = ci - tt * KC, t = tt * 32 + c, hh = q >> 1, st = q & 1;
  float v[8];
  if (t < m) {
    const float* x = X + (size_t)t * K + 32 * kc + 8 * q;
    const float4 a = *reinterpret_cast<const float4*>(x), b = *reinterpret_cast<const float4*>(x + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = 0.f;
  }
  uint32_t hw[4], lw[4];
  float sum = 0.f;
#pragma unroll
  for (int e = 0; e < 8; e += 2) {
    const _Float16 h0 = (_Float16)v[e], h1 = (_Float16)v[e + 1];
    const _Float16 l0 = (_Float16)(v[e] - (float)h0), l1 = (_Float16)(v[e + 1] - (float)h1);
    hw[e / 2] = (uint32_t)__builtin_bit_cast(uint16_t, h0) | (uint32_t)__builtin_bit_cast(uint16_t, h1) << 16;
    lw[e / 2] = (uint32_t)__builtin_bit_cast(uint16_t, l0) | (uint32_t)__builtin_bit_cast(uint16_t, l1) << 16;
    sum += v[e];
    sum += v[e + 1];
  }
  uint4* o = reinterpret_cast<uint4*>(XT) + ((((size_t)tt * KC + kc) * 2) * 2 + st) * 64 + 32 * hh + c;
  o[0] = make_uint4(hw[0], hw[1], hw[2], hw[3]);
  o[2 * 64] = make_uint4(lw[0], lw[1], lw[2], lw[3]);
  __shared__ float part[2][4][32];                       // the block's two chunks
  const int cb = (threadIdx.x >> 7) & 1;
  part[cb][q][c] = sum;
  __syncthreads();
  if (q == 0) {
    const float s = (part[cb][0][c] + part[cb][1][c]) + (part[cb][2][c] + part[cb][3][c]);
    const _Float16 hi = (_Float16)s;
    uint16_t* sx = SXT + ((((size_t)tt * NB + (kc >> 3)) * 2) * 32 + c) * 8 + (kc & 7);
    sx[0] = __builtin_bit_cast(uint16_t, hi);
    sx[32 * 8] = __builtin_bit_cast(uint16_t, (_Float16)(s - (float)hi));
  }
}

hipError_t launch_prefill_x(const float* X, void* XT, void* SXT, int m, int K, hipStream_t s) {
  if (m < 1 || K % 256) return hipErrorInvalidValue;
  const int mp = (m + 63) / 64 * 64;
  const size_t n = (size_t)mp * (K / 8);                 // a multiple of 256 (mp and K / 8 multiples of 32)
  hipLaunchKernelGGL(k_prefill_x, dim3((unsigned)(n / 256)), dim3(256), 0, s, X, static_cast<uint16_t*>(XT),
                     static_cast<uint16_t*>(SXT), m, K);
  return hipGetLastError();
}

size_t prefill_x_bytes(int m, int K) { return (size_t)((m + 63) / 64 * 64) * K * 4; }
size_t prefill_sx_bytes(int m, int K) { return (size_t)((m + 63) / 64 * 64) * (K / 32) * 4; }

hipError_t launch_gemm_prefill(const DevMat& M, const uint8_t* CT, int row0, int nrows, const void* XT,
                               const void* SXT, int m, float* Y, int ldy, hipStream_t s) {
  if (nrows < 1 || m < 1 || nrows % 64 || M.K % 256) return hipErrorInvalidValue;
  const dim3 grid(nrows / 64, (m + 31) / 32), block(64 * GEMM_WAVES);
  const uint16_t* x = static_cast<const uint16_t*>(XT);
  const uint16_t* sx = static_cast<const uint16_t*>(SXT);
  switch (M.kqt) {
    case KQ_Q4_K: hipLaunchKernelGGL(k_gemm_prefill<KQ_Q4_K>, grid, block, 0, s, M, CT, row0, x, sx, m, Y, ldy); break;
    case KQ_Q5_K: hipLaunchKernelGGL(k_gemm_prefill<KQ_Q5_K>, grid, block, 0, s, M, CT, row0, x, sx, m, Y, ldy); break;
    case KQ_Q6_K: hipLaunchKernelGGL(k_gemm_prefill_sub<KQ_Q6_K>, grid, block, 0, s, M, CT, row0, x, m, Y, ldy); break;
    case KQ_IQ4_XS: hipLaunchKernelGGL(k_gemm_prefill_sub<KQ_IQ4_XS>, grid, block, 0, s, M, CT, row0, x, m, Y, ldy); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// ── prefill through a library GEMM: decoded codes -> fp16 hi + lo weights (path 2, the default for m > 8) ────
// The reference's prefill dequantizes every weight to fp32, w = s f(q) - o (kernels/llmrt.cu:201-343, kq_w4), and runs
// a fp32 GEMM. Here w (the same fp32 value: product, then difference, no contraction) is split into fp16 hi = fp16(w)
// and lo = fp16(w - hi), stored per row as [hi x K | lo x K], and x likewise ([x hi | x hi] and [x lo]), so two fp16
// GEMMs with fp32 accumulation give x_hi w_hi + x_hi w_lo + x_lo w_hi: w and x to about 22 bits.
// WW is column-major for the GEMM (row n of the chunk, weight k): hi at WW[k nrows + n], lo at WW[(K + k) nrows + n],
// so the 64 rows of a tile store one weight as one 128-byte line.
// One thread = one sub-block of GW weights of one row; consecutive threads take consecutive rows.
template <int KQ>
__global__ void __launch_bounds__(256) k_dequant_hilo(DevMat M, const uint8_t* __restrict__ codes, int row0,
                                                      int nrows, uint16_t* __restrict__ WW) {
  constexpr int GW = kq_gw(KQ), SB = kq_sbytes(KQ), NSUB = 256 / GW;
  const int K = M.K, per_row = K / GW;
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (size_t)nrows * per_row) return;
  const int g = (int)(i / nrows), r = (int)(i - (size_t)g * nrows), b = g / NSUB, jj = g - b * NSUB;
  uint32_t sw[5];
  side_load<KQ>(M.side + side_record(row0 + r, b, M.KT, M.symbits == 4 ? 2 : 1) * SB, sw);
  float sc, o;
  side_scale<KQ>(sw, jj, sc, o);
  const uint8_t* cr = codes + (size_t)r * K + (size_t)g * GW;
  uint16_t* hc = WW + (size_t)g * GW * nrows + r;
  const size_t lo_off = (size_t)K * nrows;
#pragma unroll
  for (int c = 0; c < GW; c += 4) {
    const uint32_t q4 = *reinterpret_cast<const uint32_t*>(cr + c);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t q = (q4 >> (8 * e)) & 255u;
      const float f = KQ == KQ_Q6_K ? (float)q - 32.f : (KQ == KQ_IQ4_XS ? (float)IQ4_GRID[q & 15u] : (float)q);
      const float w = __fsub_rn(__fmul_rn(sc, f), o);
      const _Float16 hi = (_Float16)w;
      const _Float16 lo = (_Float16)(w - (float)hi);
      hc[(size_t)(c + e) * nrows] = __builtin_bit_cast(uint16_t, hi);
      hc[lo_off + (size_t)(c + e) * nrows] = __builtin_bit_cast(uint16_t, lo);
    }
  }
}

hipError_t launch_dequant_hilo(const DevMat& M, const uint8_t* codes, int row0, int nrows, void* WW, hipStream_t s) {
  if (nrows < 1 || M.K % 256) return hipErrorInvalidValue;
  const size_t n = (size_t)nrows * (M.K / kq_gw(M.kqt));
  const dim3 grid((unsigned)((n + 255) / 256));
  uint16_t* w = static_cast<uint16_t*>(WW);
  switch (M.kqt) {
    case KQ_Q4_K: hipLaunchKernelGGL(k_dequant_hilo<KQ_Q4_K>, grid, dim3(256), 0, s, M, codes, row0, nrows, w); break;
    case KQ_Q5_K: hipLaunchKernelGGL(k_dequant_hilo<KQ_Q5_K>, grid, dim3(256), 0, s, M, codes, row0, nrows, w); break;
    case KQ_Q6_K: hipLaunchKernelGGL(k_dequant_hilo<KQ_Q6_K>, grid, dim3(256), 0, s, M, codes, row0, nrows, w); break;
    case KQ_IQ4_XS: hipLaunchKernelGGL(k_dequant_hilo<KQ_IQ4_XS>, grid, dim3(256), 0, s, M, codes, row0, nrows, w); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// Decode + dequant in one kernel for the prefill GEMM: tile rows [tr0, tr1) of a coded K-quant matrix straight to
// WW (column-major hi then lo, as k_dequant_hilo). One block of 4 waves per tile, the tile and its decode table
// staged in LDS, 8 chains per lane over the load-time split offsets (as k_fused_split): wave w decodes symbols
// [64 w, 64 w + 64) of row l (lanes 0-31) and row l + 32 (lanes 32-63) and stores each weight as it comes, one
// 128-byte line per wave and weight (the tile's 64 rows).
template <int KQ>
__global__ void __launch_bounds__(256) k_decode_hilo(DevMat M, int tr0, int tr1, uint16_t* __restrict__ WW,
                                                     int stage_rows) {
  constexpr int SYMB = kq_symbits(KQ);
  constexpr int TW = SYMB == 4 ? 2 * TK : TK;
  constexpr int GW = kq_gw(KQ), SB = kq_sbytes(KQ), NSB = TW / 256;
  constexpr int WPP = SYMB == 4 ? 4 : 2;  // weights per symbol pair
  typedef __attribute__((address_space(3))) const uint32_t LdsU32;
  __shared__ uint32_t lut4[LUTN];
  extern __shared__ __align__(16) uint32_t tw[];
  const int KT = M.KT, K = M.K;
  const int t = tr0 * KT + (int)blockIdx.x;
  if (t >= tr1 * KT) return;
  const int tc = t % KT, tr = t / KT;
  const int R = min((int)M.rows[t] + 2, stage_rows);
  for (int i = threadIdx.x; i < LUTN / 4; i += 256)
    reinterpret_cast<uint4*>(lut4)[i] = reinterpret_cast<const uint4*>(M.lut4)[i];
  const uint4* src = reinterpret_cast<const uint4*>(M.words + M.tbase[t]);
  for (int i = threadIdx.x; i < 8 * R; i += 256) reinterpret_cast<uint4*>(tw)[i] = src[i];
  __syncthreads();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63, l = lane & 31, f = lane >> 5;
  const int k = 4 * f + wave;
  uint32_t P = (uint32_t)M.split[((size_t)t * SPLITS + k * (SPLITS / 8)) * 32 + (uint32_t)l] - GUARD_BITS + 64u;
  const uint32_t tsel = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const uint32_t*)lut4;
  uint32_t tmask = 0x1FFCu;
  asm volatile("" : "+v"(tmask));
  const uint32_t rlb = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint32_t*)(tw + l);
  uint32_t slot = __builtin_amdgcn_ubfe(P, 5, 8);
  uint32_t A = *(LdsU32*)(rlb + ((slot - 2u) << 7));
  uint32_t B = *(LdsU32*)(rlb + ((slot - 1u) << 7));
  uint32_t C = *(LdsU32*)(rlb + (slot << 7));
  const int n = tr * TN + f * 32 + l;          // matrix row
  const int col0 = tc * TW + wave * (TW / 4);  // the chain's first weight: 64 symbols = a quarter of the tile row
  const int b = col0 / 256;                    // the chain's super-block (a quarter never spans two)
  uint32_t sw[5];
  side_load<KQ>(M.side + side_record(n, b, KT, NSB) * SB, sw);
  const int nrows = (tr1 - tr0) * TN;
  uint16_t* hc = WW + (size_t)col0 * nrows + (n - tr0 * TN);
  const size_t lo_off = (size_t)K * nrows;
#pragma unroll 1
  for (int gi = 0; gi < 4; ++gi) {
    // the group's 16 symbols = 32 (4-bit) or 16 weights: one sub-block scale (Q5_K: half a sub-block)
    const int jj = ((col0 - 256 * b) + gi * 8 * WPP) / GW;
    float sc, o;
    side_scale<KQ>(sw, jj, sc, o);
#pragma unroll
    for (int p2 = 0; p2 < 8; p2 += 2) {
#pragma unroll
      for (int pp = 0; pp < 2; ++pp) {
        const uint32_t w1 = __builtin_amdgcn_alignbit(B, A, P);
        const uint32_t e1 = *(LdsU32*)table_addr(w1, tsel, tmask);
        const uint32_t w2 = w1 >> (e1 & 31u);
        const uint32_t e2 = *(LdsU32*)table_addr(w2, tsel, tmask);
        P = P + e1 + e2;
        const uint32_t nslot = __builtin_amdgcn_ubfe(P, 5, 8);
        const bool slide = nslot != slot;
        A = slide ? B : A;
        B = slide ? C : B;
        slot = nslot;
        C = *(LdsU32*)(rlb + (nslot << 7));
        float fv[WPP];
        if (SYMB == 4) {  // entry bytes 2, 3: the symbol's two grid bytes (IQ4_XS: kv[q] + 128)
          const float bias = KQ == KQ_IQ4_XS ? 128.f : 0.f;
          fv[0] = (float)((e1 >> 16) & 255u) - bias;
          fv[1] = (float)(e1 >> 24) - bias;
          fv[2] = (float)((e2 >> 16) & 255u) - bias;
          fv[3] = (float)(e2 >> 24) - bias;
        } else {  // bits 16-31: fp16 f(q)
          fv[0] = h2f(e1 >> 16);
          fv[1] = h2f(e2 >> 16);
        }
        const int c = (gi * 8 + p2 + pp) * WPP;  // the pair's first weight within the chain
#pragma unroll
        for (int e = 0; e < WPP; ++e) {
          const float w = __fsub_rn(__fmul_rn(sc, fv[e]), o);
          const _Float16 hi = (_Float16)w;
          const _Float16 lo = (_Float16)(w - (float)hi);
          hc[(size_t)(c + e) * nrows] = __builtin_bit_cast(uint16_t, hi);
          hc[lo_off + (size_t)(c + e) * nrows] = __builtin_bit_cast(uint16_t, lo);
        }
      }
    }
  }
}

hipError_t launch_decode_hilo(const DevMat& M, int tr0, int tr1, void* WW, hipStream_t s) {
  if (M.packed || !M.split || !M.lut4 || !M.rows || tr0 < 0 || tr1 > M.NT || tr0 >= tr1 || M.K % 256)
    return hipErrorInvalidValue;
  const int rows = M.max_rows + 2;
  const size_t smem = (size_t)rows * 128;
  if (rows > 256 || smem + 4 * LUTN > 160 * 1024) return hipErrorInvalidValue;
  const dim3 grid((unsigned)((tr1 - tr0) * M.KT));
  uint16_t* w = static_cast<uint16_t*>(WW);
  const void* f = nullptr;
  switch (M.kqt) {
    case KQ_Q4_K: f = reinterpret_cast<const void*>(&k_decode_hilo<KQ_Q4_K>); break;
    case KQ_Q5_K: f = reinterpret_cast<const void*>(&k_decode_hilo<KQ_Q5_K>); break;
    case KQ_Q6_K: f = reinterpret_cast<const void*>(&k_decode_hilo<KQ_Q6_K>); break;
    case KQ_IQ4_XS: f = reinterpret_cast<const void*>(&k_decode_hilo<KQ_IQ4_XS>); break;
    default: return hipErrorInvalidValue;
  }
  hipError_t e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
  if (e != hipSuccess) return e;
  switch (M.kqt) {
    case KQ_Q4_K: hipLaunchKernelGGL(k_decode_hilo<KQ_Q4_K>, grid, dim3(256), smem, s, M, tr0, tr1, w, rows); break;
    case KQ_Q5_K: hipLaunchKernelGGL(k_decode_hilo<KQ_Q5_K>, grid, dim3(256), smem, s, M, tr0, tr1, w, rows); break;
    case KQ_Q6_K: hipLaunchKernelGGL(k_decode_hilo<KQ_Q6_K>, grid, dim3(256), smem, s, M, tr0, tr1, w, rows); break;
    default: hipLaunchKernelGGL(k_decode_hilo<KQ_IQ4_XS>, grid, dim3(256), smem, s, M, tr0, tr1, w, rows); break;
  }
  return hipGetLastError();
}

// x [m][K] fp32 -> XX [m][2K] = [hi | hi] and XL [m][K] = lo (fp16)
__global__ void k_split_x_gemm(const float* __restrict__ X, uint16_t* __restrict__ XX, uint16_t* __restrict__ XL,
                               int m, int K) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (size_t)m * K) return;
  const size_t j = i / K, k = i - j * K;
  const float x = X[i];
  const _Float16 hi = (_Float16)x;
  const _Float16 lo = (_Float16)(x - (float)hi);
  XX[j * 2 * K + k] = XX[j * 2 * K + K + k] = __builtin_bit_cast(uint16_t, hi);
  XL[i] = __builtin_bit_cast(uint16_t, lo);
}

// x [m][K] fp32 -> XB [2m][2K] fp16: rows t < m = [hi | hi], rows m + t = [lo | 0] (the B operand of the one-GEMM
// prefill form, whose 2m columns give x_hi w_hi + x_hi w_lo and x_lo w_hi side by side)
__global__ void k_split_x_gemm2(const float* __restrict__ X, uint16_t* __restrict__ XB, int m, int K) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (size_t)m * K) return;
  const size_t j = i / K, k = i - j * K;
  const float x = X[i];
  const _Float16 hi = (_Float16)x;
  const _Float16 lo = (_Float16)(x - (float)hi);
  uint16_t* r = XB + j * 2 * K;
  r[k] = r[K + k] = __builtin_bit_cast(uint16_t, hi);
  uint16_t* q = XB + ((size_t)m + j) * 2 * K;
  q[k] = __builtin_bit_cast(uint16_t, lo);
  q[K + k] = 0;
}

hipError_t launch_split_x_gemm2(const float* X, void* XB, int m, int K, hipStream_t s) {
  const size_t n = (size_t)m * K;
  hipLaunchKernelGGL(k_split_x_gemm2, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, X, static_cast<uint16_t*>(XB),
                     m, K);
  return hipGetLastError();
}

// Y[t][n] = T[t][n] + T[m + t][n] for the one-GEMM prefill form (T [2m][nr] fp32, Y rows ldy apart)
__global__ void k_add_halves(const float* __restrict__ T, float* __restrict__ Y, int m, int nr, int ldy) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (size_t)m * nr) return;
  const size_t t = i / nr, n = i - t * nr;
  Y[t * ldy + n] = T[i] + T[(size_t)m * nr + i];
}

hipError_t launch_add_halves(const float* T, float* Y, int m, int nr, int ldy, hipStream_t s) {
  const size_t n = (size_t)m * nr;
  hipLaunchKernelGGL(k_add_halves, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, T, Y, m, nr, ldy);
  return hipGetLastError();
}

hipError_t launch_split_x_gemm(const float* X, void* XX, void* XL, int m, int K, hipStream_t s) {
  const size_t n = (size_t)m * K;
  hipLaunchKernelGGL(k_split_x_gemm, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, X,
                     static_cast<uint16_t*>(XX), static_cast<uint16_t*>(XL), m, K);
  return hipGetLastError();
}

// ── HBM streaming-read control ──────────────────────────────────────────────────────────────────────────
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
// p[i] = v for i < n (clears counters in caller-owned scratch; a kernel, so that a graph capture records no memset)
__global__ void __launch_bounds__(256) k_fill_u32(uint32_t* __restrict__ p, size_t n, uint32_t v) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) p[i] = v;
}

hipError_t launch_fill_u32(uint32_t* p, size_t n, uint32_t v, hipStream_t s) {
  if (!n) return hipSuccess;
  const int blocks = (int)std::min<size_t>((n + 255) / 256, 1024);
  hipLaunchKernelGGL(k_fill_u32, dim3(blocks), dim3(256), 0, s, p, n, v);
  return hipGetLastError();
}

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

#ifdef LW_TIMELINE
// the diagnostic build's timestamps (see g_timeline): copied out, or cleared
extern "C" int lw_timeline_read(void* dst, size_t bytes) {
  return (int)hipMemcpyFromSymbol(dst, HIP_SYMBOL(lw::g_timeline), bytes, 0, hipMemcpyDeviceToHost);
}
extern "C" int lw_timeline_clear() {
  void* p = nullptr;
  hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(lw::g_timeline));
  if (e == hipSuccess) e = hipMemset(p, 0, sizeof(lw::g_timeline));
  if (e == hipSuccess) e = hipDeviceSynchronize();
  return (int)e;
}
#endif
