// Device-side matrix descriptor and kernel launchers (host interface of lw_kernels.hip).
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>

namespace lw {

// One coded matrix resident in HBM, in the device layout built by the runtime at load time:
//   lut   u16[2048]            the bundle's decode table (sym | len << 8)
//   tbase u32[T]               word index (into words) of tile t's first word row
//   mid   u16[T][32]           bit offset, within lane l's stream, of the lane's second row (symbol 256)
//   words u32[...]             tile t: word i of lane l at tbase[t] + 32 i + l, i < rows[t]; every lane stream
//                              starts at bit 0 of its word 0; rows[t] = the tile's longest lane in words; zero tail
//   side  u8[N*K/256][SB]      K-quant side records of the bundle's <name>.kqs in tile-major order (side_record)
//   sched u32x4[T]             ring staging schedule of each tile (lw_layout.h, Layout::sched); w bit 0: no schedule
// Every lane stream starts with GUARD = 2 zero bits (symbol 0 at stream bit 2).
struct DevMat {
  const uint16_t* lut;
  const uint32_t* lut4;  // the ring kernels' 4-byte table entries (decode_table4 in lw_layout.h); null if kqt == 0
  const uint32_t* luti8; // the same with int8 grid values (decode_table_i8), for int8 activations
  const uint32_t* canon; // the comparator form of lut4 (canon_table in lw_layout.h); null if the codes are not canonical
  const uint32_t* tbase;
  const uint16_t* mid;
  const uint16_t* split;  // [T][SPLITS][32] chain starts of the low-latency and whole-tile kernels (Layout::split)
  const uint16_t* rows;
  const uint32_t* hrow;  // [T] the half-tile units' rows (Layout::hrow)
  // [T][2 f][64 lanes][4] the half-tile kernel's chain starts: lane 32 h + s of unit (t, f) starts its chain j at
  // split offset 8 f + 4 h + j of lane stream s
  const uint16_t* hsplit;
  // [T][2 f][32 s] the whole-tile kernels' chain starts of lane stream s, row f: after the first (mid for f = 1, the
  // guard for f = 0) 7 deltas of 32 symbols each, less 32, 9 bits each
  const uint64_t* dsplit;
  const uint32_t* words;
  const uint8_t* side;
  const uint4* sched;
  int N, K;         // weights
  int kqt;          // 1 Q4_K, 2 Q5_K, 3 Q6_K, 4 IQ4_XS (0: none -> decode only)
  int symbits;      // 4 (huf4p) or 8 (huf8)
  int KT, NT;       // tile columns, tile rows
  int max_rows;     // max over tiles of rows[t]
  int tstride;      // > 0: tile t's words at words + 32 tstride t (= tbase[t]), tstride = max_rows; 0: read tbase
  int max_hrows;    // max over tiles and halves of a half-tile unit's rows
  int ring_rows;    // 16 / 32: ring kernel usable with that ring; 0: whole-tile kernel only
  // tiles the ring kernel skips (no schedule for ring_rows): the first nexc32 have a 32-row ring schedule (decoded
  // by the flat ring kernel from this list), the rest go through the whole-tile kernel
  const uint32_t* exc;
  int nexc, nexc32;
  // 1: a packed (fixed-rate) matrix: words = the symbols as 16-byte chunks [T][16][64], lut4 = 256 symbol entries
  int packed;
};

// Matrices of one grouped launch of the ring kernel (same K-quant type and ring size). Matrix i owns blocks
// [block0, block0 + KT * ceil(NT / WPB)); X2 = its fp16 activations [mt][K] as pairs, P its partials [KT][mt][N]
// (the exception tiles' partials are written by the whole-tile kernel's pass).
constexpr int MAX_GROUP = 8;
// A partials slot between a reduction's read and the next partial's store (a signalling NaN: no arithmetic result
// is one). Every reduction puts its slots back to this value; a partials buffer starts filled with it.
constexpr uint32_t kNoPartial = 0x7F80A5A5u;
// re-reads of a counted partial that is not yet visible before the in-launch reduction gives up (NaN, not a hang)
constexpr int kPartialSpins = 1 << 16;
struct GroupEntry {
  DevMat M;
  const uint32_t* X2;
  float* P;
  int block0;
};
struct GroupPlan {
  GroupEntry e[MAX_GROUP];
  int n;
  int mt;
  int blocks;
};
// Matrices of one launch of the flat ring kernel (m = 1, or up to 8 tokens of int8 activations; same K-quant type and
// ring size). Their tiles form one list:
// matrix i owns tiles [tile0, tile0 + NT * KT), column-major; block b decodes tiles [b W, b W + W). Every matrix must
// have at least W tiles, so a block spans at most two matrices.
struct FlatEntry {
  DevMat M;
  const uint32_t* X2;
  float* P;
  // null: every tile of the matrix (the ring and packed kernels take them column-major, the whole-tile kernels
  // row-major); else these tile indices (exception pass)
  const uint32_t* list;
  int tile0, ntile;
  // Y non-null (the launch decodes every tile of the matrix): Y[n] = the ordered sum of P over tile columns, formed
  // in the launch by the last wave of each tile row; cnt = NT zeroed counters (left zeroed)
  float* Y;
  uint32_t* cnt;
  // int8 activations (plan.i8): x quantized per 32 weights (launch_quant_x8): XQ [mt][K] int8, DX / SX [mt][K / 32]
  const int8_t* XQ;
  const float* DX;
  const float* SX;
  // plan.mt > 1: P is [KT][mt][N] and token j's Y row starts at Y + j ldy
  int ldy;
};
struct FlatPlan {
  FlatEntry e[MAX_GROUP];
  int n;
  int W;       // waves (tiles) per block, <= 16 (<= 8 for 32-row rings)
  int ntiles;  // all tiles of the plan
  // 16-row launches: spare 16-row ring pairs per block for exception tiles with a 32-row schedule (>= the most
  // such tiles in any block); 0: exception tiles are skipped (decoded by an exception pass)
  int nspare;
  int i8;  // 1: int8 activations (the entries' XQ / DX / SX)
  int mt;  // tokens: 0 or 1, or 2..8 with int8 activations (the flat ring and low-latency kernels, one pass)
  int canon;  // 1: the whole-tile kernel (fp16 activations) looks codes up by the comparator form (DevMat::canon)
  // the whole-tile kernel (fp16 activations) over two K-quant types: entries [0, nfa) of one, [nfa, n) of the other;
  // nfa = n (or 0) when every entry has the first entry's type
  int nfa;
};
hipError_t launch_fused_flat(const FlatPlan& plan, hipStream_t s);
// waves of the flat kernel one CU holds at once (its register use) for int8 activations, mt tokens (1, or 2..8)
int flat_waves_per_cu(int kqt, int rs, int mt);
// The low-latency kernel over the same kind of plan (one tile per block of 4 waves, 8 chains per lane; W and
// nspare are ignored; exception tiles included). Every matrix needs a K-quant table and the split offsets.
hipError_t launch_fused_split(const FlatPlan& plan, hipStream_t s);
// int8 activations as the reference's k_quant_x8 (kernels/llmrt.cu:1035-1055): X [m][K] (fp32, or fp16 when x_f16)
// in blocks of 32: d = amax / 127, q = round-to-nearest-even(x / d) (0 when d = 0), XQ = q, DX = d, SX = d sum q.
hipError_t launch_quant_x8(const void* X, int x_f16, int m, int K, int8_t* XQ, float* DX, float* SX, hipStream_t s);
// up to MAX_GROUP vectors in one launch: job i quantizes nb[i] blocks of 32 from X[i]
struct QuantJobs {
  const void* X[MAX_GROUP];
  int8_t* XQ[MAX_GROUP];
  float* DX[MAX_GROUP];
  float* SX[MAX_GROUP];
  int nb[MAX_GROUP];
  int b0[MAX_GROUP];  // first block-of-8 index of each job in the launch
  int n, x_f16;
};
hipError_t launch_quant_x8_group(const QuantJobs& q, hipStream_t s);
// LDS rows the low-latency kernel stages per tile for this plan (max over its matrices of max_rows + 2)
int split_stage_rows(const FlatPlan& plan);
// whole-tile kernel for flat launches (m = 1): block = plan.W waves over `per` consecutive tiles (>= W), a tile per
// wave in LDS at a time (tiles_buf_rows rows), 8 chains per lane; every tile of the entries (exceptions included)
// and the in-launch reduction for entries with Y. With fp16 activations the entries may hold two K-quant types
// (FlatPlan::nfa: the first nfa entries of the smaller type code, the rest of the larger), one launch for both.
hipError_t launch_fused_tiles(const FlatPlan& plan, int per, hipStream_t s);
// the most waves of a whole-tile block with the comparator lookup (FlatPlan::canon)
constexpr int TILES_CANON_WAVES = 12;
// LDS row counters of the whole-tile kernel (m = 1): a tile row that starts within this many tiles of a block's first
// tile and ends among its tiles is counted in LDS; the static LDS is the tables plus 4 + TILES_ROWC words
constexpr int TILES_ROWC = 64;
// The half-tile kernel (m = 1, fp16 activations, no int8): as launch_fused_tiles, but a wave decodes half-tile units
// (a tile's rows 32 f .. 32 f + 31) with two LDS buffers, the next unit's copy in flight while one decodes; the
// in-launch reduction per tile row and half (each entry's cnt holds 2 NT counters). W waves per block, each with two
// buffers of halves_buf_rows word rows.
hipError_t launch_fused_halves(const FlatPlan& plan, int per, hipStream_t s);
int halves_buf_rows(const FlatPlan& plan);
int tiles_buf_rows(const FlatPlan& plan);
// The whole-tile kernel for 2..8 tokens of fp16 activations (every format, plan.mt tokens, every tile of each entry):
// the products on the matrix cores (4x4x4 blocks, x broadcast from one block), every token in one pass over the
// tiles; each block forms the x sums of its tile columns in LDS (tiles_mma_xs_bytes beside W tile buffers of
// tiles_buf_rows word rows)
hipError_t launch_fused_tiles_mma(const FlatPlan& plan, int per, hipStream_t s);
size_t tiles_mma_xs_bytes(const FlatPlan& plan, int per);
// The same for int8 activations (plan.i8, 2..8 tokens, every format; the entries' XQ / DX / SX from
// launch_quant_x8): integer products on the matrix cores per sub-block, folded with the block scales in fp32
hipError_t launch_fused_tiles_mma8(const FlatPlan& plan, int per, hipStream_t s);
int tiles_mma_max_waves(int kqt, int mt);  // the block limit of both matrix-core whole-tile kernels

// One launch of the ring kernel over all matrices of the plan (returns hipErrorInvalidValue if the plan mixes
// K-quant types or ring sizes, or a matrix has no ring schedule).
hipError_t launch_fused_group(const GroupPlan& plan, hipStream_t s);
int group_waves_per_block(int ring_rows);
// The packed (fixed-rate) twin over a plan of packed matrices of one K-quant type: blocks of 16 tile rows of one
// tile column (block0 as for the ring kernel with 16 waves per block); partials as the ring kernel's.
hipError_t launch_fused_packed(const GroupPlan& plan, hipStream_t s);
// The packed twin for m = 1 over a flat plan (one tile per wave, W waves per block, every matrix whole; no lists).
hipError_t launch_fused_packed_flat(const FlatPlan& plan, hipStream_t s);

// Ordered reduction of several matrices in one launch: Y_i[j][n] (row stride ldy) = the sum over tile columns tc (in
// order) of P_i[tc][jj][n], jj over the `per` pseudo-tokens of token j (per = 1: fp16 activations; per = 2: fp32
// activations split into fp16 hi + lo).
struct ReduceEntry {
  float* P;  // read, then every slot set back to kNoPartial
  float* Y;
  int N, KT, ldy, out0;  // out0 = first output index of this matrix in the flattened launch (m * N each)
};
struct ReducePlan {
  ReduceEntry e[MAX_GROUP];
  int n, m, per, total;
};
hipError_t launch_reduce_group(const ReducePlan& plan, hipStream_t s);

// X16 [mt][K] fp16 (mt pseudo-tokens); P [KT][mt][N] fp32 per-tile-column partials.
hipError_t launch_fused(const DevMat& M, const void* X16, int mt, float* P, hipStream_t s);
// the whole-tile kernel over M.exc[nexc32 .. nexc) (exception tiles without any ring schedule); no-op if none
hipError_t launch_fused_exceptions(const DevMat& M, const void* X16, int mt, float* P, hipStream_t s);
// fp32 X [m][K] -> fp16 X16 [2m][K] (row 2j = hi, 2j + 1 = lo = x - hi)
hipError_t launch_split_x(const float* X, void* X16, int m, int K, hipStream_t s);
// codes [N][K] (one byte per weight) for tile rows [tr0, tr1)
hipError_t launch_decode(const DevMat& M, uint8_t* out, int tr0, int tr1, hipStream_t s);
// simple K-quant GEMM from decoded codes (m > 8 or path 2): Y[m][N] = X[m][K] dequant(codes, side)^T
hipError_t launch_gemm_codes(const DevMat& M, const uint8_t* codes, int row0, int nrows, const float* X, int m,
                             float* Y, int ldy, hipStream_t s);
// the same on the matrix cores, with X16 = fp16 hi / lo rows [2m][K] (launch_split_x), rows [row0, row0 + nrows)
// Prefill through a library GEMM: codes rows [row0, row0 + nrows) (from launch_decode, [nrows][K]) -> WW, the
// column-major [nrows x 2K] fp16 matrix of w = s f(q) - o (fp32, as the reference's kq_w4): hi of weight k of row r
// at WW[k nrows + r], lo at WW[(K + k) nrows + r]
hipError_t launch_dequant_hilo(const DevMat& M, const uint8_t* codes, int row0, int nrows, void* WW, hipStream_t s);
// The same from the coded matrix directly (decode + dequant in one kernel; coded K-quant matrices with split
// offsets): tile rows [tr0, tr1) -> WW rows relative to tr0 * 64
hipError_t launch_decode_hilo(const DevMat& M, int tr0, int tr1, void* WW, hipStream_t s);
// Prefill GEMM on the matrix cores, every K-quant format (k_gemm_prefill: Q4_K / Q5_K; k_gemm_prefill_sub: Q6_K /
// IQ4_XS): Y[t][row0 + r] for the chunk's rows r < nrows (a multiple of 64) from its codes in the tiled layout
// (launch_decode_tiled) and x in the tiled layouts of launch_prefill_x (SXT read for Q4_K / Q5_K only); K a multiple
// of 256
hipError_t launch_gemm_prefill(const DevMat& M, const uint8_t* CT, int row0, int nrows, const void* XT,
                               const void* SXT, int m, float* Y, int ldy, hipStream_t s);
// codes of tile rows [tr0, tr1) in the prefill GEMM's tiled layout: per 32-row tile and 32-code chunk a 1 KB piece,
// lane (h, c) = 32 h + c holding row c's codes 16 h .. 16 h + 15 of the chunk (IQ4_XS: their grid bytes kv[q] + 128);
// hipErrorNotSupported unless decode_tiled_ok (packed matrices, coded ones with split offsets)
bool decode_tiled_ok(const DevMat& M);
hipError_t launch_decode_tiled(const DevMat& M, uint8_t* out, int tr0, int tr1, hipStream_t s);
// fp32 X [m][K] -> XT (fp16 hi / lo pieces, prefill_x_bytes) and SXT (per-sub-block sums as fp16 hi / lo,
// prefill_sx_bytes), tokens padded with zeros to a multiple of 64; K a multiple of 256
hipError_t launch_prefill_x(const float* X, void* XT, void* SXT, int m, int K, hipStream_t s);
size_t prefill_x_bytes(int m, int K);
size_t prefill_sx_bytes(int m, int K);
// x [m][K] fp32 -> XB [2m][2K] fp16: rows t < m [hi | hi], rows m + t [lo | 0]
hipError_t launch_split_x_gemm2(const float* X, void* XB, int m, int K, hipStream_t s);
// Y[t][n] (rows ldy apart) = T[t][n] + T[m + t][n], T [2m][nr] fp32
hipError_t launch_add_halves(const float* T, float* Y, int m, int nr, int ldy, hipStream_t s);
// x [m][K] fp32 -> XX [m][2K] fp16 = [hi | hi], XL [m][K] fp16 = lo
hipError_t launch_split_x_gemm(const float* X, void* XX, void* XL, int m, int K, hipStream_t s);
hipError_t launch_gemm_codes_mfma(const DevMat& M, const uint8_t* codes, int row0, int nrows, const void* X16, int m,
                                  float* Y, int ldy, hipStream_t s);
// p[i] = v for i < n, as a kernel on stream s
hipError_t launch_fill_u32(uint32_t* p, size_t n, uint32_t v, hipStream_t s);
// streaming read of n16 16-byte words (achievable HBM bandwidth control); out gets one value per block
hipError_t launch_stream_read(const void* src, size_t n16, float* out, int blocks, hipStream_t s);

}  // namespace lw
