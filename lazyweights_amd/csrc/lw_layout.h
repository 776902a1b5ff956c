// Host-side load-time transforms of coded matrices: bundle blob (or the reference's pre-interleaved export) ->
// the device layout read by the kernels, and the CPU decode of a raw blob.
#pragma once
#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

namespace lw {

// Every lane stream starts with GUARD zero bits in the device layout, so the window of the symbol at stream bit p is
// read at q = p - GUARD and the byte offset of its 4-byte table entry is (window & 0x1FFC): one AND per symbol.
constexpr int GUARD = 2;
// Zero rows appended after the last tile (read-ahead of the staging copies and of the 64-bit windows; the
// whole-tile kernel copies rows + 2 rounded up to 8).
constexpr int TAIL_ROWS = 16;
// Symbols per staging group (one sub-block of the 4-bit formats) and groups per chain (256 symbols).
constexpr int GROUP_SYMS = 16;
constexpr int GROUPS = 16;
// Rows per staged chunk (one 8-byte load per lane of a 32-lane front) and most chunks a front loads per group.
constexpr int CHUNK_ROWS = 2;
constexpr int MAX_CHUNKS_PER_GROUP = 2;

// Device layout of one coded matrix (see DevMat in lw_kernels.h for the field meanings).
struct Layout {
  uint16_t lut[2048];
  std::vector<uint32_t> tbase;  // [T]
  std::vector<uint16_t> mid;    // [T][32] device bit offset of symbol 256 (guard included)
  // [T][16][32] device bit offsets of symbols 32 k, k = 0..15 (guard included; k = 8 is mid): the chain starts
  // of the low-latency kernel (every second one) and the whole-tile kernel
  std::vector<uint16_t> split;
  std::vector<uint16_t> rows;   // [T]
  // [T] the half-tile units' word rows: bits 0-15 = rows [0, r) hold every bit of the lanes' first rows (symbols
  // 0..255), bits 16-31 = the first row the second rows' windows read (the row of each lane's bit mid - 2; their
  // last row is rows[t] - 1)
  std::vector<uint32_t> hrow;
  std::vector<uint32_t> words;  // tiles' word rows + zero tail
  // ring staging schedule per tile, 2 x u64: word 0 = 2-bit counts of 2-row chunks that front 0 (bits 2g) and
  // front 1 (bits 32 + 2g) load at group g; word 1 = base row of front 1 (bits 0-7), initial chunks of front 0
  // (8-15) and front 1 (16-23), bit 32: no schedule for ring_rows (an exception tile), bit 33: an exception tile
  // whose schedule (in words 0-1) is for a 32-row ring
  std::vector<uint64_t> sched;
  int ring_rows = 0;            // 16 or 32 rows per front; 0: the ring schedule does not fit (whole-tile kernels)
  // tiles without a schedule for ring_rows (bit 32 of their sched word 1 set): decoded with 32-row rings (in the
  // ring launch's spare rings, or a one-wave launch over this list) or by the whole-tile kernel
  std::vector<uint32_t> exc;
  int nexc32 = 0;  // the first nexc32 exception tiles have a 32-row ring schedule (in sched)
  int max_rows = 0;
  // > 0: tile t's rows start at word 32 tstride t (tstride = max_rows; tbase holds the same offsets); 0: tiles are
  // back to back
  int tstride = 0;
  int max_hrows = 0;  // max over tiles and halves of a half-tile unit's rows
  uint64_t payload_bits = 0;    // coded bits of all lanes
};

// From a raw huf8/huf4p blob (lazyweights/bundle.py:14-21). N rows, KS symbols per row. Every lane is decoded once
// on the host to find its second-row offset, exact length and the staging schedule, which also validates the blob.
bool build_layout_raw(const uint8_t* blob, size_t len, int N, int KS, int threads, Layout& L, std::string& err);

// From the reference's pre-interleaved export (enc suffix _il / _ilc; kernels/llmrt.cu:454-470, 1206-1257).
bool build_layout_il(const uint8_t* data, size_t len, int N, int KS, bool compact, int threads, Layout& L,
                     std::string& err);

// CPU decode of a raw blob (nbytes long) to symbols [N, KS]: the semantics of the reference's cpu_decode
// (kernels/llmrt.cu:2513-2541: one table lookup per symbol from each lane's absolute start, lane l of tile t writing
// row 64 tr + l then row 64 tr + 32 + l). Each lane reads through its own 64-bit bit buffer; tiles are split into
// contiguous ranges over `threads` threads. The header, every lane start and every lane's end are checked against
// the blob's size: false (with err) on a truncated or corrupt blob. *seconds = decode time (blob already in memory).
bool cpu_decode(const uint8_t* blob, size_t nbytes, int N, int KS, int threads, uint8_t* out, double* seconds,
                std::string& err);

int default_threads();

// The ring kernels' decode table for K-quant type kqt (1..4): entry i = code length (bits 0-7) and, for 4-bit
// symbols, the two grid bytes at bytes 2 and 3 (Q4_K: q; IQ4_XS: kv[q] + 128), for 8-bit symbols fp16(f(q)) in bits
// 16-31 (Q5_K: q; Q6_K: q - 32).
void decode_table4(int kqt, const uint16_t* lut, uint32_t* out);
// The int8-activation kernels' table: as decode_table4, with the grid values as int8 bytes (4-bit symbols: bytes 2
// and 3 = f(q) of the low and high code, Q4_K q, IQ4_XS kv[q]; 8-bit symbols: byte 2 = f(q), Q5_K q, Q6_K q - 32).
void decode_table_i8(int kqt, const uint16_t* lut, uint32_t* out);
// The comparator form of the table (reference hw/huff/huff_engine.h:39-77, build_canon + lookup): out[0..9] = the
// limits of code lengths 1..10 (an 11-bit window value v, first code bit most significant, holds a code longer
// than k when v >= limit k), out[10..20] = for lengths l = 1..11: (4 (base_l - first_l)) << 16 | (11 - l), out[21..31]
// = 0, out[32..287] = entries[] (decode_table4 entries) of the symbols in canonical order (by length, then
// symbol), so that entry index base_l + (v >> (11 - l)) - first_l is the code's. False when the table's codes are
// not the canonical code of their lengths (no window may then be looked up this way).
constexpr int CANON_WORDS = 288;
bool canon_table(const uint16_t* lut, const uint32_t* entries, uint32_t* out);

}  // namespace lw
