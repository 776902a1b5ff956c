// Host-side load-time transforms of coded matrices: bundle blob (or the reference's pre-interleaved export) ->
// the device layout read by the kernels, and the CPU decode of a raw blob.
#pragma once
#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

namespace lw {

// Device layout of one coded matrix (see DevMat in lw_kernels.h for the field meanings).
struct Layout {
  uint16_t lut[2048];
  std::vector<uint32_t> tbase;  // [T]
  std::vector<uint16_t> mid;    // [T][32]
  std::vector<uint16_t> rows;   // [T]
  std::vector<uint32_t> words;  // tiles' word rows + zero tail
  int max_rows = 0;
  uint64_t payload_bits = 0;    // coded bits of all lanes
};

// Zero rows appended after the last tile (read-ahead of the staging copy and of the 64-bit window).
constexpr int TAIL_ROWS = 3;

// From a raw huf8/huf4p blob (lazyweights/bundle.py:14-21). N rows, KS symbols per row. Every lane is decoded once
// on the host to find its second-row offset and exact length, which also validates the blob.
bool build_layout_raw(const uint8_t* blob, size_t len, int N, int KS, int threads, Layout& L, std::string& err);

// From the reference's pre-interleaved export (enc suffix _il / _ilc; kernels/llmrt.cu:454-470, 1206-1257).
bool build_layout_il(const uint8_t* data, size_t len, int N, int KS, bool compact, int threads, Layout& L,
                     std::string& err);

// CPU decode of a raw blob to symbols [N, KS] (kernels/llmrt.cu:2513-2541: per-lane scalar LUT decode with a 64-bit
// window from the lane's absolute start, tiles strided across `threads`). Returns seconds.
double cpu_decode(const uint8_t* blob, int N, int KS, int threads, uint8_t* out);

int default_threads();

}  // namespace lw
