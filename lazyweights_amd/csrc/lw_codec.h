// Host-side codec: length-limited canonical Huffman tables, the huf8/huf4p blob encoder, the seeded synthetic
// K-quant matrix generator and the bundle directory writer. None of this is on the decode path; it produces the
// bundles that the runtime opens.
#pragma once
#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

#include "lw_format.h"

namespace lw {

// Heap Huffman code lengths; ties broken by (count, insertion order) exactly as lazyweights/huffman.py:8-26.
void code_lengths(const int64_t* counts, int n, int* lens);
// Length limit by halving the counts until the longest code fits (lazyweights/lanecodecs.py:28-38).
void limited_lengths(const int64_t* counts, int n, int lmax, uint8_t* L);
// Canonical codes, ascending by (length, symbol) (lazyweights/lanecodecs.py:41-51).
void canonical_codes(const uint8_t* L, int n, uint32_t* codes);
uint32_t bitrev(uint32_t v, int nbits);
// 2048-entry decode table: lut[rev(code) + (j << len)] = sym | len << 8 (lazyweights/bundle.py:46-54).
void build_lut(const uint8_t* L, uint16_t* lut);

struct Encoded {
  std::vector<uint8_t> blob;
  uint64_t payload_bits = 0;
  uint8_t lengths[256] = {0};
};
// Symbols [N, KS] -> blob (lazyweights/bundle.py:57-85): lut ‖ lane starts ‖ payload words (+2 zero tail words).
bool encode_huf8(const uint8_t* sym, int N, int KS, int threads, Encoded& out, std::string& err);

// Blob byte size for a given payload bit count.
inline size_t blob_bytes(int N, int KS, uint64_t bits) {
  const size_t T = (size_t)(N / TN) * (KS / TK);
  return (size_t)2 * LUTN + T * LANES * 4 + 4 * ((bits + 31) / 32 + 2);
}

// fp32 -> fp16 bits, round to nearest even (host).
uint16_t f32_to_f16(float f);
float f16_to_f32(uint16_t h);

// Two-sided geometric code distribution P(q) ∝ rho^|q - centre| over [0, ncodes), rho solved for `entropy` bits.
void code_distribution(int ncodes, int centre, double entropy, double* p);

// Seeded synthetic K-quant matrix: codes [N, K] (one byte per weight, the format's own code values) and side bytes
// [N, K / 256 * SB]. Rows are generated from per-row seeds, so the result does not depend on `threads`.
void synth_matrix(int kqt, int N, int K, double entropy, uint64_t seed, uint8_t* codes, uint8_t* side, int threads);

// Codes [N, K] -> symbols [N, KS] (pairs for 4-bit formats: low nibble = even column; scripts/a2_kq_bundle.py:108).
void form_symbols(int kqt, const uint8_t* codes, int N, int K, uint8_t* sym);

}  // namespace lw
