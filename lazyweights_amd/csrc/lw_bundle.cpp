// Synthetic K-quant matrices, blob encoding and bundle directories (C-ABI extensions; host only).
//
// Bundle directory format of lazyweights/bundle.py:10-21 and 114-136 (Writer): manifest.txt lines
// `t <name> <enc> <N> <K> <scale> <zp> <offset> <nbytes>`, every blob 256-byte aligned in weights.bin; K-quant side
// tensors `<name>.kqs` with enc kq_<type> and shape [N, K / 256 * SB] (scripts/a2_kq_bundle.py:216-218).
#include <sys/stat.h>

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/lazyweights_amd.h"
#include "lw_codec.h"
#include "lw_format.h"
#include "lw_layout.h"

namespace {
const char* kq_name(int kqt) {
  static const char* kn[] = {"", "kq_Q4_K", "kq_Q5_K", "kq_Q6_K", "kq_IQ4_XS"};
  return kqt >= 1 && kqt <= 4 ? kn[kqt] : nullptr;
}
bool shape_ok(int kqt, long long N, long long K) {
  return kq_name(kqt) && N > 0 && K > 0 && N % lw::TN == 0 && K % (lw::kq_symbits(kqt) == 4 ? 512 : 256) == 0;
}
}  // namespace

extern "C" {

int lw_synth_matrix(int kqt, int N, int K, double entropy, uint64_t seed, uint8_t* codes, uint8_t* side,
                    int threads) {
  if (!shape_ok(kqt, N, K) || !codes || !side || entropy <= 0) return -1;
  lw::synth_matrix(kqt, N, K, entropy, seed, codes, side, threads);
  return 0;
}

int lw_form_symbols(int kqt, const uint8_t* codes, int N, int K, uint8_t* sym) {
  if (!shape_ok(kqt, N, K) || !codes || !sym) return -1;
  lw::form_symbols(kqt, codes, N, K, sym);
  return 0;
}

long long lw_encode(const uint8_t* sym, int N, int KS, uint8_t* blob, long long cap, uint64_t* bits) {
  lw::Encoded e;
  std::string err;
  if (!sym || !lw::encode_huf8(sym, N, KS, 8, e, err)) return -1;
  if (bits) *bits = e.payload_bits;
  if (blob && cap >= (long long)e.blob.size()) memcpy(blob, e.blob.data(), e.blob.size());
  return (long long)e.blob.size();
}

int lw_write_bundle(const char* dir, int count, const char* const* names, const int* kqts, const int* Ns,
                    const int* Ks, const double* entropies, const uint64_t* seeds, int threads) {
  if (!dir || count < 1 || !names || !kqts || !Ns || !Ks || !entropies || !seeds) return -1;
  for (int i = 0; i < count; ++i)
    if (!names[i] || !shape_ok(kqts[i], Ns[i], Ks[i])) return -1;
  mkdir(dir, 0755);
  const std::string d(dir);
  FILE* w = fopen((d + "/weights.bin").c_str(), "wb");
  if (!w) return -1;
  std::string manifest;
  uint64_t off = 0;
  auto add = [&](const std::string& name, const char* enc, long long N, long long K, const uint8_t* p, size_t n) {
    static const uint8_t zeros[256] = {0};
    const size_t pad = (size_t)((256 - off % 256) % 256);
    if (pad) fwrite(zeros, 1, pad, w);
    off += pad;
    fwrite(p, 1, n, w);
    char line[512];
    snprintf(line, sizeof line, "t %s %s %lld %lld %.9g %d %llu %zu\n", name.c_str(), enc, N, K, 1.0, 0,
             (unsigned long long)off, n);
    manifest += line;
    off += n;
  };
  std::vector<uint8_t> codes, side, sym;
  for (int i = 0; i < count; ++i) {
    const int kqt = kqts[i], N = Ns[i], K = Ks[i], SB = lw::kq_sbytes(kqt);
    codes.resize((size_t)N * K);
    side.resize((size_t)N * (K / 256) * SB);
    lw::synth_matrix(kqt, N, K, entropies[i], seeds[i], codes.data(), side.data(), threads);
    const int KS = lw::kq_symbits(kqt) == 4 ? K / 2 : K;
    sym.resize((size_t)N * KS);
    lw::form_symbols(kqt, codes.data(), N, K, sym.data());
    lw::Encoded e;
    std::string err;
    if (!lw::encode_huf8(sym.data(), N, KS, threads, e, err)) {
      fclose(w);
      return -1;
    }
    add(names[i], lw::kq_symbits(kqt) == 4 ? "huf4p" : "huf8", N, K, e.blob.data(), e.blob.size());
    add(std::string(names[i]) + ".kqs", kq_name(kqt), N, (long long)(K / 256) * SB, side.data(), side.size());
  }
  const bool ok = fclose(w) == 0;
  FILE* m = fopen((d + "/manifest.txt").c_str(), "w");
  if (!m) return -1;
  fwrite(manifest.data(), 1, manifest.size(), m);
  return (fclose(m) == 0 && ok) ? 0 : -1;
}

int lw_huffman_lengths(const int64_t* hist, int n, int lmax, uint8_t* L) {
  if (!hist || !L || n < 1 || n > 256) return -1;
  if (lmax > 0) {
    lw::limited_lengths(hist, n, lmax, L);
  } else {
    std::vector<int> len(n);
    lw::code_lengths(hist, n, len.data());
    for (int i = 0; i < n; ++i) L[i] = (uint8_t)std::min(255, len[i]);
  }
  return 0;
}

long long lw_build_layout(const uint8_t* blob, long long len, int N, int KS, int pre_il, int compact, uint32_t* tbase,
                          uint16_t* mid, uint16_t* split, uint16_t* rows, uint64_t* sched, int* ring_rows,
                          uint32_t* words, long long words_cap) {
  if (!blob || len <= 0) return -1;
  lw::Layout L;
  std::string err;
  const bool ok = pre_il ? lw::build_layout_il(blob, (size_t)len, N, KS, compact != 0, lw::default_threads(), L, err)
                         : lw::build_layout_raw(blob, (size_t)len, N, KS, lw::default_threads(), L, err);
  if (!ok) return -1;
  const size_t T = L.tbase.size();
  if (tbase) memcpy(tbase, L.tbase.data(), 4 * T);
  if (mid) memcpy(mid, L.mid.data(), 2 * L.mid.size());
  if (split) memcpy(split, L.split.data(), 2 * L.split.size());
  if (rows) memcpy(rows, L.rows.data(), 2 * T);
  if (sched) memcpy(sched, L.sched.data(), 16 * T);
  if (ring_rows) *ring_rows = L.ring_rows;
  if (words && words_cap >= (long long)L.words.size()) memcpy(words, L.words.data(), 4 * L.words.size());
  return (long long)L.words.size();
}

}  // extern "C"
