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

}  // extern "C"

namespace {
// An open bundle directory: weights.bin is written as tensors arrive, each blob at the next 256-byte boundary; the
// manifest text (cfg lines first, then one t line per tensor in write order) is kept in memory and written by
// finish(). A refused name or key writes nothing and is reported by the call; an I/O error sticks, and finish() then
// reports failure.
// The directory and any missing parents (the reference Writer's os.makedirs(path, exist_ok=True),
// lazyweights/bundle.py:114-120); a failure shows as weights.bin failing to open.
void make_dirs(const std::string& dir) {
  for (size_t i = 1; i <= dir.size(); ++i)
    if (i == dir.size() || dir[i] == '/') mkdir(dir.substr(0, i).c_str(), 0755);
}

class BundleWriter {
 public:
  explicit BundleWriter(const std::string& dir) : dir_(dir) {
    make_dirs(dir);
    bin_ = fopen((dir + "/weights.bin").c_str(), "wb");
    ok_ = bin_ != nullptr;
  }
  ~BundleWriter() {
    if (bin_) fclose(bin_);
  }
  bool ok() const { return ok_; }
  static bool word(const char* w) { return w && *w && !strpbrk(w, " \t\n\r"); }
  bool cfg(const char* key, const char* value) {
    if (!word(key) || !word(value)) return false;
    cfg_ += std::string("cfg ") + key + " " + value + "\n";
    return true;
  }
  bool tensor(const char* name, const char* enc, long long N, long long K, double scale, int zp, const void* data,
              size_t n) {
    if (!ok_ || !word(name) || !word(enc) || (!data && n)) return false;
    static const uint8_t zeros[kAlign] = {0};
    const size_t gap = (size_t)((kAlign - at_ % kAlign) % kAlign);
    if (gap && fwrite(zeros, 1, gap, bin_) != gap) ok_ = false;
    at_ += gap;
    if (n && fwrite(data, 1, n, bin_) != n) ok_ = false;
    char line[640];
    snprintf(line, sizeof line, "t %s %s %lld %lld %.9g %d %llu %zu\n", name, enc, N, K, scale, zp,
             (unsigned long long)at_, n);
    t_ += line;
    at_ += n;
    return ok_;
  }
  bool finish() {
    if (bin_ && fclose(bin_) != 0) ok_ = false;
    bin_ = nullptr;
    if (!ok_) return false;
    FILE* m = fopen((dir_ + "/manifest.txt").c_str(), "w");
    if (!m) return false;
    const std::string text = cfg_ + t_;
    const bool wrote = fwrite(text.data(), 1, text.size(), m) == text.size();
    return (fclose(m) == 0) && wrote;
  }

 private:
  static constexpr size_t kAlign = 256;
  std::string dir_, cfg_, t_;
  FILE* bin_ = nullptr;
  uint64_t at_ = 0;
  bool ok_ = false;
};
}  // namespace

extern "C" {

void* lw_bundle_create(const char* dir) {
  if (!dir) return nullptr;
  auto* w = new BundleWriter(dir);
  if (!w->ok()) {
    delete w;
    return nullptr;
  }
  return w;
}

int lw_bundle_cfg(void* w, const char* key, const char* value) {
  if (!w) return -1;
  return static_cast<BundleWriter*>(w)->cfg(key, value) ? 0 : -1;
}

int lw_bundle_add(void* w, const char* name, const char* enc, long long N, long long K, double scale, int zp,
                  const void* data, long long nbytes) {
  if (!w || nbytes < 0) return -1;
  return static_cast<BundleWriter*>(w)->tensor(name, enc, N, K, scale, zp, data, (size_t)nbytes) ? 0 : -1;
}

int lw_bundle_finish(void* w) {
  if (!w) return -1;
  auto* b = static_cast<BundleWriter*>(w);
  const bool ok = b->finish();
  delete b;
  return ok ? 0 : -1;
}

int lw_write_bundle(const char* dir, int count, const char* const* names, const int* kqts, const int* Ns,
                    const int* Ks, const double* entropies, const uint64_t* seeds, int threads) {
  if (!dir || count < 1 || !names || !kqts || !Ns || !Ks || !entropies || !seeds) return -1;
  for (int i = 0; i < count; ++i)
    if (!names[i] || !shape_ok(kqts[i], Ns[i], Ks[i])) return -1;
  BundleWriter w(dir);
  if (!w.ok()) return -1;
  std::vector<uint8_t> codes, side, sym;
  for (int i = 0; i < count && w.ok(); ++i) {
    const int kqt = kqts[i], N = Ns[i], K = Ks[i], SB = lw::kq_sbytes(kqt);
    codes.resize((size_t)N * K);
    side.resize((size_t)N * (K / 256) * SB);
    lw::synth_matrix(kqt, N, K, entropies[i], seeds[i], codes.data(), side.data(), threads);
    const int KS = lw::kq_symbits(kqt) == 4 ? K / 2 : K;
    sym.resize((size_t)N * KS);
    lw::form_symbols(kqt, codes.data(), N, K, sym.data());
    lw::Encoded e;
    std::string err;
    if (!lw::encode_huf8(sym.data(), N, KS, threads, e, err)) return -1;
    if (!w.tensor(names[i], lw::kq_symbits(kqt) == 4 ? "huf4p" : "huf8", N, K, 1.0, 0, e.blob.data(), e.blob.size()) ||
        !w.tensor((std::string(names[i]) + ".kqs").c_str(), kq_name(kqt), N, (long long)(K / 256) * SB, 1.0, 0,
                  side.data(), side.size()))
      return -1;
  }
  return w.finish() ? 0 : -1;
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

int lw_canon_table(int kqt, const uint16_t* lut, uint32_t* out) {
  if (!lut || !out || kqt < 1 || kqt > 4) return -1;
  std::vector<uint32_t> entries(lw::LUTN);
  lw::decode_table4(kqt, lut, entries.data());
  return lw::canon_table(lut, entries.data(), out) ? 0 : -1;
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
