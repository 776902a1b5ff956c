// Host-side codec and synthetic bundle generation (see lw_codec.h).
#include "lw_codec.h"

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstring>
#include <functional>
#include <queue>
#include <thread>

namespace lw {

// ── Huffman tables ───────────────────────────────────────────────────────────────────────────────────────

void code_lengths(const int64_t* counts, int n, int* lens) {
  // Min-heap on (count, tie); tie = insertion counter: leaves first in ascending symbol order, then merged nodes.
  // A leaf's length is the number of merges it takes part in, i.e. its depth (lazyweights/huffman.py:8-26).
  struct Node {
    int64_t cnt, tie;
    int id;
  };
  struct Greater {
    bool operator()(const Node& a, const Node& b) const { return a.cnt != b.cnt ? a.cnt > b.cnt : a.tie > b.tie; }
  };
  for (int i = 0; i < n; ++i) lens[i] = 0;
  std::vector<int> syms;
  for (int i = 0; i < n; ++i)
    if (counts[i] > 0) syms.push_back(i);
  if (syms.empty()) return;
  if (syms.size() == 1) {
    lens[syms[0]] = 1;
    return;
  }
  std::priority_queue<Node, std::vector<Node>, Greater> heap;
  std::vector<int> parent(2 * syms.size(), -1);
  int64_t tie = 0;
  for (size_t i = 0; i < syms.size(); ++i) heap.push(Node{counts[syms[i]], tie++, (int)i});
  int next = (int)syms.size();
  while (heap.size() > 1) {
    const Node a = heap.top();
    heap.pop();
    const Node b = heap.top();
    heap.pop();
    parent[a.id] = parent[b.id] = next;
    heap.push(Node{a.cnt + b.cnt, tie++, next});
    ++next;
  }
  for (size_t i = 0; i < syms.size(); ++i) {
    int d = 0;
    for (int v = (int)i; parent[v] >= 0; v = parent[v]) ++d;
    lens[syms[i]] = d;
  }
}

void limited_lengths(const int64_t* counts, int n, int lmax, uint8_t* L) {
  std::vector<int64_t> cc(n);
  std::vector<int> len(n);
  int nz = 0;
  for (int i = 0; i < n; ++i) nz += counts[i] > 0;
  for (int k = 0;; ++k) {
    for (int i = 0; i < n; ++i) cc[i] = counts[i] > 0 ? std::max<int64_t>(1, k < 63 ? counts[i] >> k : 0) : 0;
    code_lengths(cc.data(), n, len.data());
    int mx = 0;
    for (int i = 0; i < n; ++i) mx = std::max(mx, len[i]);
    if (mx <= lmax) {
      for (int i = 0; i < n; ++i) L[i] = (uint8_t)(nz == 1 ? (counts[i] > 0 ? 1 : 0) : len[i]);
      return;
    }
  }
}

void canonical_codes(const uint8_t* L, int n, uint32_t* codes) {
  int mx = 0;
  for (int i = 0; i < n; ++i) mx = std::max(mx, (int)L[i]);
  uint32_t code = 0;
  for (int i = 0; i < n; ++i) codes[i] = 0;
  for (int l = 1; l <= mx; ++l) {
    for (int s = 0; s < n; ++s)
      if (L[s] == l) codes[s] = code++;
    code <<= 1;
  }
}

uint32_t bitrev(uint32_t v, int nbits) {
  uint32_t r = 0;
  for (int i = 0; i < nbits; ++i) r |= ((v >> i) & 1u) << (nbits - 1 - i);
  return r;
}

void build_lut(const uint8_t* L, uint16_t* lut) {
  uint32_t codes[256];
  canonical_codes(L, 256, codes);
  for (int i = 0; i < LUTN; ++i) lut[i] = 0;
  for (int s = 0; s < 256; ++s) {
    if (!L[s]) continue;
    const uint32_t rc = bitrev(codes[s], L[s]);
    for (uint32_t j = 0; j < (1u << (LMAX - L[s])); ++j) lut[rc + (j << L[s])] = (uint16_t)(s | L[s] << 8);
  }
}

// ── encoder ──────────────────────────────────────────────────────────────────────────────────────────────

static void run_threads(int threads, const std::function<void(int)>& f);

bool encode_huf8(const uint8_t* sym, int N, int KS, int threads, Encoded& out, std::string& err) {
  if (N <= 0 || KS <= 0 || N % TN || KS % TK) {
    err = "encode: N must be a multiple of 64 and symbols per row a multiple of 256";
    return false;
  }
  threads = std::max(1, threads);
  const int KT = KS / TK, NT = N / TN, T = NT * KT;
  // histogram
  std::vector<std::vector<int64_t>> hp(threads, std::vector<int64_t>(256, 0));
  run_threads(threads, [&](int id) {
    for (int r = id; r < N; r += threads) {
      const uint8_t* row = sym + (size_t)r * KS;
      int64_t* h = hp[id].data();
      for (int c = 0; c < KS; ++c) ++h[row[c]];
    }
  });
  int64_t hist[256] = {0};
  for (auto& h : hp)
    for (int i = 0; i < 256; ++i) hist[i] += h[i];
  uint8_t* L = out.lengths;
  limited_lengths(hist, 256, LMAX, L);
  uint32_t codes[256], rcode[256];
  canonical_codes(L, 256, codes);
  for (int s = 0; s < 256; ++s) rcode[s] = bitrev(codes[s], std::max<int>(L[s], 1));
  // bits per lane, in stream order (tile-major, lane-major)
  std::vector<uint64_t> lane_bits((size_t)T * LANES);
  run_threads(threads, [&](int id) {
    for (int t = id; t < T; t += threads) {
      const int tr = t / KT, tc = t - tr * KT;
      for (int l = 0; l < LANES; ++l) {
        uint64_t b = 0;
        for (int h = 0; h < 2; ++h) {
          const uint8_t* row = sym + (size_t)(tr * TN + h * 32 + l) * KS + (size_t)tc * TK;
          for (int c = 0; c < TK; ++c) b += L[row[c]];
        }
        lane_bits[(size_t)t * LANES + l] = b;
      }
    }
  });
  std::vector<uint64_t> start((size_t)T * LANES + 1);
  start[0] = 0;
  for (size_t i = 0; i < lane_bits.size(); ++i) start[i + 1] = start[i] + lane_bits[i];
  const uint64_t total = start.back();
  if (total >= (1ull << 32)) {
    err = "encode: payload exceeds 2^32 bits";
    return false;
  }
  out.payload_bits = total;
  const size_t nw = (size_t)((total + 31) / 32) + 2;
  out.blob.assign((size_t)2 * LUTN + (size_t)T * LANES * 4 + nw * 4, 0);
  uint16_t* lut = reinterpret_cast<uint16_t*>(out.blob.data());
  build_lut(L, lut);
  uint32_t* st = reinterpret_cast<uint32_t*>(out.blob.data() + 2 * LUTN);
  for (size_t i = 0; i < (size_t)T * LANES; ++i) st[i] = (uint32_t)start[i];
  uint32_t* words = st + (size_t)T * LANES;
  // Tiles are packed in parallel; words shared by neighbouring tiles are OR-ed atomically (bits are disjoint).
  run_threads(threads, [&](int id) {
    const int t0 = (int)((int64_t)T * id / threads), t1 = (int)((int64_t)T * (id + 1) / threads);
    for (int t = t0; t < t1; ++t) {
      const int tr = t / KT, tc = t - tr * KT;
      const uint64_t tb0 = start[(size_t)t * LANES], tb1 = start[(size_t)(t + 1) * LANES];
      uint64_t acc = 0;
      int nacc = 0;
      uint64_t wi = tb0 >> 5;
      // first partial word: pre-shift the accumulator
      nacc = (int)(tb0 & 31);
      for (int l = 0; l < LANES; ++l)
        for (int h = 0; h < 2; ++h) {
          const uint8_t* row = sym + (size_t)(tr * TN + h * 32 + l) * KS + (size_t)tc * TK;
          for (int c = 0; c < TK; ++c) {
            const uint8_t s = row[c];
            acc |= (uint64_t)rcode[s] << nacc;
            nacc += L[s];
            if (nacc >= 32) {
              const uint32_t v = (uint32_t)acc;
              if (wi == (tb0 >> 5) || wi == ((tb1 - 1) >> 5))
                __atomic_fetch_or(&words[wi], v, __ATOMIC_RELAXED);
              else
                words[wi] = v;
              ++wi;
              acc >>= 32;
              nacc -= 32;
            }
          }
        }
      if (nacc > 0 && tb1 > tb0) __atomic_fetch_or(&words[wi], (uint32_t)acc, __ATOMIC_RELAXED);
    }
  });
  return true;
}

// ── fp16 ─────────────────────────────────────────────────────────────────────────────────────────────────

uint16_t f32_to_f16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t ax = x & 0x7FFFFFFFu;
  if (ax >= 0x7F800000u) return (uint16_t)(sign | 0x7C00u | (ax > 0x7F800000u ? 0x200u : 0u));
  if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);  // rounds to inf
  if (ax < 0x38800000u) {  // subnormal half (or zero): round(m * 2^(e - 126)) to nearest even
    if (ax < 0x33000000u) return (uint16_t)sign;
    const int e = (int)(ax >> 23), sh = 126 - e;
    const uint32_t m = (ax & 0x7FFFFFu) | 0x800000u;
    const uint32_t mant = m >> sh, rem = m & ((1u << sh) - 1), half = 1u << (sh - 1);
    return (uint16_t)(sign | (mant + ((rem > half || (rem == half && (mant & 1))) ? 1u : 0u)));
  }
  const uint32_t e = ((ax >> 23) - 112) << 10;
  const uint32_t m = ax & 0x7FFFFFu;
  uint32_t h = e | (m >> 13);
  const uint32_t rem = m & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1))) ++h;
  return (uint16_t)(sign | h);
}

float f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 31, m = h & 1023;
  uint32_t x;
  if (e == 0) {
    if (m == 0) {
      x = sign;
    } else {
      float f = (float)m * 5.9604644775390625e-08f;  // 2^-24
      memcpy(&x, &f, 4);
      x |= sign;
    }
  } else if (e == 31) {
    x = sign | 0x7F800000u | (m << 13);
  } else {
    x = sign | ((e + 112) << 23) | (m << 13);
  }
  float f;
  memcpy(&f, &x, 4);
  return f;
}

// ── synthetic matrices ───────────────────────────────────────────────────────────────────────────────────

static inline uint64_t splitmix64(uint64_t& s) {
  uint64_t z = (s += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

struct Xoshiro {
  uint64_t s[4];
  explicit Xoshiro(uint64_t seed) {
    for (auto& v : s) v = splitmix64(seed);
  }
  static inline uint64_t rotl(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }
  inline uint64_t next() {
    const uint64_t r = rotl(s[1] * 5, 7) * 9, t = s[1] << 17;
    s[2] ^= s[0];
    s[3] ^= s[1];
    s[1] ^= s[2];
    s[0] ^= s[3];
    s[2] ^= t;
    s[3] = rotl(s[3], 45);
    return r;
  }
  inline double uniform() { return (double)(next() >> 11) * (1.0 / 9007199254740992.0); }
};

static double entropy_of(int n, int c, double rho, double* p) {
  double z = 0;
  for (int q = 0; q < n; ++q) z += p[q] = std::pow(rho, std::abs(q - c));
  double h = 0;
  for (int q = 0; q < n; ++q) {
    p[q] /= z;
    if (p[q] > 0) h -= p[q] * std::log2(p[q]);
  }
  return h;
}

void code_distribution(int ncodes, int centre, double entropy, double* p) {
  double lo = 1e-9, hi = 1.0;  // entropy grows with rho
  for (int it = 0; it < 200; ++it) {
    const double mid = 0.5 * (lo + hi);
    if (entropy_of(ncodes, centre, mid, p) < entropy) lo = mid;
    else hi = mid;
  }
  entropy_of(ncodes, centre, 0.5 * (lo + hi), p);
}

void synth_matrix(int kqt, int N, int K, double entropy, uint64_t seed, uint8_t* codes, uint8_t* side, int threads) {
  const int nc = kq_ncodes(kqt), centre = nc / 2, SB = kq_sbytes(kqt), NSB = K / 256;
  double p[64];
  code_distribution(nc, centre, entropy, p);
  // 2^16-entry inverse-CDF table
  std::vector<uint8_t> icdf(65536);
  {
    int q = 0;
    double edge = p[0];
    for (int u = 0; u < 65536; ++u) {
      const double x = (u + 0.5) / 65536.0;
      while (x > edge && q < nc - 1) {
        ++q;
        edge += p[q];
      }
      icdf[u] = (uint8_t)q;
    }
  }
  run_threads(std::max(1, threads), [&](int id) {
    for (int r = id; r < N; r += std::max(1, threads)) {
      uint64_t rs = seed ^ (0xD1B54A32D192ED03ull * (uint64_t)(r + 1));
      Xoshiro g(splitmix64(rs));
      uint8_t* cr = codes + (size_t)r * K;
      for (int k = 0; k < K; k += 4) {
        const uint64_t v = g.next();
        cr[k] = icdf[v & 0xFFFF];
        cr[k + 1] = icdf[(v >> 16) & 0xFFFF];
        cr[k + 2] = icdf[(v >> 32) & 0xFFFF];
        cr[k + 3] = icdf[(v >> 48) & 0xFFFF];
      }
      uint8_t* sr = side + (size_t)r * NSB * SB;
      for (int b = 0; b < NSB; ++b) {
        uint8_t* s = sr + (size_t)b * SB;
        const uint16_t d = f32_to_f16((float)(0.005 + 0.015 * g.uniform()));
        if (kqt == KQ_Q4_K || kqt == KQ_Q5_K) {
          const uint16_t dmin = f32_to_f16((float)(0.005 + 0.015 * g.uniform()));
          uint8_t sc[8], m[8];
          for (int j = 0; j < 8; ++j) {
            const uint64_t v = g.next();
            sc[j] = (uint8_t)(v & 63);
            m[j] = (uint8_t)((v >> 8) & 63);
          }
          // field packing of scripts/kq_quant.py:213-215 (llama.cpp Q4_K/Q5_K scales)
          memcpy(s, &d, 2);
          memcpy(s + 2, &dmin, 2);
          for (int j = 0; j < 4; ++j) {
            s[4 + j] = (uint8_t)(sc[j] | ((sc[4 + j] >> 4) << 6));
            s[8 + j] = (uint8_t)(m[j] | ((m[4 + j] >> 4) << 6));
            s[12 + j] = (uint8_t)((sc[4 + j] & 15) | ((m[4 + j] & 15) << 4));
          }
        } else if (kqt == KQ_Q6_K) {
          for (int j = 0; j < 16; ++j) s[j] = (uint8_t)(int8_t)((int)(g.next() % 255) - 127);
          memcpy(s + 16, &d, 2);
        } else {  // IQ4_XS: fp16 d, u16 high 2 bits of the 8 ls, 4 bytes of low nibbles (scripts/kq_quant.py:218-221)
          uint8_t ls[8];
          for (int j = 0; j < 8; ++j) ls[j] = (uint8_t)(g.next() & 63);
          uint16_t hi = 0;
          for (int j = 0; j < 8; ++j) hi |= (uint16_t)((ls[j] >> 4) << (2 * j));
          memcpy(s, &d, 2);
          memcpy(s + 2, &hi, 2);
          for (int j = 0; j < 4; ++j) s[4 + j] = (uint8_t)((ls[2 * j] & 15) | ((ls[2 * j + 1] & 15) << 4));
        }
      }
    }
  });
}

void form_symbols(int kqt, const uint8_t* codes, int N, int K, uint8_t* sym) {
  if (kq_symbits(kqt) == 8) {
    memcpy(sym, codes, (size_t)N * K);
    return;
  }
  const size_t n = (size_t)N * K / 2;
  for (size_t i = 0; i < n; ++i) sym[i] = (uint8_t)(codes[2 * i] | (codes[2 * i + 1] << 4));
}

static void run_threads(int threads, const std::function<void(int)>& f) {
  if (threads <= 1) {
    f(0);
    return;
  }
  std::vector<std::thread> th;
  for (int i = 0; i < threads; ++i) th.emplace_back(f, i);
  for (auto& t : th) t.join();
}

}  // namespace lw
