// Load-time layout transforms and CPU decode (see lw_layout.h).
#include "lw_layout.h"

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cstring>
#include <functional>
#include <mutex>
#include <thread>

#include "lw_format.h"

namespace lw {

int default_threads() {
  const unsigned n = std::thread::hardware_concurrency();
  return (int)std::max(1u, std::min(n ? n : 1u, 16u));
}

static void parallel_for(int n, int threads, const std::function<void(int, int)>& f) {
  threads = std::max(1, std::min(threads, n));
  if (threads <= 1) {
    f(0, n);
    return;
  }
  std::vector<std::thread> th;
  for (int i = 0; i < threads; ++i) {
    const int a = (int)((int64_t)n * i / threads), b = (int)((int64_t)n * (i + 1) / threads);
    th.emplace_back(f, a, b);
  }
  for (auto& t : th) t.join();
}

namespace {

// A lane's bit stream: `nw` words starting at a word-aligned position, read through `word(i)`.
template <class W>
inline bool decode_lane(const uint16_t* lut, W word, uint64_t nw, uint64_t start, uint32_t& mid, uint64_t& end) {
  uint64_t bp = start;
  for (int i = 0; i < LANE_SYMS; ++i) {
    if (i == TK) mid = (uint32_t)(bp - start);
    const uint64_t wi = bp >> 5;
    if (wi >= nw) return false;
    const uint64_t lo = word(wi), hi = wi + 1 < nw ? word(wi + 1) : 0;
    const uint16_t e = lut[((lo | (hi << 32)) >> (bp & 31)) & (LUTN - 1)];
    bp += e >> 8;
  }
  end = bp;
  return true;
}

inline uint32_t bits_at(const uint32_t* pay, uint64_t pw, uint64_t b) {
  const uint64_t wi = b >> 5;
  const uint64_t lo = wi < pw ? pay[wi] : 0, hi = wi + 1 < pw ? pay[wi + 1] : 0;
  return (uint32_t)((lo | (hi << 32)) >> (b & 31));
}

// Fill tile rows from per-lane word sources once lane lengths are known.
void finish_layout(Layout& L, int T, const std::vector<uint64_t>& lane_bits,
                   const std::function<uint32_t(int, int, uint32_t)>& lane_word, int threads) {
  L.rows.assign(T, 0);
  L.tbase.assign(T, 0);
  L.max_rows = 0;
  uint64_t total = 0, nwords = 0;
  for (int t = 0; t < T; ++t) {
    uint32_t r = 0;
    for (int l = 0; l < LANES; ++l) {
      const uint64_t b = lane_bits[(size_t)t * LANES + l];
      total += b;
      r = std::max<uint32_t>(r, (uint32_t)((b + 31) / 32));
    }
    L.rows[t] = (uint16_t)r;
    L.tbase[t] = (uint32_t)nwords;
    nwords += (uint64_t)32 * r;
    L.max_rows = std::max<int>(L.max_rows, (int)r);
  }
  L.payload_bits = total;
  L.words.assign(nwords + (uint64_t)32 * TAIL_ROWS, 0);
  parallel_for(T, threads, [&](int t0, int t1) {
    for (int t = t0; t < t1; ++t)
      for (int l = 0; l < LANES; ++l) {
        const uint64_t nb = lane_bits[(size_t)t * LANES + l];
        uint32_t* o = L.words.data() + L.tbase[t] + l;
        for (uint32_t i = 0; (uint64_t)i * 32 < nb; ++i) {
          uint32_t v = lane_word(t, l, i);
          const uint64_t left = nb - (uint64_t)i * 32;
          if (left < 32) v &= (1u << left) - 1;
          o[(size_t)32 * i] = v;
        }
      }
  });
}

}  // namespace

bool build_layout_raw(const uint8_t* blob, size_t len, int N, int KS, int threads, Layout& L, std::string& err) {
  if (N <= 0 || KS <= 0 || N % TN || KS % TK) {
    err = "coded matrix: rows must be a multiple of 64 and symbols per row a multiple of 256";
    return false;
  }
  const int T = (N / TN) * (KS / TK);
  const size_t hdr = (size_t)2 * LUTN + (size_t)T * LANES * 4;
  if (len < hdr + 8) {
    err = "coded matrix: blob shorter than its header";
    return false;
  }
  memcpy(L.lut, blob, sizeof L.lut);
  const uint32_t* starts = reinterpret_cast<const uint32_t*>(blob + 2 * LUTN);
  const uint32_t* pay = starts + (size_t)T * LANES;
  const uint64_t pw = (len - hdr) / 4;
  for (size_t i = 0; i + 1 < (size_t)T * LANES; ++i)
    if (starts[i] > starts[i + 1]) {
      err = "coded matrix: lane starts not increasing";
      return false;
    }
  L.mid.assign((size_t)T * LANES, 0);
  std::vector<uint64_t> lane_bits((size_t)T * LANES);
  std::atomic<bool> bad(false);
  parallel_for(T, threads, [&](int t0, int t1) {
    for (int t = t0; t < t1 && !bad; ++t)
      for (int l = 0; l < LANES; ++l) {
        const size_t i = (size_t)t * LANES + l;
        uint32_t mid = 0;
        uint64_t end = 0;
        if (!decode_lane(L.lut, [&](uint64_t w) { return (uint64_t)pay[w]; }, pw, starts[i], mid, end)) {
          bad = true;
          break;
        }
        // a lane ends where the next one starts; the last lane of the matrix before the 2 tail words
        const uint64_t next = i + 1 < (size_t)T * LANES ? starts[i + 1] : (pw >= 2 ? (pw - 2) * 32 : 0);
        if (i + 1 < (size_t)T * LANES ? end != next : end > next) {
          bad = true;
          break;
        }
        L.mid[i] = (uint16_t)mid;
        lane_bits[i] = end - starts[i];
      }
  });
  if (bad) {
    err = "coded matrix: lane streams inconsistent with the lane starts (corrupt or truncated blob)";
    return false;
  }
  finish_layout(L, T, lane_bits,
                [&](int t, int l, uint32_t i) { return bits_at(pay, pw, starts[(size_t)t * LANES + l] + 32ull * i); },
                threads);
  return true;
}

bool build_layout_il(const uint8_t* data, size_t len, int N, int KS, bool compact, int threads, Layout& L,
                     std::string& err) {
  if (N <= 0 || KS <= 0 || N % TN || KS % TK) {
    err = "coded matrix: rows must be a multiple of 64 and symbols per row a multiple of 256";
    return false;
  }
  const int T = (N / TN) * (KS / TK);
  const size_t hw = (size_t)LUTN / 2 + T + ((T + 1) & ~1) / 2 + (size_t)T * 16;  // header words
  if (len % 4 || len / 4 < hw) {
    err = "pre-interleaved matrix: shorter than its header";
    return false;
  }
  const uint32_t* u = reinterpret_cast<const uint32_t*>(data);
  memcpy(L.lut, data, sizeof L.lut);
  const uint32_t* tb = u + LUTN / 2;
  const uint16_t* wc = reinterpret_cast<const uint16_t*>(tb + T);
  const uint16_t* ovf = wc + ((T + 1) & ~1);
  const uint32_t* words = u + hw;
  const uint64_t nwt = len / 4 - hw;
  // lane word i of (t, l): interleaved part, then (compact) the lane's overflow run
  auto lane_avail = [&](int t, int l) -> uint64_t {
    if (!compact) return wc[t];
    const uint64_t run_end = l < 31 ? ovf[(size_t)t * 32 + l + 1]
                                    : (t + 1 < T ? (uint64_t)tb[t + 1] - tb[t] - 32ull * wc[t]
                                                 : nwt - tb[t] - 32ull * wc[t]);
    return (uint64_t)wc[t] + (run_end - ovf[(size_t)t * 32 + l]);
  };
  auto lane_word = [&](int t, int l, uint64_t i) -> uint32_t {
    const uint64_t idx = i < wc[t] ? (uint64_t)tb[t] + 32ull * i + l
                                   : (uint64_t)tb[t] + 32ull * wc[t] + ovf[(size_t)t * 32 + l] + (i - wc[t]);
    return idx < nwt ? words[idx] : 0u;
  };
  for (int t = 0; t < T; ++t)
    if ((uint64_t)tb[t] + 32ull * wc[t] > nwt) {
      err = "pre-interleaved matrix: tile beyond the data";
      return false;
    }
  L.mid.assign((size_t)T * LANES, 0);
  std::vector<uint64_t> lane_bits((size_t)T * LANES);
  std::atomic<bool> bad(false);
  parallel_for(T, threads, [&](int t0, int t1) {
    for (int t = t0; t < t1 && !bad; ++t)
      for (int l = 0; l < LANES; ++l) {
        const uint64_t nw = lane_avail(t, l);
        uint32_t mid = 0;
        uint64_t end = 0;
        if (nw > 4096 || !decode_lane(L.lut, [&](uint64_t w) { return (uint64_t)lane_word(t, l, w); }, nw + 1, 0,
                                      mid, end) ||
            end > 32 * nw) {
          bad = true;
          break;
        }
        L.mid[(size_t)t * LANES + l] = (uint16_t)mid;
        lane_bits[(size_t)t * LANES + l] = end;
      }
  });
  if (bad) {
    err = "pre-interleaved matrix: lane streams inconsistent with the layout (corrupt export)";
    return false;
  }
  finish_layout(L, T, lane_bits, [&](int t, int l, uint32_t i) { return lane_word(t, l, i); }, threads);
  return true;
}

double cpu_decode(const uint8_t* blob, int N, int KS, int threads, uint8_t* out) {
  const int KT = KS / TK, T = (N / TN) * KT;
  const uint16_t* lut = reinterpret_cast<const uint16_t*>(blob);
  const uint32_t* starts = reinterpret_cast<const uint32_t*>(blob + 2 * LUTN);
  const uint8_t* payload = reinterpret_cast<const uint8_t*>(starts + (size_t)T * LANES);
  threads = std::max(1, threads);
  auto work = [&](int tid) {
    for (int tt = tid; tt < T; tt += threads) {
      const int tr = tt / KT, tc = tt - tr * KT;
      for (int lane = 0; lane < LANES; ++lane) {
        uint64_t bp = starts[(size_t)tt * LANES + lane];
        for (int half = 0; half < 2; ++half) {
          uint8_t* row = out + (size_t)(tr * TN + half * 32 + lane) * KS + (size_t)tc * TK;
          for (int c = 0; c < TK; ++c) {
            uint64_t w;
            memcpy(&w, payload + ((bp >> 5) << 2), 8);
            const uint16_t e = lut[(w >> (bp & 31)) & (LUTN - 1)];
            row[c] = (uint8_t)e;
            bp += e >> 8;
          }
        }
      }
    }
  };
  const auto t0 = std::chrono::steady_clock::now();
  std::vector<std::thread> th;
  for (int i = 1; i < threads; ++i) th.emplace_back(work, i);
  work(0);
  for (auto& x : th) x.join();
  return std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
}

}  // namespace lw
