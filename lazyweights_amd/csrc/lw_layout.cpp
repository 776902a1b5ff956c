// Load-time layout transforms and CPU decode (see lw_layout.h).
#include "lw_layout.h"

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cstring>
#include <functional>
#include <mutex>
#include <thread>

#include "lw_codec.h"
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

// Decode one lane (512 symbols) from a bit source: bits32(off) = 32 stream bits from lane offset `off`.
// pos[i] = lane bit offset before symbol i (i = 0..512). Fails if the lane runs past `limit` bits.
template <class B>
inline bool decode_lane(const uint16_t* lut, B bits32, uint64_t limit, uint32_t* pos) {
  uint64_t bp = 0;
  for (int i = 0; i < LANE_SYMS; ++i) {
    pos[i] = (uint32_t)bp;
    if (bp >= limit) return false;
    const uint16_t e = lut[bits32(bp) & (LUTN - 1)];
    bp += e >> 8;
  }
  pos[LANE_SYMS] = (uint32_t)bp;
  return bp <= limit;
}

inline uint32_t bits_at(const uint32_t* pay, uint64_t pw, uint64_t b) {
  const uint64_t wi = b >> 5;
  const uint64_t lo = wi < pw ? pay[wi] : 0, hi = wi + 1 < pw ? pay[wi + 1] : 0;
  return (uint32_t)((lo | (hi << 32)) >> (b & 31));
}

// Ring staging schedule of one tile (see the ring kernel): each front stages CHUNK_ROWS-row chunks of its rows,
// relative to its base row; chunks loaded at group g reach LDS at the start of group g + 2. mn / mx = lowest /
// highest relative row that any lane of front f reads from the ring in each group; r0 = lowest row of the windows
// read before group 0. The schedule is the same for both fronts (one chunk count per group and one initial count),
// so the kernel's staging is wave-uniform: loads are issued just in time for the front that needs them first (at
// most MAX_CHUNKS_PER_GROUP per group). Returns false if a ring of RS rows cannot hold it for either front.
bool ring_schedule_shared(const int mn[2][GROUPS], const int mx[2][GROUPS], const int r0[2], int RS, uint64_t& counts,
                          int init[2]) {
  counts = 0;
  int in = 0;
  for (int f = 0; f < 2; ++f) in = std::max(in, (std::max(mx[f][0], mx[f][1]) + CHUNK_ROWS) / CHUNK_ROWS);
  if (in > 255) return false;
  for (int f = 0; f < 2; ++f)
    if (CHUNK_ROWS * in > RS + r0[f]) return false;
  int issued = in, written = in;
  int loads[GROUPS] = {0};
  for (int g = 0; g < GROUPS; ++g) {
    if (g >= 2) written += loads[g - 2];
    for (int f = 0; f < 2; ++f)
      if (mx[f][g] > CHUNK_ROWS * written - 1 || mn[f][g] < CHUNK_ROWS * written - RS) return false;
    const int gt = std::min(g + 2, GROUPS - 1);
    const int target = std::max(mx[0][gt], mx[1][gt]);
    while (CHUNK_ROWS * issued <= target && g + 2 < GROUPS && loads[g] < MAX_CHUNKS_PER_GROUP) {
      ++loads[g];
      ++issued;
    }
    counts |= (uint64_t)loads[g] << (2 * g);
  }
  counts |= counts << 32;  // the same counts for front 1 (bits 32 + 2g)
  init[0] = init[1] = in;
  return true;
}

// The same with one schedule per front (per-lane counts in the kernel): each front's loads are issued just in time
// for its own rows. Used for tiles the shared schedule cannot hold.
bool ring_schedule_fronts(const int mn[2][GROUPS], const int mx[2][GROUPS], const int r0[2], int RS,
                          uint64_t& counts, int init[2]) {
  counts = 0;
  for (int f = 0; f < 2; ++f) {
    init[f] = (std::max(mx[f][0], mx[f][1]) + CHUNK_ROWS) / CHUNK_ROWS;
    if (CHUNK_ROWS * init[f] > RS + r0[f] || init[f] > 255) return false;
    int issued = init[f], written = init[f];
    int loads[GROUPS] = {0};
    for (int g = 0; g < GROUPS; ++g) {
      if (g >= 2) written += loads[g - 2];
      if (mx[f][g] > CHUNK_ROWS * written - 1 || mn[f][g] < CHUNK_ROWS * written - RS) return false;
      const int target = mx[f][std::min(g + 2, GROUPS - 1)];
      while (CHUNK_ROWS * issued <= target && g + 2 < GROUPS && loads[g] < MAX_CHUNKS_PER_GROUP) {
        ++loads[g];
        ++issued;
      }
      counts |= (uint64_t)loads[g] << (32 * f + 2 * g);
    }
  }
  return true;
}

// Per-tile load-time analysis shared by both input formats: lane positions -> mid offsets, lane lengths and the
// ring schedule. `bits32(t, l, off)` reads the lane stream; `limit(t, l)` bounds its length.
template <class B, class Lim, class Check>
bool analyse_tiles(Layout& L, int T, int threads, B bits32, Lim limit, Check check_end,
                   std::vector<uint64_t>& lane_bits) {
  L.mid.assign((size_t)T * LANES, 0);
  L.split.assign((size_t)T * SPLITS * LANES, 0);
  L.sched.assign(2 * (size_t)T, 0);
  lane_bits.assign((size_t)T * LANES, 0);
  std::vector<uint8_t> ring_ok(T, 0);  // bit 0: RS 16 fits, bit 1: RS 32 fits
  std::atomic<bool> bad(false);
  parallel_for(T, threads, [&](int t0, int t1) {
    std::vector<uint32_t> pos((size_t)LANES * (LANE_SYMS + 1));
    for (int t = t0; t < t1 && !bad; ++t) {
      for (int l = 0; l < LANES; ++l) {
        uint32_t* p = pos.data() + (size_t)l * (LANE_SYMS + 1);
        if (!decode_lane(L.lut, [&](uint64_t off) { return bits32(t, l, off); }, limit(t, l), p) ||
            !check_end(t, l, p[LANE_SYMS])) {
          bad = true;
          break;
        }
        L.mid[(size_t)t * LANES + l] = (uint16_t)(p[TK] + GUARD);
        for (int k = 0; k < SPLITS; ++k)
          L.split[((size_t)t * SPLITS + k) * LANES + l] = (uint16_t)(p[k * (LANE_SYMS / SPLITS)] + GUARD);
        lane_bits[(size_t)t * LANES + l] = p[LANE_SYMS];
      }
      if (bad) break;
      int base1 = 1 << 30;
      for (int l = 0; l < LANES; ++l) base1 = std::min<int>(base1, (int)(pos[(size_t)l * (LANE_SYMS + 1) + TK] >> 5));
      // The kernel reads rows r, r + 1, r + 2 of the window at a front's first symbol (r = its row), then, after
      // each pair of symbols, row r + 2 of the window at the next pair: in group g (pairs at s0, s0 + 2, ..,
      // s0 + 14) that is rows row(s0 + 2) + 2 .. row(s0 + 16) + 2.
      int mn[2][GROUPS], mx[2][GROUPS], r0[2];
      for (int f = 0; f < 2; ++f) {
        const int base = f ? base1 : 0;
        r0[f] = 1 << 30;
        for (int l = 0; l < LANES; ++l)
          r0[f] = std::min<int>(r0[f], (int)(pos[(size_t)l * (LANE_SYMS + 1) + f * TK] >> 5) - base);
        for (int g = 0; g < GROUPS; ++g) {
          const int s0 = f * TK + g * GROUP_SYMS;
          int lo = 1 << 30, hi = 0;
          for (int l = 0; l < LANES; ++l) {
            const uint32_t* p = pos.data() + (size_t)l * (LANE_SYMS + 1);
            lo = std::min<int>(lo, (int)(p[s0 + 2] >> 5) + 2 - base);
            hi = std::max<int>(hi, (int)(p[s0 + GROUP_SYMS] >> 5) + 2 - base);
          }
          mn[f][g] = lo;
          mx[f][g] = hi;
        }
      }
      // Preferably both fronts share one schedule (front 1 may then start its staging up to 4 rows below its first
      // needed row, base1 - d, to align the two fronts' progress; the first shift that fits is taken), else each
      // front gets its own.
      int init[2] = {0, 0}, base_used = base1;
      uint64_t counts = 0;
      uint8_t ok = 0;
      for (int k = 1; k >= 0; --k) {  // a schedule valid for 16 rows is valid for 32 (same loads, looser checks)
        bool found = false;
        for (int d = 0; d <= 4 && d <= base1 && !found; ++d) {
          int mn1[2][GROUPS], mx1[2][GROUPS], r01[2] = {r0[0], r0[1] + d};
          for (int g = 0; g < GROUPS; ++g) {
            mn1[0][g] = mn[0][g];
            mx1[0][g] = mx[0][g];
            mn1[1][g] = mn[1][g] + d;
            mx1[1][g] = mx[1][g] + d;
          }
          uint64_t c;
          int in[2];
          if (base1 - d < 256 && ring_schedule_shared(mn1, mx1, r01, k ? 32 : 16, c, in)) {
            ok |= (uint8_t)(1 << k);
            counts = c;
            init[0] = in[0];
            init[1] = in[1];
            base_used = base1 - d;
            found = true;
          }
        }
        uint64_t c;
        int in[2];
        if (!found && base1 < 256 && ring_schedule_fronts(mn, mx, r0, k ? 32 : 16, c, in)) {
          ok |= (uint8_t)(1 << k);
          counts = c;
          init[0] = in[0];
          init[1] = in[1];
          base_used = base1;
        }
      }
      ring_ok[t] = ok;
      if (ok) {
        L.sched[2 * (size_t)t] = counts;
        L.sched[2 * (size_t)t + 1] = (uint64_t)base_used | (uint64_t)init[0] << 8 | (uint64_t)init[1] << 16;
      }
    }
  });
  if (bad) return false;
  // one ring size per matrix: 16 rows when at most 1/32 of the tiles need the whole-tile fallback, else 32 if
  // every tile fits, else none (whole-tile kernel for the matrix)
  int n16 = 0;
  bool all32 = true;
  for (int t = 0; t < T; ++t) {
    n16 += ring_ok[t] & 1;
    all32 = all32 && (ring_ok[t] & 2);
  }
  L.exc.clear();
  L.nexc32 = 0;
  if (32 * (T - n16) <= T) {
    L.ring_rows = 16;
    for (int pass = 0; pass < 2; ++pass)  // exception tiles with a 32-row schedule first
      for (int t = 0; t < T; ++t)
        if (!(ring_ok[t] & 1) && (pass == 0) == ((ring_ok[t] & 2) != 0)) {
          L.exc.push_back((uint32_t)t);
          L.sched[2 * (size_t)t + 1] |= (pass == 0 ? 3ull : 1ull) << 32;  // bit 33: has a 32-row schedule
          L.nexc32 += pass == 0;
        }
  } else {
    L.ring_rows = all32 ? 32 : 0;
  }
  return true;
}

// Fill tile rows from per-lane bit sources once lane lengths are known. Device lane streams carry GUARD leading
// zero bits; word i of a lane holds its stream bits [32 i - GUARD, 32 i + 32 - GUARD).
template <class B>
void finish_layout(Layout& L, int T, const std::vector<uint64_t>& lane_bits, B bits32, int threads) {
  L.rows.assign(T, 0);
  L.tbase.assign(T, 0);
  L.hrow.assign(T, 0);
  L.max_rows = 0;
  L.max_hrows = 0;
  uint64_t total = 0, nwords = 0;
  for (int t = 0; t < T; ++t) {
    uint32_t r = 0;
    for (int l = 0; l < LANES; ++l) {
      const uint64_t b = lane_bits[(size_t)t * LANES + l];
      total += b;
      r = std::max<uint32_t>(r, (uint32_t)((b + GUARD + 31) / 32));
    }
    L.rows[t] = (uint16_t)r;
    nwords += (uint64_t)32 * r;
    L.max_rows = std::max<int>(L.max_rows, (int)r);
    // half-tile units: the first rows' bits end before each lane's mid (device bits, guard included); the second
    // rows' windows start at the row of mid - 2
    uint32_t r1 = 0, r0 = 1u << 30;
    for (int l = 0; l < LANES; ++l) {
      const uint32_t m = L.mid[(size_t)t * LANES + l];
      r1 = std::max<uint32_t>(r1, ((m - 1) >> 5) + 1);
      r0 = std::min<uint32_t>(r0, (m - 2) >> 5);
    }
    L.hrow[t] = r1 | r0 << 16;
    L.max_hrows = std::max<int>(L.max_hrows, (int)std::max<uint32_t>(r1, r - r0));
  }
  L.payload_bits = total;
  // Tiles at a fixed stride of max_rows word rows when that pads the words by at most 1/8: a tile's place is then
  // known without reading tbase (the whole-tile kernels' first copies); else back to back.
  L.tstride = (uint64_t)T * L.max_rows * 32 <= nwords + nwords / 8 ? L.max_rows : 0;
  if (L.tstride) nwords = (uint64_t)T * L.max_rows * 32;
  for (uint64_t t = 0, o = 0; t < (uint64_t)T; ++t) {
    L.tbase[t] = (uint32_t)(L.tstride ? 32 * L.tstride * t : o);
    o += (uint64_t)32 * L.rows[t];
  }
  L.words.assign(nwords + (uint64_t)32 * TAIL_ROWS, 0);
  parallel_for(T, threads, [&](int t0, int t1) {
    for (int t = t0; t < t1; ++t)
      for (int l = 0; l < LANES; ++l) {
        const uint64_t nb = lane_bits[(size_t)t * LANES + l] + GUARD;
        uint32_t* o = L.words.data() + L.tbase[t] + l;
        for (uint32_t i = 0; (uint64_t)i * 32 < nb; ++i) {
          uint32_t v = i == 0 ? bits32(t, l, 0) << GUARD : bits32(t, l, 32ull * i - GUARD);
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
  const uint64_t nlanes = (uint64_t)T * LANES;
  for (size_t i = 0; i + 1 < nlanes; ++i)
    if (starts[i] > starts[i + 1]) {
      err = "coded matrix: lane starts not increasing";
      return false;
    }
  if (pw < 2 || starts[nlanes - 1] > (pw - 2) * 32) {
    err = "coded matrix: lane starts beyond the payload";
    return false;
  }
  auto st = [&](int t, int l) { return (uint64_t)starts[(size_t)t * LANES + l]; };
  auto bits32 = [&](int t, int l, uint64_t off) { return bits_at(pay, pw, st(t, l) + off); };
  // a lane ends where the next one starts; the last lane of the matrix before the 2 tail words
  auto next = [&](int t, int l) {
    const size_t i = (size_t)t * LANES + l;
    return i + 1 < nlanes ? (uint64_t)starts[i + 1] : (pw - 2) * 32;
  };
  auto limit = [&](int t, int l) { return next(t, l) - st(t, l); };
  auto check_end = [&](int t, int l, uint64_t end) {
    const size_t i = (size_t)t * LANES + l;
    return i + 1 < nlanes ? end == limit(t, l) : end <= limit(t, l);
  };
  std::vector<uint64_t> lane_bits;
  if (!analyse_tiles(L, T, threads, bits32, limit, check_end, lane_bits)) {
    err = "coded matrix: lane streams inconsistent with the lane starts (corrupt or truncated blob)";
    return false;
  }
  finish_layout(L, T, lane_bits, bits32, threads);
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
  for (int t = 0; t < T; ++t)
    if ((uint64_t)tb[t] + 32ull * wc[t] > nwt || (t + 1 < T && tb[t + 1] < tb[t])) {
      err = "pre-interleaved matrix: tile beyond the data";
      return false;
    }
  // lane word i of (t, l): interleaved part, then (compact) the lane's overflow run
  auto lane_avail = [&](int t, int l) -> uint64_t {
    if (!compact) return wc[t];
    const uint64_t tile_end = t + 1 < T ? (uint64_t)tb[t + 1] : nwt;
    const uint64_t run0 = (uint64_t)tb[t] + 32ull * wc[t] + ovf[(size_t)t * 32 + l];
    const uint64_t run1 = l < 31 ? (uint64_t)tb[t] + 32ull * wc[t] + ovf[(size_t)t * 32 + l + 1] : tile_end;
    return (uint64_t)wc[t] + (run1 > run0 ? std::min(run1, tile_end) - run0 : 0);
  };
  auto lane_word = [&](int t, int l, uint64_t i) -> uint32_t {
    if (i >= lane_avail(t, l)) return 0u;
    const uint64_t idx = i < wc[t] ? (uint64_t)tb[t] + 32ull * i + l
                                   : (uint64_t)tb[t] + 32ull * wc[t] + ovf[(size_t)t * 32 + l] + (i - wc[t]);
    return idx < nwt ? words[idx] : 0u;
  };
  auto bits32 = [&](int t, int l, uint64_t off) {
    const uint64_t w = off >> 5;
    return (uint32_t)((((uint64_t)lane_word(t, l, w + 1) << 32) | lane_word(t, l, w)) >> (off & 31));
  };
  auto limit = [&](int t, int l) { return 32 * std::min<uint64_t>(lane_avail(t, l), 4096); };
  auto check_end = [&](int, int, uint64_t) { return true; };
  std::vector<uint64_t> lane_bits;
  if (!analyse_tiles(L, T, threads, bits32, limit, check_end, lane_bits)) {
    err = "pre-interleaved matrix: lane streams inconsistent with the layout (corrupt export)";
    return false;
  }
  finish_layout(L, T, lane_bits, bits32, threads);
  return true;
}

// One lane stream of a raw blob as a bit source: a 64-bit buffer topped up a word at a time from the payload, so
// each symbol costs one table lookup and one shift; words past the payload's end read as zero.
struct LaneBits {
  const uint32_t* pay;
  uint64_t nwords, next;  // payload words, next word to load
  uint64_t buf = 0;       // unread bits, LSB first
  int have = 0;           // valid bits in buf
  LaneBits(const uint32_t* p, uint64_t n, uint64_t bit) : pay(p), nwords(n), next(bit >> 5) {
    fill();
    const int skip = (int)(bit & 31);
    buf >>= skip;
    have -= skip;
  }
  void fill() {
    while (have <= 32) {
      const uint64_t w = next < nwords ? pay[next] : 0u;
      ++next;
      buf |= w << have;
      have += 32;
    }
  }
  uint32_t peek() const { return (uint32_t)buf; }
  void drop(int n) {
    buf >>= n;
    have -= n;
    if (have <= 32) fill();
  }
};

bool cpu_decode(const uint8_t* blob, size_t nbytes, int N, int KS, int threads, uint8_t* out, double* seconds,
                std::string& err) {
  if (N <= 0 || KS <= 0 || N % TN || KS % TK) {
    err = "cpu decode: shape is not a whole number of 64 x 256 tiles";
    return false;
  }
  const int KT = KS / TK, T = (N / TN) * KT;
  const size_t head = sizeof(uint16_t) * LUTN + sizeof(uint32_t) * (size_t)T * LANES;
  if (!blob || nbytes < head + 8) {
    err = "cpu decode: blob shorter than its header";
    return false;
  }
  uint16_t lut[LUTN];
  memcpy(lut, blob, sizeof lut);
  std::vector<uint32_t> start((size_t)T * LANES);
  memcpy(start.data(), blob + sizeof(uint16_t) * LUTN, 4 * start.size());
  const uint64_t nwords = (nbytes - head) / 4, nbits = 32 * nwords;
  std::vector<uint32_t> pay(nwords);
  memcpy(pay.data(), blob + head, 4 * nwords);
  for (uint32_t s : start)
    if (s >= nbits) {
      err = "cpu decode: a lane starts beyond the payload (truncated or corrupt blob)";
      return false;
    }
  std::atomic<int> bad{0};
  // tiles are split into contiguous ranges, one per thread; a lane writes row 64 tr + l, then row 64 tr + 32 + l
  auto work = [&](int t0, int t1) {
    for (int t = t0; t < t1 && !bad.load(std::memory_order_relaxed); ++t) {
      const int tr = t / KT, tc = t % KT;
      for (int l = 0; l < LANES; ++l) {
        LaneBits lb(pay.data(), nwords, start[(size_t)t * LANES + l]);
        uint64_t used = start[(size_t)t * LANES + l];
        for (int r = 0; r < 2; ++r) {
          uint8_t* dst = out + ((size_t)tr * TN + 32 * r + l) * KS + (size_t)tc * TK;
          for (int c = 0; c < TK; ++c) {
            const uint16_t e = lut[lb.peek() & (LUTN - 1)];
            const int len = e >> 8;
            if (len == 0) {  // only a degenerate table has empty entries; a stream that reaches one is corrupt
              bad = 1;
              return;
            }
            dst[c] = (uint8_t)e;
            lb.drop(len);
            used += len;
          }
        }
        if (used > nbits) {
          bad = 1;
          return;
        }
      }
    }
  };
  const auto t0 = std::chrono::steady_clock::now();
  parallel_for(T, std::max(1, threads), work);
  const double dt = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
  if (bad) {
    err = "cpu decode: a lane runs past the end of the payload (truncated or corrupt blob)";
    return false;
  }
  if (seconds) *seconds = dt;
  return true;
}

}  // namespace lw

namespace lw {

void decode_table4(int kqt, const uint16_t* lut, uint32_t* out) {
  for (int i = 0; i < LUTN; ++i) {
    const uint32_t sym = lut[i] & 255u, len = lut[i] >> 8;
    uint32_t v = len;
    if (kq_symbits(kqt) == 4) {
      const uint32_t lo = sym & 15u, hi = sym >> 4;
      if (kqt == KQ_IQ4_XS) v |= (uint32_t)(IQ4_GRID[lo] + 128) << 16 | (uint32_t)(IQ4_GRID[hi] + 128) << 24;
      else v |= lo << 16 | hi << 24;
    } else {
      const float g = kqt == KQ_Q6_K ? (float)sym - 32.f : (float)sym;
      v |= (uint32_t)f32_to_f16(g) << 16;
    }
    out[i] = v;
  }
}

void decode_table_i8(int kqt, const uint16_t* lut, uint32_t* out) {
  auto f = [kqt](uint32_t q) -> uint32_t {
    const int v = kqt == KQ_IQ4_XS ? IQ4_GRID[q & 15] : kqt == KQ_Q6_K ? (int)q - 32 : (int)q;
    return (uint32_t)(uint8_t)(int8_t)v;
  };
  for (int i = 0; i < LUTN; ++i) {
    const uint32_t sym = lut[i] & 255u, len = lut[i] >> 8;
    uint32_t v = len;
    if (kq_symbits(kqt) == 4) v |= f(sym & 15u) << 16 | f(sym >> 4) << 24;
    else v |= f(sym) << 16;
    out[i] = v;
  }
}

bool canon_table(const uint16_t* lut, const uint32_t* entries, uint32_t* out) {
  int len[256] = {}, cnt[LMAX + 1] = {};
  int idx_of[256];  // a window index of each symbol's code (any)
  for (int i = 0; i < LUTN; ++i) {
    const int sym = lut[i] & 255, l = lut[i] >> 8;
    if (l < 1 || l > LMAX) continue;
    if (len[sym] && len[sym] != l) return false;
    len[sym] = l;
    idx_of[sym] = i;
  }
  for (int sym = 0; sym < 256; ++sym) cnt[len[sym]] += len[sym] ? 1 : 0;
  memset(out, 0, CANON_WORDS * 4);
  int code = 0, b = 0;
  for (int l = 1; l <= LMAX; ++l) {
    out[10 + l - 1] = (uint32_t)(4 * (b - code)) << 16 | (uint32_t)(LMAX - l);
    for (int sym = 0; sym < 256; ++sym)
      if (len[sym] == l) out[32 + b++] = entries[idx_of[sym]];
    code += cnt[l];
    if (code > (1 << l)) return false;  // not a prefix code
    if (l < LMAX) out[l - 1] = (uint32_t)code << (LMAX - l);
    code <<= 1;
  }
  // every window that the table decodes must give the same entry by comparison
  for (int i = 0; i < LUTN; ++i) {
    const int l = lut[i] >> 8;
    if (l < 1 || l > LMAX) continue;
    uint32_t v = 0;
    for (int k = 0; k < LMAX; ++k) v |= ((uint32_t)i >> k & 1u) << (LMAX - 1 - k);
    uint32_t p = out[10];
    for (int k = 0; k < LMAX - 1; ++k) p = v >= out[k] ? out[11 + k] : p;
    const int e = (int)(v >> (p & 31u)) + ((int32_t)p >> 16) / 4;
    if ((int)(p & 31u) != LMAX - l || e < 0 || e >= b || out[32 + e] != entries[i]) return false;
  }
  return true;
}

}  // namespace lw
