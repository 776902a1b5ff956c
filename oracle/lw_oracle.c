/* ORACLE — test infrastructure only. Nothing in the product links, loads or calls this file: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg use it, and only as the checker or the CPU baseline.
 *
 * Plain-C restatement of the reference's CPU-side algorithms for the decode-on-demand weight path
 * (paths relative to the reference tree):
 *   orc_decode_lockstep  lazyweights/bundle.py:88-106 (decode_huf8: all lanes of a tile in lock step, 64-bit window)
 *                        and hw/huff/tb/csim_main.cpp:44-62 (ref_decode, add = 0)
 *   orc_cpu_decode       kernels/llmrt.cu:2513-2541 (cpu_decode: per-lane scalar LUT decode, tiles across threads)
 *   orc_canon_build      hw/huff/huff_engine.h:39-52 (build_canon: comparator tables from the LUT)
 *   orc_canon_lookup     hw/huff/huff_engine.h:54-77 (lookup<1>: rev11 window against per-length limits)
 *   orc_sub_scales       scripts/a2_kq_bundle.py:50-68 (sub_sm) = kernels/llmrt.cu:125-149 (kq_side)
 *   orc_dequant          scripts/a2_kq_bundle.py:71-82 (fq, dequant): w = s f(q) - o in fp32
 *   orc_unpack_symbols   scripts/a2_kq_bundle.py:108 inverted (pair symbol -> two codes, low nibble first)
 *   orc_gemv_f64         dequantize-then-matmul in fp64 (the north-star accuracy reference)
 *   orc_decode_gemv      decode + dequant + fp32-accumulate GEMV: the CPU baseline timed beside the GPU
 *
 * Parity pins (tests/): decode functions against golden blobs and decodes written by the reference's own
 * lazyweights/bundle.py (tests/golden/) and against the reference C++ decoder compiled under oracle/_ref;
 * the comparator decode against the LUT over all 2048 windows; sub-scale extraction against the reference's field
 * packing (scripts/kq_quant.py:204-221, restated independently in the test) and hand-built known answers;
 * the GEMV against numpy's fp64 matmul.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define TN 64
#define TK 256
#define LMAX 11
#define LUTN (1 << LMAX)
#define LANES 32

static float h2f(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 31, m = h & 1023;
  uint32_t x;
  float f;
  if (e == 0) {
    f = (float)m * 5.9604644775390625e-08f;
    return (h & 0x8000u) ? -f : f;
  }
  x = e == 31 ? (sign | 0x7F800000u | (m << 13)) : (sign | ((e + 112) << 23) | (m << 13));
  memcpy(&f, &x, 4);
  return f;
}

/* Lock-step decode of a huf8/huf4p blob to symbols [N, KS] (bundle.py:88-106). */
int orc_decode_lockstep(const uint8_t* blob, int N, int KS, uint8_t* out) {
  const int KT = KS / TK, T = (N / TN) * KT;
  const uint16_t* lut = (const uint16_t*)blob;
  const uint32_t* starts = (const uint32_t*)(blob + 2 * LUTN);
  const uint32_t* words = starts + (size_t)T * LANES;
  uint64_t bp[LANES];
  if (N % TN || KS % TK) return -1;
  for (int t = 0; t < T; ++t) {
    const int tr = t / KT, tc = t % KT;
    for (int l = 0; l < LANES; ++l) bp[l] = starts[(size_t)t * LANES + l];
    for (int i = 0; i < 2 * TK; ++i)
      for (int l = 0; l < LANES; ++l) {
        const uint64_t wi = bp[l] >> 5;
        const uint64_t v = (((uint64_t)words[wi] | ((uint64_t)words[wi + 1] << 32)) >> (bp[l] & 31)) & (LUTN - 1);
        const uint16_t e = lut[v];
        const int row = tr * TN + (i >= TK ? 32 : 0) + l, col = tc * TK + (i % TK);
        out[(size_t)row * KS + col] = (uint8_t)(e & 255);
        bp[l] += e >> 8;
      }
  }
  return 0;
}

/* cpu_decode (llmrt.cu:2513-2541): lanes decoded one after another from their absolute starts, with a 64-bit
 * window read at the word containing the bit position; tiles strided across threads. */
typedef struct {
  const uint8_t* blob;
  int N, KS, threads, tid;
  uint8_t* out;
} DecJob;

static void* dec_worker(void* p) {
  const DecJob* j = (const DecJob*)p;
  const int KT = j->KS / TK, T = (j->N / TN) * KT;
  const uint16_t* lut = (const uint16_t*)j->blob;
  const uint32_t* starts = (const uint32_t*)(j->blob + 2 * LUTN);
  const uint8_t* payload = (const uint8_t*)(starts + (size_t)T * LANES);
  for (int tt = j->tid; tt < T; tt += j->threads) {
    const int tr = tt / KT, tc = tt - tr * KT;
    for (int lane = 0; lane < LANES; ++lane) {
      uint64_t bp = starts[(size_t)tt * LANES + lane];
      for (int half = 0; half < 2; ++half) {
        uint8_t* row = j->out + (size_t)(tr * TN + half * 32 + lane) * j->KS + (size_t)tc * TK;
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
  return NULL;
}

int orc_cpu_decode(const uint8_t* blob, int N, int KS, int threads, uint8_t* out) {
  pthread_t th[256];
  DecJob jobs[256];
  if (N % TN || KS % TK) return -1;
  if (threads < 1) threads = 1;
  if (threads > 256) threads = 256;
  for (int i = 0; i < threads; ++i) {
    jobs[i].blob = blob;
    jobs[i].N = N;
    jobs[i].KS = KS;
    jobs[i].threads = threads;
    jobs[i].tid = i;
    jobs[i].out = out;
  }
  for (int i = 1; i < threads; ++i) pthread_create(&th[i], NULL, dec_worker, &jobs[i]);
  dec_worker(&jobs[0]);
  for (int i = 1; i < threads; ++i) pthread_join(th[i], NULL);
  return 0;
}

/* Canonical comparator tables (huff_engine.h:39-52): limit[l] = (first[l] + count[l]) << (11 - l). */
void orc_canon_build(const uint16_t* lut, uint16_t* limit, uint16_t* first, uint16_t* base, uint8_t* sorted) {
  int len[256], cnt[LMAX + 2], code = 0, b = 0;
  memset(len, 0, sizeof len);
  memset(cnt, 0, sizeof cnt);
  for (int i = 0; i < LUTN; ++i) len[lut[i] & 255] = lut[i] >> 8;
  for (int s = 0; s < 256; ++s)
    if (len[s]) ++cnt[len[s]];
  for (int l = 0; l <= LMAX; ++l) limit[l] = first[l] = base[l] = 0;
  for (int l = 1; l <= LMAX; ++l) {
    first[l] = (uint16_t)code;
    base[l] = (uint16_t)b;
    for (int s = 0; s < 256; ++s)
      if (len[s] == l) sorted[b++] = (uint8_t)s;
    code += cnt[l];
    limit[l] = (uint16_t)(code << (LMAX - l));
    code <<= 1;
  }
}

/* Comparator lookup (huff_engine.h:54-77) of an 11-bit LSB-first window: returns sym | len << 8. */
int orc_canon_lookup(const uint16_t* limit, const uint16_t* first, const uint16_t* base, const uint8_t* sorted,
                     uint32_t win) {
  uint32_t v = 0, l = 1;
  for (int i = 0; i < LMAX; ++i) v |= ((win >> i) & 1u) << (LMAX - 1 - i);
  for (int k = 1; k < LMAX; ++k) l += v >= limit[k] ? 1u : 0u;
  return sorted[base[l] + (v >> (LMAX - l)) - first[l]] | (int)(l << 8);
}

/* (s, o) of the sub-blocks of n super-blocks, fp32 as the kernels form them (a2_kq_bundle.py:50-68). kqt:
 * 1 Q4_K, 2 Q5_K (8 sub-blocks), 3 Q6_K (16), 4 IQ4_XS (8). s, o: [n, sub-blocks]. */
int orc_sub_scales(int kqt, const uint8_t* side, long long n, float* s, float* o) {
  const int SB = kqt == 3 ? 18 : kqt == 4 ? 8 : 16, G = kqt == 3 ? 16 : 8;
  for (long long i = 0; i < n; ++i) {
    const uint8_t* b = side + (size_t)i * SB;
    float* si = s + (size_t)i * G;
    float* oi = o + (size_t)i * G;
    if (kqt == 1 || kqt == 2) {
      const float d = h2f((uint16_t)(b[0] | b[1] << 8)), dm = h2f((uint16_t)(b[2] | b[3] << 8));
      const uint8_t* q = b + 4;
      for (int j = 0; j < 8; ++j) {
        int sc, m;
        if (j < 4) {
          sc = q[j] & 63;
          m = q[j + 4] & 63;
        } else {
          sc = (q[j + 4] & 15) | ((q[j - 4] >> 6) << 4);
          m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
        }
        si[j] = d * (float)sc;
        oi[j] = dm * (float)m;
      }
    } else if (kqt == 3) {
      const float d = h2f((uint16_t)(b[16] | b[17] << 8));
      for (int j = 0; j < 16; ++j) {
        si[j] = d * (float)(int8_t)b[j];
        oi[j] = 0.f;
      }
    } else if (kqt == 4) {
      const float d = h2f((uint16_t)(b[0] | b[1] << 8));
      const int hi = b[2] | b[3] << 8;
      for (int j = 0; j < 8; ++j) {
        const int ls = ((b[4 + j / 2] >> (4 * (j & 1))) & 15) | (((hi >> (2 * j)) & 3) << 4);
        si[j] = d * (float)(ls - 32);
        oi[j] = 0.f;
      }
    } else {
      return -1;
    }
  }
  return 0;
}

static const float KV[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};

static float fq(int kqt, int q) { return kqt == 4 ? KV[q & 15] : (float)q - (kqt == 3 ? 32.f : 0.f); }

/* Dequantized weights [N, K] (fp32): w = s f(q) - o per sub-block (a2_kq_bundle.py:71-82). */
int orc_dequant(int kqt, const uint8_t* codes, const uint8_t* side, int N, int K, float* w) {
  const int G = kqt == 3 ? 16 : 8, GW = 256 / G;
  const long long nsb = (long long)N * (K / 256);
  float* s = (float*)malloc(sizeof(float) * nsb * G);
  float* o = (float*)malloc(sizeof(float) * nsb * G);
  if (!s || !o || K % 256 || orc_sub_scales(kqt, side, nsb, s, o)) {
    free(s);
    free(o);
    return -1;
  }
  for (long long i = 0; i < (long long)N * K; ++i) {
    const long long b = i / 256;
    const int g = (int)((i % 256) / GW);
    w[i] = s[b * G + g] * fq(kqt, codes[i]) - o[b * G + g];
  }
  free(s);
  free(o);
  return 0;
}

/* Symbols [N, KS] -> codes [N, K] (pair symbols: even column = low nibble). */
void orc_unpack_symbols(int symbits, const uint8_t* sym, int N, int KS, uint8_t* codes) {
  if (symbits == 8) {
    memcpy(codes, sym, (size_t)N * KS);
    return;
  }
  for (size_t i = 0; i < (size_t)N * KS; ++i) {
    codes[2 * i] = sym[i] & 15;
    codes[2 * i + 1] = sym[i] >> 4;
  }
}

/* Y[m, N] = X[m, K] W[N, K]^T in fp64. */
void orc_gemv_f64(const float* w, const double* x, int m, int N, int K, double* y) {
  for (int j = 0; j < m; ++j)
    for (int n = 0; n < N; ++n) {
      const float* wr = w + (size_t)n * K;
      const double* xr = x + (size_t)j * K;
      double a = 0;
      for (int k = 0; k < K; ++k) a += (double)wr[k] * xr[k];
      y[(size_t)j * N + n] = a;
    }
}

/* CPU baseline: cpu_decode of the raw blob to symbols, then per row dequant + fp32-accumulate GEMV
 * (rows split across threads). x fp32 [K]; y [N]. Returns 0. */
typedef struct {
  int kqt, N, K, KS, threads, tid;
  const uint8_t* sym;
  const uint8_t* side;
  const float* x;
  float* y;
} GemvJob;

static void* gemv_worker(void* p) {
  const GemvJob* j = (const GemvJob*)p;
  const int G = j->kqt == 3 ? 16 : 8, GW = 256 / G, NSB = j->K / 256, SB = j->kqt == 3 ? 18 : j->kqt == 4 ? 8 : 16;
  float s[16], o[16];
  for (int n = j->tid; n < j->N; n += j->threads) {
    const uint8_t* sr = j->sym + (size_t)n * j->KS;
    float acc = 0.f;
    for (int b = 0; b < NSB; ++b) {
      orc_sub_scales(j->kqt, j->side + ((size_t)n * NSB + b) * SB, 1, s, o);
      for (int g = 0; g < G; ++g) {
        float a = 0.f, xs = 0.f;
        for (int k = b * 256 + g * GW; k < b * 256 + (g + 1) * GW; ++k) {
          const int q = (j->kqt == 1 || j->kqt == 4) ? ((sr[k >> 1] >> (4 * (k & 1))) & 15) : sr[k];
          a += fq(j->kqt, q) * j->x[k];
          xs += j->x[k];
        }
        acc += s[g] * a - o[g] * xs;
      }
    }
    j->y[n] = acc;
  }
  return NULL;
}

int orc_decode_gemv(int kqt, const uint8_t* blob, const uint8_t* side, int N, int K, const float* x, int threads,
                    uint8_t* sym_scratch, float* y) {
  const int KS = (kqt == 1 || kqt == 4) ? K / 2 : K;
  pthread_t th[256];
  GemvJob jobs[256];
  if (threads < 1) threads = 1;
  if (threads > 256) threads = 256;
  if (orc_cpu_decode(blob, N, KS, threads, sym_scratch)) return -1;
  for (int i = 0; i < threads; ++i) {
    jobs[i].kqt = kqt;
    jobs[i].N = N;
    jobs[i].K = K;
    jobs[i].KS = KS;
    jobs[i].threads = threads;
    jobs[i].tid = i;
    jobs[i].sym = sym_scratch;
    jobs[i].side = side;
    jobs[i].x = x;
    jobs[i].y = y;
  }
  for (int i = 1; i < threads; ++i) pthread_create(&th[i], NULL, gemv_worker, &jobs[i]);
  gemv_worker(&jobs[0]);
  for (int i = 1; i < threads; ++i) pthread_join(th[i], NULL);
  return 0;
}
