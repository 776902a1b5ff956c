// Runtime and C-ABI of the decode-on-demand weight path (include/lazyweights_amd.h).
//
// Reference counterparts (kernels/llmrt.cu): rt_open 1921-2237 (manifest, residency, interleave at load, .kqs side
// tensors), matmul() K-quant branch 1806-1842, rt_test_matmul 2441, rt_test_decode 2461, rt_gpu_decode_all 2482,
// cpu_decode / rt_test_cpu_decode / rt_cpu_decode_all 2513-2573, rt_stat 2276. Differences by design: no exit() on
// bad input (error codes + lw_last_error), matrix-only bundles open, the device layout is this library's own
// (lw_kernels.h), and there is no model runtime or weight streaming.
#include <fcntl.h>
#include <hip/hip_runtime.h>
#include <rocblas/rocblas.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <map>
#include <memory>
#include <mutex>
#include <sstream>
#include <string>
#include <vector>

#include "../../include/lazyweights_amd.h"
#include "lw_codec.h"
#include "lw_format.h"
#include "lw_kernels.h"
#include "lw_layout.h"

namespace {

thread_local std::string g_err;

bool fail(const std::string& m) {
  g_err = m;
  return false;
}

#define HIPCHECK(x)                                                                                  \
  do {                                                                                               \
    hipError_t e_ = (x);                                                                             \
    if (e_ != hipSuccess) {                                                                          \
      g_err = std::string("HIP error ") + hipGetErrorString(e_) + " at " + __FILE__ + ":" + std::to_string(__LINE__); \
      return -1;                                                                                     \
    }                                                                                                \
  } while (0)

long long meminfo_kb(const char* key) {
  FILE* f = fopen("/proc/meminfo", "r");
  if (!f) return -1;
  char k[64];
  long long v = -1, x;
  while (fscanf(f, "%63s %lld kB", k, &x) == 2)
    if (!strncmp(k, key, strlen(key)) && k[strlen(key)] == ':') {
      v = x;
      break;
    }
  fclose(f);
  return v;
}

bool pread_all(int fd, void* buf, size_t n, uint64_t off) {
  uint8_t* p = static_cast<uint8_t*>(buf);
  while (n) {
    const ssize_t r = pread(fd, p, n, (off_t)off);
    if (r <= 0) return false;
    p += r;
    n -= (size_t)r;
    off += (uint64_t)r;
  }
  return true;
}

struct Tensor {
  std::string name, enc;
  long long N = 0, K = 0;
  double scale = 1.0;
  long long zp = 0;
  uint64_t off = 0, nbytes = 0;
  bool pre_il = false, compact = false;
  int symbits = 8, kqt = 0;
  int side_idx = -1;
  bool resident = false;
  void* dev = nullptr;  // device layout (one allocation)
  size_t dev_bytes = 0;
  uint8_t* dside = nullptr;
  size_t side_bytes = 0;
  uint64_t payload_bits = 0;
  lw::DevMat dm{};
  std::vector<uint32_t> exc32;  // host copy of the exception tiles with a 32-row schedule (dm.exc[0, nexc32))
  bool coded() const { return enc == "huf8" || enc == "huf4p"; }
  // the fixed-rate twin: the symbols stored as plain bytes (reference enc pk4 / pk8, kernels/llmrt.cu:1731-1750)
  bool packed() const { return enc == "pk4" || enc == "pk8"; }
  bool matrix() const { return coded() || packed(); }
  int KS() const { return (int)(symbits == 4 ? K / 2 : K); }
  int T() const { return (int)((N / lw::TN) * (KS() / lw::TK)); }
};

struct Model {
  std::string dir;
  std::map<std::string, std::string> cfg;
  std::vector<Tensor> ts;
  std::map<std::string, int> by_name;
  int fd = -1;
  uint64_t file_size = 0;
  bool gpu = false;
  hipStream_t stream = nullptr;
  size_t resident_bytes = 0, coded_bytes = 0, device_bytes = 0, pad_bytes = 0;
  long long avail_after_kb = -1;
  int pos = 0, window = 0;
  // device scratch, grown on demand
  float* P = nullptr;
  size_t P_cap = 0;
  uint32_t* cnt = nullptr;  // tile-row counters of the in-launch reduction, zeroed (every launch leaves them zeroed)
  size_t cnt_cap = 0;
  uint16_t* X16 = nullptr;
  size_t X16_cap = 0;
  uint16_t* SX = nullptr;  // per-sub-block activation sums (prefill GEMM)
  size_t SX_cap = 0;
  uint8_t* x8 = nullptr;  // int8 activations: per vector [K int8][K / 32 d][K / 32 d sum q], 256-B aligned parts
  size_t x8_cap = 0;
  uint8_t* codes = nullptr;
  size_t codes_cap = 0;
  uint16_t* W16 = nullptr;  // prefill: fp16 [hi | lo] weights of a chunk of rows
  size_t W16_cap = 0;
  float* T32 = nullptr;  // prefill, one-GEMM form: the GEMM's [2m][rows] output
  size_t T32_cap = 0;
  rocblas_handle blas = nullptr;  // prefill GEMMs, created on first use
  int verbose = 0;
  Tensor* find(const char* name) {
    if (!name) return nullptr;
    auto it = by_name.find(name);
    return it == by_name.end() ? nullptr : &ts[it->second];
  }
};

bool ends_with(const std::string& s, const std::string& x) {
  return s.size() > x.size() && !s.compare(s.size() - x.size(), x.size(), x);
}

template <class T>
int grow(T*& p, size_t& cap, size_t bytes) {
  if (bytes <= cap) return 0;
  if (p) (void)hipFree(p);
  p = nullptr;
  cap = 0;
  HIPCHECK(hipMalloc(reinterpret_cast<void**>(&p), bytes));
  cap = bytes;
  return 0;
}

// as grow, zero-filled when (re)allocated
template <class T>
int grow_zeroed(T*& p, size_t& cap, size_t bytes) {
  if (bytes <= cap) return 0;
  if (grow(p, cap, bytes)) return -1;
  HIPCHECK(hipMemset(p, 0, cap));
  return 0;
}

// ── load ─────────────────────────────────────────────────────────────────────────────────────────────────

bool parse_manifest(Model& M) {
  std::ifstream mf(M.dir + "/manifest.txt");
  if (!mf) return fail("cannot open " + M.dir + "/manifest.txt");
  std::string line;
  int ln = 0;
  while (std::getline(mf, line)) {
    ++ln;
    std::istringstream is(line);
    std::string tag;
    if (!(is >> tag)) continue;
    if (tag == "cfg") {
      std::string k, v;
      if (!(is >> k >> v)) return fail("manifest line " + std::to_string(ln) + ": bad cfg line");
      M.cfg[k] = v;
    } else if (tag == "t") {
      Tensor t;
      if (!(is >> t.name >> t.enc >> t.N >> t.K >> t.scale >> t.zp >> t.off >> t.nbytes))
        return fail("manifest line " + std::to_string(ln) + ": bad tensor line");
      for (const char* x : {"_ilc", "_il"}) {  // pre-interleaved export (kernels/llmrt.cu:1938-1947)
        if (ends_with(t.enc, x)) {
          t.enc.resize(t.enc.size() - strlen(x));
          t.pre_il = true;
          t.compact = x[3] == 'c';
          break;
        }
      }
      if (t.N <= 0 || t.K <= 0) return fail("manifest line " + std::to_string(ln) + ": non-positive shape");
      t.symbits = t.enc == "huf4p" || t.enc == "pk4" ? 4 : 8;
      if (M.by_name.count(t.name)) return fail("manifest: duplicate tensor " + t.name);
      M.by_name[t.name] = (int)M.ts.size();
      M.ts.push_back(t);
    }
  }
  return true;
}

bool validate(Model& M) {
  static const char* kn[] = {"", "kq_Q4_K", "kq_Q5_K", "kq_Q6_K", "kq_IQ4_XS"};
  for (auto& t : M.ts) {
    if (t.off + t.nbytes > M.file_size)
      return fail(t.name + ": extends past the end of weights.bin");
    if (!t.matrix()) continue;
    if (t.packed() && t.pre_il) return fail(t.name + ": " + t.enc + " has no pre-interleaved form");
    if (t.packed() && t.nbytes < (uint64_t)t.N * t.KS()) return fail(t.name + ": packed blob shorter than N x K");
    if (t.N % lw::TN || t.K % (t.symbits == 4 ? 2 * lw::TK : lw::TK))
      return fail(t.name + ": shape " + std::to_string(t.N) + "x" + std::to_string(t.K) +
                  " is not a whole number of 64 x 256-symbol tiles");
    if (t.K >= (1ll << 31) || t.N >= (1ll << 31)) return fail(t.name + ": shape too large");
    auto it = M.by_name.find(t.name + ".kqs");
    if (it == M.by_name.end()) continue;  // decode-only matrix (no K-quant side bytes)
    const Tensor& x = M.ts[it->second];
    int kqt = 0;
    for (int i = 1; i <= 4; ++i)
      if (x.enc == kn[i]) kqt = i;
    if (!kqt) return fail(t.name + ": side tensor " + x.name + " has unknown enc " + x.enc);
    if (x.N != t.N || x.K != (t.K / 256) * lw::kq_sbytes(kqt) || x.nbytes < (uint64_t)x.N * x.K)
      return fail(t.name + ": side tensor " + x.name + " shape does not match the matrix");
    if (t.symbits != lw::kq_symbits(kqt))
      return fail(t.name + ": " + x.enc + " needs enc " + (lw::kq_symbits(kqt) == 4 ? "huf4p / pk4" : "huf8 / pk8"));
    t.kqt = kqt;
    t.side_idx = it->second;
  }
  return true;
}

// Upload a K-quant matrix's side bytes in the kernels' tile-major record order (lw::side_record).
bool upload_side(Model& M, Tensor& t) {
  lw::DevMat& dm = t.dm;
  const Tensor& x = M.ts[t.side_idx];
  t.side_bytes = (size_t)x.N * x.K;
  std::vector<uint8_t> raw(t.side_bytes), sb(t.side_bytes);
  if (!pread_all(M.fd, raw.data(), t.side_bytes, x.off)) return fail(t.name + ": side read error");
  // bundle order [N][K/256][SB] -> the kernels' tile-major record order (lw::side_record)
  const int SB = lw::kq_sbytes(t.kqt), nb = (int)(t.K / 256), nsb = t.symbits == 4 ? 2 : 1;
  for (int n = 0; n < (int)t.N; ++n)
    for (int b = 0; b < nb; ++b)
      memcpy(sb.data() + lw::side_record(n, b, dm.KT, nsb) * SB, raw.data() + ((size_t)n * nb + b) * SB, SB);
  std::vector<uint8_t>().swap(raw);
  // 16 bytes past the records: the half-tile kernel reads a Q6_K record as the 5 aligned dwords holding it
  if (hipMalloc(reinterpret_cast<void**>(&t.dside), t.side_bytes + 16) != hipSuccess) {
    (void)hipGetLastError();
    return fail(t.name + ": device allocation failed (side)");
  }
  if (hipMemset(t.dside + t.side_bytes, 0, 16) != hipSuccess) return fail(t.name + ": upload failed (side)");
  if (hipMemcpy(t.dside, sb.data(), t.side_bytes, hipMemcpyHostToDevice) != hipSuccess)
    return fail(t.name + ": upload failed (side)");
  dm.side = t.dside;
  return true;
}

// Build and upload the device layout (and side bytes) of a coded tensor.
bool make_resident(Model& M, Tensor& t, int threads) {
  std::vector<uint8_t> blob(t.nbytes + 16, 0);
  if (!pread_all(M.fd, blob.data(), t.nbytes, t.off)) return fail(t.name + ": read error");
  lw::Layout L;
  std::string err;
  const bool ok = t.pre_il ? lw::build_layout_il(blob.data(), t.nbytes, (int)t.N, t.KS(), t.compact, threads, L, err)
                           : lw::build_layout_raw(blob.data(), t.nbytes, (int)t.N, t.KS(), threads, L, err);
  if (!ok) return fail(t.name + ": " + err);
  std::vector<uint8_t>().swap(blob);
  const int T = t.T();
  // [lut 4096 B][4-byte table 8192 B][int8 table 8192 B][comparator table 1152 B][tbase 4T][mid 64T][split 1024T][rows 2T]
  // [sched 16T (16-aligned)][hrow 4T][hsplit 1024T][dsplit 512T][exception tiles 4E] padded to 256 B, then the words
  const size_t nexc = L.exc.size();
  const size_t o_lut4 = 2 * lw::LUTN, o_luti8 = o_lut4 + 4 * lw::LUTN, o_canon = o_luti8 + 4 * lw::LUTN;
  const size_t o_tb = o_canon + 4 * lw::CANON_WORDS;
  const size_t o_mid = o_tb + 4ull * T;
  const size_t o_split = o_mid + 64ull * T, o_rows = o_split + 64ull * lw::SPLITS * T;
  const size_t o_sched = (o_rows + 2ull * T + 15) & ~(size_t)15, o_hrow = o_sched + 16ull * T;
  const size_t o_hsplit = (o_hrow + 4ull * T + 15) & ~(size_t)15, o_dsplit = o_hsplit + 1024ull * T;
  const size_t o_exc = o_dsplit + 512ull * T;
  const size_t o_words = (o_exc + 4 * nexc + 255) & ~(size_t)255;
  const size_t bytes = o_words + 4 * L.words.size();
  std::vector<uint8_t> host(o_words, 0);
  memcpy(host.data(), L.lut, 2 * lw::LUTN);
  bool canon = false;
  if (t.kqt) {
    lw::decode_table4(t.kqt, L.lut, reinterpret_cast<uint32_t*>(host.data() + o_lut4));
    lw::decode_table_i8(t.kqt, L.lut, reinterpret_cast<uint32_t*>(host.data() + o_luti8));
    canon = lw::canon_table(L.lut, reinterpret_cast<const uint32_t*>(host.data() + o_lut4),
                            reinterpret_cast<uint32_t*>(host.data() + o_canon));
  }
  memcpy(host.data() + o_tb, L.tbase.data(), 4ull * T);
  memcpy(host.data() + o_mid, L.mid.data(), 64ull * T);
  memcpy(host.data() + o_split, L.split.data(), 64ull * lw::SPLITS * T);
  memcpy(host.data() + o_rows, L.rows.data(), 2ull * T);
  memcpy(host.data() + o_sched, L.sched.data(), 16ull * T);
  memcpy(host.data() + o_hrow, L.hrow.data(), 4ull * T);
  {  // the half-tile kernel's chain starts: unit (t, f), lane 32 h + s, chains j = the split offsets 8 f + 4 h + j
    uint16_t* hs = reinterpret_cast<uint16_t*>(host.data() + o_hsplit);
    for (size_t t = 0; t < (size_t)T; ++t)
      for (int f = 0; f < 2; ++f)
        for (int h = 0; h < 2; ++h)
          for (int s = 0; s < lw::LANES; ++s)
            for (int j = 0; j < 4; ++j)
              hs[((t * 2 + f) * 64 + 32 * h + s) * 4 + j] = L.split[(t * lw::SPLITS + 8 * f + 4 * h + j) * lw::LANES + s];
  }
  {  // the whole-tile kernels' chain starts of (t, f, lane stream s) after the first (mid or the guard): 7 deltas of
     // 32 symbols each (32 .. 352 bits), less 32, in 9 bits each
    uint64_t* ds = reinterpret_cast<uint64_t*>(host.data() + o_dsplit);
    for (size_t u = 0; u < (size_t)T; ++u)
      for (int f = 0; f < 2; ++f)
        for (int s = 0; s < lw::LANES; ++s) {
          uint64_t v = 0;
          for (int j = 0; j < 7; ++j) {
            const int a = L.split[(u * lw::SPLITS + 8 * f + j) * lw::LANES + s];
            const int b = L.split[(u * lw::SPLITS + 8 * f + j + 1) * lw::LANES + s];
            if (b - a < 32 || b - a > 32 + 511) return fail(t.name + ": chain start delta out of range");
            v |= (uint64_t)(b - a - 32) << (9 * j);
          }
          ds[(u * 2 + f) * lw::LANES + s] = v;
        }
  }
  if (nexc) memcpy(host.data() + o_exc, L.exc.data(), 4 * nexc);
  void* d = nullptr;
  if (hipMalloc(&d, bytes) != hipSuccess) {
    (void)hipGetLastError();
    return fail(t.name + ": device allocation failed");
  }
  if (hipMemcpy(d, host.data(), o_words, hipMemcpyHostToDevice) != hipSuccess ||
      hipMemcpy(static_cast<uint8_t*>(d) + o_words, L.words.data(), 4 * L.words.size(), hipMemcpyHostToDevice) !=
          hipSuccess) {
    (void)hipFree(d);
    return fail(t.name + ": upload failed");
  }
  t.dev = d;
  t.dev_bytes = bytes;
  t.payload_bits = L.payload_bits;
  lw::DevMat& dm = t.dm;
  uint8_t* b = static_cast<uint8_t*>(d);
  dm.lut = reinterpret_cast<const uint16_t*>(b);
  dm.lut4 = t.kqt ? reinterpret_cast<const uint32_t*>(b + o_lut4) : nullptr;
  dm.luti8 = t.kqt ? reinterpret_cast<const uint32_t*>(b + o_luti8) : nullptr;
  dm.canon = canon ? reinterpret_cast<const uint32_t*>(b + o_canon) : nullptr;
  dm.tbase = reinterpret_cast<const uint32_t*>(b + o_tb);
  dm.mid = reinterpret_cast<const uint16_t*>(b + o_mid);
  dm.split = reinterpret_cast<const uint16_t*>(b + o_split);
  dm.rows = reinterpret_cast<const uint16_t*>(b + o_rows);
  dm.hrow = reinterpret_cast<const uint32_t*>(b + o_hrow);
  dm.hsplit = reinterpret_cast<const uint16_t*>(b + o_hsplit);
  dm.dsplit = reinterpret_cast<const uint64_t*>(b + o_dsplit);
  dm.words = reinterpret_cast<const uint32_t*>(b + o_words);
  dm.sched = reinterpret_cast<const uint4*>(b + o_sched);
  dm.ring_rows = L.ring_rows;
  dm.exc = nexc ? reinterpret_cast<const uint32_t*>(b + o_exc) : nullptr;
  dm.nexc = (int)nexc;
  dm.nexc32 = L.nexc32;
  t.exc32.assign(L.exc.begin(), L.exc.begin() + L.nexc32);
  dm.side = nullptr;
  dm.N = (int)t.N;
  dm.K = (int)t.K;
  dm.kqt = t.kqt;
  dm.symbits = t.symbits;
  dm.KT = t.KS() / lw::TK;
  dm.NT = (int)(t.N / lw::TN);
  dm.max_rows = L.max_rows;
  dm.tstride = L.tstride;
  dm.max_hrows = L.max_hrows;
  if (t.kqt && !upload_side(M, t)) return false;
  t.resident = true;
  M.resident_bytes += bytes + t.side_bytes;
  M.device_bytes += bytes;
  M.coded_bytes += t.nbytes + t.side_bytes;
  const size_t blob_pay = (size_t)((t.payload_bits + 31) / 32) * 4;
  M.pad_bytes += bytes > blob_pay ? bytes - blob_pay : 0;
  return true;
}

// Build and upload the device layout of a packed (fixed-rate) tensor: [symbol table 256 x 4 B, the payload bits of
// decode_table4 for every symbol] padded to 256 B, then the symbols as 16-byte chunks [T][16 groups][64 rows]: chunk
// (t, g, L) = symbols 16 g .. 16 g + 15 of tile row L, so a wave reads one group of its tile as 1 KB.
bool make_resident_packed(Model& M, Tensor& t) {
  const int KS = t.KS(), NT = (int)(t.N / lw::TN), KT = KS / lw::TK, T = NT * KT;
  std::vector<uint8_t> blob((size_t)t.N * KS);
  if (!pread_all(M.fd, blob.data(), blob.size(), t.off)) return fail(t.name + ": read error");
  const size_t o_words = 2 * 256 * 4, bytes = o_words + (size_t)T * lw::TN * lw::TK + 8 * 128;
  std::vector<uint8_t> host(bytes, 0);
  if (t.kqt) {  // [symbol table 256 x 4 B][int8 symbol table 256 x 4 B]
    std::vector<uint16_t> ident(lw::LUTN);
    for (int i = 0; i < lw::LUTN; ++i) ident[i] = (uint16_t)(i & 255);
    std::vector<uint32_t> tab(lw::LUTN);
    lw::decode_table4(t.kqt, ident.data(), tab.data());
    memcpy(host.data(), tab.data(), 256 * 4);
    lw::decode_table_i8(t.kqt, ident.data(), tab.data());
    memcpy(host.data() + 256 * 4, tab.data(), 256 * 4);
  }
  uint8_t* w = host.data() + o_words;
  for (int tr = 0; tr < NT; ++tr)
    for (int tc = 0; tc < KT; ++tc)
      for (int g = 0; g < 16; ++g)
        for (int L = 0; L < lw::TN; ++L)
          memcpy(w + ((((size_t)tr * KT + tc) * 16 + g) * lw::TN + L) * 16,
                 blob.data() + (size_t)(tr * lw::TN + L) * KS + tc * lw::TK + 16 * g, 16);
  std::vector<uint8_t>().swap(blob);
  void* d = nullptr;
  if (hipMalloc(&d, bytes) != hipSuccess) {
    (void)hipGetLastError();
    return fail(t.name + ": device allocation failed");
  }
  if (hipMemcpy(d, host.data(), bytes, hipMemcpyHostToDevice) != hipSuccess) {
    (void)hipFree(d);
    return fail(t.name + ": upload failed");
  }
  t.dev = d;
  t.dev_bytes = bytes;
  t.payload_bits = (uint64_t)t.N * KS * 8;
  lw::DevMat& dm = t.dm;
  dm = lw::DevMat{};
  uint8_t* b = static_cast<uint8_t*>(d);
  dm.lut4 = t.kqt ? reinterpret_cast<const uint32_t*>(b) : nullptr;
  dm.luti8 = t.kqt ? reinterpret_cast<const uint32_t*>(b + 256 * 4) : nullptr;
  dm.words = reinterpret_cast<const uint32_t*>(b + o_words);
  dm.packed = 1;
  dm.N = (int)t.N;
  dm.K = (int)t.K;
  dm.kqt = t.kqt;
  dm.symbits = t.symbits;
  dm.KT = KT;
  dm.NT = NT;
  if (t.kqt && !upload_side(M, t)) return false;
  t.resident = true;
  M.resident_bytes += bytes + t.side_bytes;
  M.device_bytes += bytes;
  M.coded_bytes += t.nbytes + t.side_bytes;
  return true;
}

void release(Model* M) {
  if (!M) return;
  for (auto& t : M->ts) {
    if (t.dev) (void)hipFree(t.dev);
    if (t.dside) (void)hipFree(t.dside);
  }
  if (M->P) (void)hipFree(M->P);
  if (M->cnt) (void)hipFree(M->cnt);
  if (M->X16) (void)hipFree(M->X16);
  if (M->SX) (void)hipFree(M->SX);
  if (M->x8) (void)hipFree(M->x8);
  if (M->codes) (void)hipFree(M->codes);
  if (M->W16) (void)hipFree(M->W16);
  if (M->T32) (void)hipFree(M->T32);
  if (M->blas) (void)rocblas_destroy_handle(M->blas);
  if (M->stream) (void)hipStreamDestroy(M->stream);
  if (M->fd >= 0) close(M->fd);
  delete M;
}

// ── matmul ───────────────────────────────────────────────────────────────────────────────────────────────

int check_matmul(Tensor* t, const char* name) {
  if (!t) {
    g_err = std::string("no tensor ") + (name ? name : "(null)");
    return -1;
  }
  if (!t->resident) {
    g_err = t->name + ": not resident";
    return -1;
  }
  if (!t->kqt) {
    g_err = t->name + ": not a K-quant coded matrix (no .kqs side tensor)";
    return -1;
  }
  return 0;
}

// Kernel selection for the fused path: 0 = ring kernels wherever the matrix has a ring schedule (default; the flat
// kernel for m = 1), 2 = the block-per-column ring kernel for every m,
// 1 = whole-tile kernel everywhere (kept as the fallback and for tests).
int g_kernel_mode = 0;

// CUs of the current device (256 if it cannot be read), read once
int cu_count() {
  static int cus = 0;
  if (!cus) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1)
      cus = 256;
  }
  return cus;
}

// Cost model of a flat launch: every block is w waves of one tile each and stays resident until its slowest wave
// ends. The blocks spread evenly over the CUs; a CU runs its share in rounds of as many blocks as fit at once (LDS:
// `lds` bytes per block of 160 KB; waves: wcu, 32 unless registers allow fewer), and a round takes about
// max(its waves, 16) tile times (below 16 waves a CU is no longer issue-bound). Returns the busiest CU's sum over
// rounds, in tile times.
long long flat_cost(int total, int w, int lds, int wcu = 32) {
  const int cus = cu_count();
  const long long per_cu = std::max(1, std::min(160 * 1024 / lds, wcu / w));
  const long long blocks = (total + w - 1) / w, b = (blocks + cus - 1) / cus;
  const long long full = b / per_cu, rest = b % per_cu;
  return full * std::max<long long>(per_cu * w, 16) + (rest ? std::max<long long>(rest * w, 16) : 0);
}

// LDS of a flat block: one or two 8 KB decode tables + w x 2 rings of rs rows + extra (spare rings)
int flat_lds(int w, int rs, int extra) { return (w > 1 ? 2 : 1) * 8192 + w * 2 * rs * 128 + extra; }

// Waves per block of the flat kernel for a launch of `total` tiles: the width of least flat_cost (ties: the larger
// W) within the kernel's limits: 16 waves per block and W <= the smallest matrix's tile count (a block holds at most
// two tables). Config 2's 6656 tiles on 256 CUs give W = 13: 512 blocks, one round of 26 waves on every CU (W = 16
// leaves 96 CUs with one block of 16 waves and 160 with two).
int flat_width(int total, int rs, int mintiles, int spare_bytes, int wcu = 32) {
  const int wmax = std::min(std::min(rs == 16 ? 16 : 8, mintiles), std::max(1, wcu));
  int best = 1;
  long long best_cost = -1;
  for (int w = 1; w <= wmax; ++w) {
    const long long cost = flat_cost(total, w, flat_lds(w, rs, spare_bytes), wcu);
    if (best_cost < 0 || cost <= best_cost) {
      best_cost = cost;
      best = w;
    }
  }
  return std::max(1, best);
}

// Both kernels in units of one dependent symbol-pair step (about 630 cycles at full load). The ring kernel's waves
// run 128 pairs per tile; the low-latency kernel's blocks (4 waves, one tile, whole tile staged in LDS) run 32 pairs
// after staging (counted as 8 more) and a combine step.
long long ring_cost(int total, int w, int lds, int wcu = 32) { return flat_cost(total, w, lds, wcu) * 128; }
long long split_cost(int total, int stage_rows, int kqt) {
  const int cus = cu_count();
  const int nsubt = lw::kq_symbits(kqt) == 4 ? 2 * lw::TK / lw::kq_gw(kqt) : lw::TK / lw::kq_gw(kqt);
  const int lds = 4 * lw::LUTN + lw::TN * nsubt * 4 + stage_rows * 128;
  const long long per_cu = std::max(1, std::min(160 * 1024 / lds, 8));
  const long long b = (total + cus - 1) / cus, full = b / per_cu, rest = b % per_cu;
  return full * std::max<long long>(4 * per_cu, 16) * 40 + (rest ? std::max<long long>(4 * rest, 16) * 40 : 0);
}

// Int8 activations for m = 1 GEMVs (the reference's default on sm_61+, off there with LLMRT_FP_ACT=1; off by
// default here, where fp16 hi + lo activations are the default): x quantized per block of 32 (k_quant_x8), integer
// dot products per sub-block (kernels/llmrt.cu:1035-1169, 1808-1813, 2221).
int g_act8 = 0;

struct X8 {
  const int8_t* q;
  const float* d;
  const float* s;
};

// Device scratch owned by the caller of a fused launch (lw_matmul_dev_noalloc): `bytes` at `base`.
struct FixedScratch {
  uint8_t* base;
  size_t bytes;
};

// Quantize the activations of each of `count` matrices (m tokens [m][K_i], fp16 or fp32; a vector shared by several
// matrices once) into the model's x8 scratch; x8[i] = matrix i's quantized x ([m][K_i] int8, [m][K_i / 32] scales).
int quant_x8_dev(Model& M, Tensor* const* ts, const void* const* X, int x_f16, int count, std::vector<X8>& x8,
                 hipStream_t s, int m = 1) {
  auto al = [](size_t b) { return (b + 255) & ~(size_t)255; };
  std::vector<size_t> off(count);
  // one quantized copy per distinct (vector, K): owner[i] = true for the matrix whose slot quantizes it
  std::map<std::pair<const void*, long long>, int> first;
  std::vector<char> owner(count, 0);
  size_t total = 0;
  for (int i = 0; i < count; ++i) {
    const size_t K = (size_t)ts[i]->K * m;
    const auto key = std::make_pair(X[i], (long long)ts[i]->K);
    auto it = first.find(key);
    if (it != first.end()) {
      off[i] = off[it->second];
      continue;
    }
    first[key] = i;
    owner[i] = 1;
    off[i] = total;
    total += al(K) + 2 * al(K / 32 * 4);
  }
  if (grow(M.x8, M.x8_cap, total)) return -1;
  x8.resize(count);
  lw::QuantJobs q{};
  q.x_f16 = x_f16;
  int blocks = 0;
  for (int i = 0; i < count; ++i) {
    const size_t K = (size_t)ts[i]->K * m;
    uint8_t* b = M.x8 + off[i];
    x8[i] = X8{reinterpret_cast<const int8_t*>(b), reinterpret_cast<const float*>(b + al(K)),
               reinterpret_cast<const float*>(b + al(K) + al(K / 32 * 4))};
    if (!owner[i]) continue;
    if (q.n == lw::MAX_GROUP) {
      HIPCHECK(lw::launch_quant_x8_group(q, s));
      q.n = 0;
      blocks = 0;
    }
    q.X[q.n] = X[i];
    q.XQ[q.n] = reinterpret_cast<int8_t*>(b);
    q.DX[q.n] = reinterpret_cast<float*>(b + al(K));
    q.SX[q.n] = reinterpret_cast<float*>(b + al(K) + al(K / 32 * 4));
    q.nb[q.n] = (int)(K / 32);
    q.b0[q.n] = blocks;
    blocks += (int)(K / 32 + 7) / 8;
    ++q.n;
  }
  if (q.n) HIPCHECK(lw::launch_quant_x8_group(q, s));
  return 0;
}

// Waves per block and tiles per block of the whole-tile kernel for a flat plan: one tile buffer per wave
// (tiles_buf_rows) next to one or two 8 KB tables in 160 KB of LDS, at most 16 waves, a multiple of 4 when it can be
// (the waves of a block then share the 4 SIMDs evenly); `per` = the tiles that spread the plan over every CU once,
// at most the smallest matrix's tile count (a block spans at most two matrices). Returns 0 if no width fits.
int tiles_width(const lw::FlatPlan& fp, int mintiles, int& per) {
  const int cus = cu_count();
  const int rows = lw::tiles_buf_rows(fp), tables = (fp.n > 1 ? 2 : 1) * 4 * lw::LUTN;
  if (rows > 256) return 0;
  const int wmax = std::min(fp.canon ? lw::TILES_CANON_WAVES : 16,
                            (160 * 1024 - tables - 4 * (4 + lw::TILES_ROWC)) / (rows * 128));
  if (wmax < 1) return 0;
  per = (fp.ntiles + cus - 1) / cus;
  if (fp.n > 1) per = std::min(per, mintiles);
  // the fewest rounds of tiles the LDS allows, then the fewest waves that take the block's tiles in that many
  // rounds: a last round with few waves busy leaves the CU idle for a whole tile (26 tiles per CU on 12 waves ran
  // 12 + 12 + 2); the waves take tiles from a counter, so they need not spread evenly over the SIMDs
  const int rounds = (per + wmax - 1) / wmax;
  return std::min(wmax, (per + rounds - 1) / rounds);
}

// Waves per block and tiles per block of the matrix-core whole-tile kernel (2..8 tokens): the tiles as tiles_width,
// each block's x sums (tiles_mma_xs_bytes) beside the tile buffers, and as many waves as the LDS holds (measured at
// m = 2..8 on config 2: 12 waves taking 26 tiles in rounds of 12, 12 and 2 ran 6-9 % faster than 9 waves in 3
// rounds, unlike the m = 1 kernel). Returns 0 if no width fits.
int tiles_mma_width(const lw::FlatPlan& fp, int mintiles, int& per) {
  const int cus = cu_count();
  const int rows = lw::tiles_buf_rows(fp), tables = (fp.n > 1 ? 2 : 1) * 4 * lw::LUTN;
  if (rows > 256) return 0;
  per = (fp.ntiles + cus - 1) / cus;
  if (fp.n > 1) per = std::min(per, mintiles);
  const long room = 160L * 1024 - tables - 16 - (long)lw::tiles_mma_xs_bytes(fp, per);
  int wcap = lw::tiles_mma_max_waves(fp.e[0].M.kqt, fp.mt);
  for (int k = 1; k < fp.n; ++k) wcap = std::min(wcap, lw::tiles_mma_max_waves(fp.e[k].M.kqt, fp.mt));
  const int wmax = (int)std::min<long>(wcap, room / (rows * 128L));
  if (wmax < 1) return 0;
  return std::min(wmax, per);
}

// Waves per block and tiles per block of the half-tile kernel: two unit buffers per wave (halves_buf_rows) next to
// one or two 8 KB tables; `per` as tiles_width; every wave starts on a unit (at most 2 per waves). Returns 0 if no
// width fits.
int halves_width(const lw::FlatPlan& fp, int mintiles, int& per) {
  const int rows = lw::halves_buf_rows(fp), tables = (fp.n > 1 ? 2 : 1) * 4 * lw::LUTN;
  if (rows > 256) return 0;
  const int wmax = std::min(16, (160 * 1024 - tables) / (2 * rows * 128));
  if (wmax < 1) return 0;
  const int cus = cu_count();
  per = (fp.ntiles + cus - 1) / cus;
  if (fp.n > 1) per = std::min(per, mintiles);
  return std::min(wmax, 2 * per);
}

// Fused GEMV / skinny GEMM of `count` matrices with fp16 activations X16[i] ([m * per][K_i] pseudo-tokens):
// ring-capable matrices go into grouped launches (same K-quant type and ring size, up to MAX_GROUP per launch), the
// others into whole-tile launches. The ordered reduction over tile columns runs inside the flat (m = 1) launch for
// every matrix that launch decodes completely, else in one reduction launch per MAX_GROUP matrices. Partials of
// all matrices live side by side in the model's P scratch; calls that overlap on one model race (P and counters).
// `launches` (optional) counts the kernel launches. x8 (flat kernels only; m = 1, or up to 8 tokens in one pass with
// kernel modes 0, 3-5 and no packed matrix): int8 activations (quant_x8_dev) instead of X16.
int fused_group_dev(Model& M, Tensor* const* ts, const void* const* X16, int count, int m, int per, float* const* Y,
                    const int* ldy, hipStream_t s, int* launches = nullptr, const X8* x8 = nullptr,
                    const FixedScratch* fixed = nullptr) {
  const int mt = m * per;
  std::vector<size_t> off(count + 1, 0);
  for (int i = 0; i < count; ++i) off[i + 1] = off[i] + (size_t)ts[i]->dm.KT * mt * ts[i]->N;
  std::vector<size_t> coff(count + 1, 0);  // tile-row counters per entry (in-launch reduction)
  for (int i = 0; i < count; ++i) coff[i + 1] = coff[i] + 2 * (size_t)ts[i]->dm.NT;  // per tile row and half
  // partials and counters: the model's (grown on demand) or a caller's fixed scratch (nothing allocated; its counters
  // and partial slots are set by fill kernels on the stream, since the last call on that scratch may have left
  // anything there). Partial slots hold kNoPartial outside a reduction (lw_kernels.h).
  // 2..8 tokens of fp16 activations, every format: the whole-tile kernel with its products on the matrix cores
  auto mma_ok = [&](const lw::DevMat& dm) {
    return dm.kqt >= lw::KQ_Q4_K && dm.kqt <= lw::KQ_IQ4_XS && !dm.packed && dm.dsplit && dm.lut4 && dm.rows &&
           dm.max_rows + 2 <= 256;
  };
  const bool mma = !x8 && per == 1 && mt >= 2 && mt <= 8 && g_kernel_mode == 0;
  // its launches: matrices of one K-quant type, or of two (entries of the smaller type code first: one launch fewer),
  // up to MAX_GROUP each
  struct MmaLaunch {
    lw::FlatPlan fp;
    int tpb;
    std::vector<int> sel;
  };
  std::vector<MmaLaunch> mma_plans;
  if (mma) {
    std::vector<char> mdone(count, 0);
    for (;;) {  // two types per launch while two are left
      int ka = 0, kb = 0;
      for (int i = 0; i < count; ++i) {
        if (mdone[i] || !mma_ok(ts[i]->dm)) continue;
        const int k = ts[i]->dm.kqt;
        if (!ka) ka = k;
        else if (k != ka && !kb) kb = k;
      }
      if (!kb) break;
      if (kb < ka) std::swap(ka, kb);
      MmaLaunch L{};
      L.fp.mt = mt;
      int mintiles = 1 << 30;
      for (int pass = 0; pass < 2; ++pass)
        for (int j = 0; j < count && L.fp.n < lw::MAX_GROUP; ++j) {
          const lw::DevMat& dm = ts[j]->dm;
          if (mdone[j] || !mma_ok(dm) || dm.kqt != (pass ? kb : ka)) continue;
          if (!pass) ++L.fp.nfa;
          lw::FlatEntry& e = L.fp.e[L.fp.n++];
          e.M = dm;
          e.X2 = static_cast<const uint32_t*>(X16[j]);
          e.tile0 = L.fp.ntiles;
          e.ntile = dm.NT * dm.KT;
          e.Y = Y[j];
          e.ldy = ldy[j];
          L.fp.ntiles += e.ntile;
          mintiles = std::min(mintiles, e.ntile);
          L.sel.push_back(j);
        }
      if (L.fp.nfa == L.fp.n) break;  // the batch of MAX_GROUP holds one type only: the per-type launches take it
      L.fp.W = tiles_mma_width(L.fp, mintiles, L.tpb);
      if (L.fp.W < 1) break;
      for (int j : L.sel) mdone[j] = 1;
      mma_plans.push_back(std::move(L));
    }
    for (int i = 0; i < count; ++i) {
      if (mdone[i] || !mma_ok(ts[i]->dm)) continue;
      MmaLaunch L{};
      L.fp.mt = mt;
      int mintiles = 1 << 30;
      for (int j = i; j < count && L.fp.n < lw::MAX_GROUP; ++j) {
        const lw::DevMat& dm = ts[j]->dm;
        if (mdone[j] || !mma_ok(dm) || dm.kqt != ts[i]->dm.kqt) continue;
        lw::FlatEntry& e = L.fp.e[L.fp.n++];
        e.M = dm;
        e.X2 = static_cast<const uint32_t*>(X16[j]);
        e.tile0 = L.fp.ntiles;
        e.ntile = dm.NT * dm.KT;
        e.Y = Y[j];
        e.ldy = ldy[j];
        L.fp.ntiles += e.ntile;
        mintiles = std::min(mintiles, e.ntile);
        L.sel.push_back(j);
      }
      L.fp.W = tiles_mma_width(L.fp, mintiles, L.tpb);
      if (L.fp.W < 1) continue;
      for (int j : L.sel) mdone[j] = 1;
      mma_plans.push_back(std::move(L));
    }
  }
  float* Pb = nullptr;
  uint32_t* Cb = nullptr;
  if (fixed) {
    const size_t cnt_bytes = (coff[count] * sizeof(uint32_t) + 255) & ~(size_t)255;
    const size_t p_bytes = (off[count] * sizeof(float) + 255) & ~(size_t)255;
    const size_t need = cnt_bytes + p_bytes;
    if (need > fixed->bytes) {
      g_err = "scratch of " + std::to_string(fixed->bytes) + " bytes is too small: this call needs " +
              std::to_string(need);
      return -1;
    }
    Cb = reinterpret_cast<uint32_t*>(fixed->base);
    Pb = reinterpret_cast<float*>(fixed->base + cnt_bytes);
    HIPCHECK(lw::launch_fill_u32(Cb, coff[count], 0u, s));
    HIPCHECK(lw::launch_fill_u32(reinterpret_cast<uint32_t*>(Pb), off[count], lw::kNoPartial, s));
  } else {
    const size_t cap0 = M.P_cap;
    if (grow(M.P, M.P_cap, off[count] * sizeof(float))) return -1;
    if (M.P_cap != cap0)  // a new buffer: every slot empty (the reductions keep them so)
      HIPCHECK(lw::launch_fill_u32(reinterpret_cast<uint32_t*>(M.P), M.P_cap / sizeof(uint32_t), lw::kNoPartial, s));
    if (grow_zeroed(M.cnt, M.cnt_cap, coff[count] * sizeof(uint32_t))) return -1;
    Pb = M.P;
    Cb = M.cnt;
  }
  std::vector<char> reduced(count, 0);  // entries whose reduction runs inside their flat launch
  lw::GroupPlan plan{};
  plan.mt = mt;
  auto flush = [&]() -> int {
    if (plan.n) HIPCHECK(lw::launch_fused_group(plan, s));
    if (plan.n && launches) ++*launches;
    plan.n = 0;
    plan.blocks = 0;
    return 0;
  };
  const bool ring_ok = g_kernel_mode != 1;
  const bool one_pass = g_kernel_mode == 6 || g_kernel_mode == 9;  // modes taking int8 tokens one pass each
  const bool flat = ring_ok && g_kernel_mode != 2 && (mt == 1 || (x8 && mt <= 8 && !one_pass));
  if (x8 && !flat) {
    g_err = "int8 activations: a flat kernel mode (0, 3, 4, 5, 7, or 6 and 9 for m = 1) and at most 8 tokens only";
    return -1;
  }
  for (int i = 0; x8 && mt > 1 && i < count; ++i)
    if (ts[i]->dm.packed) {
      g_err = "int8 activations: packed matrices take one token per pass";
      return -1;
    }
  auto set8 = [&](lw::FlatPlan& fp, lw::FlatEntry& e, int j) {
    if (!x8) return;
    fp.i8 = 1;
    fp.mt = mt;
    e.XQ = x8[j].q;
    e.DX = x8[j].d;
    e.SX = x8[j].s;
    e.ldy = ldy[j];
  };
  // waves per CU of the flat kernel: fewer than 32 when the several-token kernel's registers allow fewer
  auto waves_cu = [&](const lw::DevMat& dm) {
    const int w = x8 && mt > 1 ? lw::flat_waves_per_cu(dm.kqt, dm.ring_rows, mt) : 32;
    return w > 0 ? w : 32;
  };
  // m = 1 (fp16 x): one flat launch (balanced blocks) per (K-quant type, ring size) and batch of MAX_GROUP
  // matrices, whatever their order: the ring kernel, or the low-latency kernel when the cost model favours it (few
  // tiles per CU) or a matrix has no ring schedule. In a 16-row ring launch, exception tiles with a 32-row schedule
  // are decoded in place in spare rings when those fit the LDS the launch's block width assumed.
  std::vector<char> done(count, 0), exc_in(count, 0), whole(count, 0);  // whole: every tile in a low-latency launch
  std::vector<lw::FlatPlan> flat_plans, split_plans;
  std::vector<std::pair<lw::FlatPlan, int>> tile_plans;  // whole-tile kernel launches and their tiles per block
  std::vector<std::pair<lw::FlatPlan, int>> half_plans;  // half-tile kernel launches and their tiles per block
  // packed (fixed-rate) matrices: the decode-free kernels, one launch per K-quant type and MAX_GROUP matrices
  // (m = 1: the flat one, which also reduces)
  for (int i = 0; mt == 1 && i < count; ++i) {
    if (done[i] || !ts[i]->dm.packed) continue;
    lw::FlatPlan fp{};
    int mintiles = 1 << 30;
    for (int j = i; j < count && fp.n < lw::MAX_GROUP; ++j) {
      const lw::DevMat& dm = ts[j]->dm;
      if (done[j] || !dm.packed || dm.kqt != ts[i]->dm.kqt) continue;
      lw::FlatEntry& e = fp.e[fp.n++];
      e.M = dm;
      e.X2 = static_cast<const uint32_t*>(X16[j]);
      set8(fp, e, j);
      e.P = Pb + off[j];
      e.tile0 = fp.ntiles;
      e.ntile = dm.NT * dm.KT;
      e.Y = Y[j];
      e.cnt = Cb + coff[j];
      fp.ntiles += e.ntile;
      mintiles = std::min(mintiles, e.ntile);
      reduced[j] = 1;
      done[j] = 1;
    }
    fp.W = flat_width(fp.ntiles, 16, mintiles, 0);
    HIPCHECK(lw::launch_fused_packed_flat(fp, s));
    if (launches) ++*launches;
  }
  for (int i = 0; i < count; ++i) {
    if (done[i] || !ts[i]->dm.packed) continue;
    lw::GroupPlan pp{};
    pp.mt = mt;
    for (int j = i; j < count && pp.n < lw::MAX_GROUP; ++j) {
      const lw::DevMat& dm = ts[j]->dm;
      if (done[j] || !dm.packed || dm.kqt != ts[i]->dm.kqt) continue;
      lw::GroupEntry& e = pp.e[pp.n++];
      e.M = dm;
      e.X2 = static_cast<const uint32_t*>(X16[j]);
      e.P = Pb + off[j];
      e.block0 = pp.blocks;
      pp.blocks += dm.KT * ((dm.NT + 15) / 16);
      done[j] = 1;
    }
    HIPCHECK(lw::launch_fused_packed(pp, s));
    if (launches) ++*launches;
  }
  // the matrix-core whole-tile launches: every tile of their matrices and the reduction in the launch (the ring
  // kernel for the other formats and kernel modes)
  for (MmaLaunch& L : mma_plans) {
    for (int k = 0; k < L.fp.n; ++k) {
      const int j = L.sel[k];
      L.fp.e[k].P = Pb + off[j];
      L.fp.e[k].cnt = Cb + coff[j];
      done[j] = reduced[j] = exc_in[j] = whole[j] = 1;
    }
    HIPCHECK(lw::launch_fused_tiles_mma(L.fp, L.tpb, s));
    if (launches) ++*launches;
  }
  // int8 activations, 2..8 tokens (kernel mode 0): the whole-tile kernel with its integer products on the matrix
  // cores, every format, one launch per K-quant type and MAX_GROUP matrices; the reduction in the launch
  for (int i = 0; x8 && mt >= 2 && mt <= 8 && g_kernel_mode == 0 && i < count; ++i) {
    auto ok8 = [&](const lw::DevMat& dm) { return !dm.packed && dm.dsplit && dm.luti8 && dm.rows && dm.max_rows + 2 <= 256; };
    if (done[i] || !ok8(ts[i]->dm)) continue;
    lw::FlatPlan fp{};
    std::vector<int> sel;
    int mintiles = 1 << 30;
    for (int j = i; j < count && fp.n < lw::MAX_GROUP; ++j) {
      const lw::DevMat& dm = ts[j]->dm;
      if (done[j] || !ok8(dm) || dm.kqt != ts[i]->dm.kqt) continue;
      lw::FlatEntry& e = fp.e[fp.n++];
      e.M = dm;
      set8(fp, e, j);
      e.P = Pb + off[j];
      e.tile0 = fp.ntiles;
      e.ntile = dm.NT * dm.KT;
      e.Y = Y[j];
      e.cnt = Cb + coff[j];
      fp.ntiles += e.ntile;
      mintiles = std::min(mintiles, e.ntile);
      sel.push_back(j);
    }
    int tpb = 0;
    fp.W = tiles_mma_width(fp, mintiles, tpb);  // (plan.i8: no x sums in LDS)
    if (fp.W < 1) continue;
    for (int j : sel) done[j] = reduced[j] = exc_in[j] = whole[j] = 1;
    HIPCHECK(lw::launch_fused_tiles_mma8(fp, tpb, s));
    if (launches) ++*launches;
  }
  // m = 1, fp16 x, kernel mode 0: matrices of two K-quant types in one whole-tile launch (entries of the smaller type
  // code first), one launch fewer than a launch per type (config 3's Q6_K down with IQ4_XS gate / up)
  auto tiles_ok = [&](const lw::DevMat& dm) {
    return dm.kqt >= lw::KQ_Q4_K && dm.kqt <= lw::KQ_IQ4_XS && !dm.packed && dm.dsplit && dm.mid && dm.lut4 &&
           dm.rows && dm.max_rows + 2 <= 256;
  };
  while (flat && mt == 1 && !x8 && g_kernel_mode == 0) {
    int ka = 0, kb = 0;
    for (int i = 0; i < count; ++i) {
      if (done[i] || !tiles_ok(ts[i]->dm)) continue;
      const int k = ts[i]->dm.kqt;
      if (!ka) ka = k;
      else if (k != ka && !kb) kb = k;
    }
    if (!kb) break;
    if (kb < ka) std::swap(ka, kb);
    std::vector<int> sel;
    for (int pass = 0; pass < 2; ++pass)
      for (int j = 0; j < count && (int)sel.size() < lw::MAX_GROUP; ++j)
        if (!done[j] && tiles_ok(ts[j]->dm) && ts[j]->dm.kqt == (pass ? kb : ka)) sel.push_back(j);
    lw::FlatPlan fp{};
    int mintiles = 1 << 30;
    for (int j : sel) {
      const lw::DevMat& dm = ts[j]->dm;
      if (dm.kqt == ka) ++fp.nfa;
      lw::FlatEntry& e = fp.e[fp.n++];
      e.M = dm;
      e.X2 = static_cast<const uint32_t*>(X16[j]);
      e.P = Pb + off[j];
      e.tile0 = fp.ntiles;
      e.ntile = dm.NT * dm.KT;
      e.Y = Y[j];
      e.cnt = Cb + coff[j];
      fp.ntiles += e.ntile;
      mintiles = std::min(mintiles, e.ntile);
    }
    if (fp.nfa == fp.n) break;  // the batch of MAX_GROUP holds one type only: the per-type launches take it
    int per = 0;
    fp.W = tiles_width(fp, mintiles, per);
    if (fp.W < 1) break;
    for (int j : sel) done[j] = reduced[j] = exc_in[j] = whole[j] = 1;
    tile_plans.emplace_back(fp, per);
  }
  for (int i = 0; flat && i < count; ++i) {
    if (done[i]) continue;
    const lw::DevMat& di = ts[i]->dm;
    std::vector<int> sel;
    for (int j = i; j < count && (int)sel.size() < lw::MAX_GROUP; ++j)
      if (!done[j] && ts[j]->dm.kqt == di.kqt && ts[j]->dm.ring_rows == di.ring_rows) sel.push_back(j);
    lw::FlatPlan fp{};
    int total = 0, mintiles = 1 << 30, nx = 0;
    for (int j : sel) {
      const lw::DevMat& dm = ts[j]->dm;
      lw::FlatEntry& e = fp.e[fp.n++];
      e.M = dm;
      e.X2 = static_cast<const uint32_t*>(X16[j]);
      set8(fp, e, j);
      e.P = Pb + off[j];
      e.list = nullptr;
      e.tile0 = total;
      e.ntile = dm.NT * dm.KT;
      total += dm.NT * dm.KT;
      mintiles = std::min(mintiles, dm.NT * dm.KT);
      nx += dm.nexc32;
      done[j] = 1;
    }
    fp.ntiles = total;
    if (mt == 1 && (g_kernel_mode == 0 || g_kernel_mode == 8) && !x8) {
      // the half-tile kernel (kernel mode 8; the m = 1 default with fp16 activations where the whole-tile kernel
      // would run fewer than 10 waves per block, i.e. few tiles per CU: half tiles keep more waves busy and balance
      // better; measured faster on config 1, equal on config 3, slower on config 2's 13 waves): every tile, the
      // reduction in the launch
      bool ok = true;
      for (int k = 0; k < fp.n; ++k) ok = ok && fp.e[k].M.hrow && fp.e[k].M.hsplit;
      if (ok && g_kernel_mode == 0) {
        int tper = 0;
        const int tw = tiles_width(fp, mintiles, tper);
        ok = tw < 10;
      }
      int hper = 0;
      fp.W = ok ? halves_width(fp, mintiles, hper) : 0;
      if (fp.W > 0) {
        for (int k = 0; k < fp.n; ++k) {
          fp.e[k].Y = Y[sel[k]];
          fp.e[k].cnt = Cb + coff[sel[k]];
          reduced[sel[k]] = exc_in[sel[k]] = whole[sel[k]] = 1;
        }
        half_plans.emplace_back(fp, hper);
        continue;
      }
    }
    if (mt == 1 && (g_kernel_mode == 0 || one_pass)) {
      // the whole-tile kernel (the m = 1 default: faster than the ring kernel on every configuration measured):
      // every tile, the reduction in the launch; the ring kernel where the tiles do not fit its LDS
      // kernel mode 9: codes looked up by the comparator form instead of the 2048-entry table (fp16 activations)
      fp.canon = g_kernel_mode == 9 && !x8;
      int rounds = 0;  // tiles per block
      fp.W = tiles_width(fp, mintiles, rounds);
      for (int k = 0; fp.W > 0 && fp.canon && k < fp.n; ++k)
        if (!fp.e[k].M.canon) {
          g_err = "kernel mode 9: a matrix's codes are not the canonical code of their lengths";
          return -1;
        }
      if (fp.W > 0) {
        for (int k = 0; k < fp.n; ++k) {
          fp.e[k].Y = Y[sel[k]];
          fp.e[k].cnt = Cb + coff[sel[k]];
          reduced[sel[k]] = exc_in[sel[k]] = whole[sel[k]] = 1;
        }
        tile_plans.emplace_back(fp, rounds);
        continue;
      }
    }
    bool split = !di.ring_rows || g_kernel_mode == 4;
    const int wcu = di.ring_rows ? waves_cu(di) : 32;
    if (!split && g_kernel_mode != 5) {
      const int w = flat_width(total, di.ring_rows, mintiles, 0, wcu);
      split = split_cost(total, lw::split_stage_rows(fp), di.kqt) <
              ring_cost(total, w, flat_lds(w, di.ring_rows, 0), wcu);
    }
    if (split) {  // every tile of these matrices, exceptions included; the reduction in the launch
      for (int k = 0; k < fp.n; ++k) {
        fp.e[k].Y = Y[sel[k]];
        fp.e[k].cnt = Cb + coff[sel[k]];
        reduced[sel[k]] = exc_in[sel[k]] = whole[sel[k]] = 1;
      }
      split_plans.push_back(fp);
      continue;
    }
    const int spare_ring = 2 * 16 * 128;
    fp.W = flat_width(total, di.ring_rows, mintiles, nx && di.ring_rows == 16 ? spare_ring : 0, wcu);
    if (nx && di.ring_rows == 16 && g_kernel_mode != 3) {
      // spare rings per block = the most 32-row exception tiles in one block (tile list position / W)
      std::map<int, int> per_block;
      int most = 0;
      for (int k = 0; k < fp.n; ++k) {
        const lw::DevMat& dm = fp.e[k].M;
        for (uint32_t t : ts[sel[k]]->exc32) {
          const int u = (int)(t % dm.KT) * dm.NT + (int)(t / dm.KT);
          most = std::max(most, ++per_block[(fp.e[k].tile0 + u) / fp.W]);
        }
      }
      // in place when the spare rings cost no more than the one spare ring the width was chosen with
      if (fp.W + most <= 32 && flat_cost(total, fp.W, flat_lds(fp.W, 16, most * spare_ring), wcu) <=
                                   flat_cost(total, fp.W, flat_lds(fp.W, 16, spare_ring), wcu)) {
        fp.nspare = most;
        for (int j : sel) exc_in[j] = 1;
      }
    }
    // the launch decodes every tile of a matrix without exceptions or with all of them in place: it also reduces
    for (int k = 0; k < fp.n; ++k) {
      const int j = sel[k];
      const lw::DevMat& dm = ts[j]->dm;
      if (dm.nexc && !(exc_in[j] && dm.nexc == dm.nexc32)) continue;
      fp.e[k].Y = Y[j];
      fp.e[k].cnt = Cb + coff[j];
      reduced[j] = 1;
    }
    flat_plans.push_back(fp);
  }
  // exception tiles not decoded in place, ahead of the ring launches on the same stream: those with a 32-row
  // schedule through the flat kernel (m = 1) in one-wave blocks, one launch per K-quant type; the rest through the
  // low-latency kernel (m = 1) or the whole-tile kernel (m > 1). (A second stream overlapped them with the ring launch
  // but its join cost more than the serial pass.)
  if (ring_ok) {
    std::vector<char> xdone(exc_in);
    for (int i = 0; flat && i < count; ++i) {
      if (xdone[i] || !ts[i]->dm.ring_rows || !ts[i]->dm.nexc32) continue;
      lw::FlatPlan fp{};
      for (int j = i; j < count && fp.n < lw::MAX_GROUP; ++j) {
        const lw::DevMat& dm = ts[j]->dm;
        if (xdone[j] || !dm.ring_rows || !dm.nexc32 || dm.kqt != ts[i]->dm.kqt) continue;
        lw::FlatEntry& e = fp.e[fp.n++];
        e.M = dm;
        e.M.ring_rows = 32;  // these tiles' schedules are for a 32-row ring
        e.X2 = static_cast<const uint32_t*>(X16[j]);
        set8(fp, e, j);
        e.P = Pb + off[j];
        e.list = dm.exc;
        e.tile0 = fp.ntiles;
        e.ntile = dm.nexc32;
        fp.ntiles += dm.nexc32;
        xdone[j] = 1;
      }
      fp.W = 1;
      HIPCHECK(lw::launch_fused_flat(fp, s));
      if (launches) ++*launches;
    }
    for (int i = 0; i < count; ++i) {
      const lw::DevMat& dm = ts[i]->dm;
      if (!dm.ring_rows || !dm.nexc || whole[i]) continue;
      lw::DevMat rest = dm;
      if (flat) {  // the flat launches took the first nexc32
        rest.exc = dm.exc + dm.nexc32;
        rest.nexc = dm.nexc - dm.nexc32;
      }
      if (!rest.nexc) continue;
      if (flat) {  // m = 1: the low-latency kernel over the list (the same bits as the ring kernels)
        lw::FlatPlan fp{};
        lw::FlatEntry& e = fp.e[fp.n++];
        e.M = dm;
        e.X2 = static_cast<const uint32_t*>(X16[i]);
        set8(fp, e, i);
        e.P = Pb + off[i];
        e.list = rest.exc;
        e.ntile = fp.ntiles = rest.nexc;
        HIPCHECK(lw::launch_fused_split(fp, s));
      } else {
        HIPCHECK(lw::launch_fused_exceptions(rest, X16[i], mt, Pb + off[i], s));
      }
      if (launches) ++*launches;
    }
  }
  for (const lw::FlatPlan& fp : flat_plans) {
    HIPCHECK(lw::launch_fused_flat(fp, s));
    if (launches) ++*launches;
  }
  for (const lw::FlatPlan& fp : split_plans) {
    HIPCHECK(lw::launch_fused_split(fp, s));
    if (launches) ++*launches;
  }
  for (const auto& tp : tile_plans) {
    HIPCHECK(lw::launch_fused_tiles(tp.first, tp.second, s));
    if (launches) ++*launches;
  }
  for (const auto& hp : half_plans) {
    HIPCHECK(lw::launch_fused_halves(hp.first, hp.second, s));
    if (launches) ++*launches;
  }
  for (int i = 0; i < count; ++i) {
    if (done[i]) continue;
    const lw::DevMat& di = ts[i]->dm;
    if (!ring_ok || di.ring_rows == 0) {
      HIPCHECK(lw::launch_fused(di, X16[i], mt, Pb + off[i], s));
      if (launches) ++*launches;
      done[i] = 1;
      continue;
    }
    for (int j = i; j < count; ++j) {
      const lw::DevMat& dm = ts[j]->dm;
      if (done[j] || dm.kqt != di.kqt || dm.ring_rows != di.ring_rows) continue;
      if (plan.n == lw::MAX_GROUP && flush()) return -1;
      lw::GroupEntry& e = plan.e[plan.n++];
      e.M = dm;
      e.X2 = static_cast<const uint32_t*>(X16[j]);
      e.P = Pb + off[j];
      e.block0 = plan.blocks;
      const int wpb = lw::group_waves_per_block(dm.ring_rows);
      plan.blocks += dm.KT * ((dm.NT + wpb - 1) / wpb);
      done[j] = 1;
    }
    if (flush()) return -1;
  }
  // ordered reduction over tile columns, up to MAX_GROUP matrices per launch
  lw::ReducePlan rp{};
  rp.m = m;
  rp.per = per;
  for (int i = 0; i < count; ++i) {
    if (reduced[i]) continue;
    lw::ReduceEntry& e = rp.e[rp.n++];
    e.P = Pb + off[i];
    e.Y = Y[i];
    e.N = (int)ts[i]->N;
    e.KT = ts[i]->dm.KT;
    e.ldy = ldy[i];
    e.out0 = rp.total;
    rp.total += m * (int)ts[i]->N;
    if (rp.n == lw::MAX_GROUP) {
      HIPCHECK(lw::launch_reduce_group(rp, s));
      if (launches) ++*launches;
      rp.n = 0;
      rp.total = 0;
    }
  }
  if (rp.n) {
    HIPCHECK(lw::launch_reduce_group(rp, s));
    if (launches) ++*launches;
  }
  return 0;
}

// lw_group_matmul_dev's work (fp16 x [m][K_i] per matrix): the fused path, after the quantization launch when int8
// activations are on (m = 1)
// Int8-activation matmuls of `count` matrices for m <= 8 tokens (x [m][K_i], fp16 or fp32, rows K_i apart; y rows
// ldy apart): one quantization launch, then one fused pass over the weights for all tokens (the reference's MT-token
// int8 kernel, kernels/llmrt.cu:1057-1169), which gives every token the bits of an m = 1 call. Packed matrices and
// kernel modes 6 and 9 take one m = 1 pass per token.
int act8_tokens(Model& M, Tensor* const* ts, const void* const* X, int x_f16, int count, int m, float* const* Y,
                const int* ldy, hipStream_t s, int* launches) {
  std::vector<X8> x8;
  bool one = m > 1 && g_kernel_mode != 6 && g_kernel_mode != 9;
  for (int i = 0; i < count; ++i) one = one && !ts[i]->dm.packed;
  if (one || m == 1) {
    if (quant_x8_dev(M, ts, X, x_f16, count, x8, s, m)) return -1;
    if (launches) ++*launches;
    return fused_group_dev(M, ts, X, count, m, 1, Y, ldy, s, launches, x8.data());
  }
  std::vector<const void*> xj(count);
  std::vector<float*> yj(count);
  for (int j = 0; j < m; ++j) {
    for (int i = 0; i < count; ++i) {
      xj[i] = static_cast<const char*>(X[i]) + (size_t)j * ts[i]->K * (x_f16 ? 2 : 4);
      yj[i] = Y[i] + (size_t)j * ldy[i];
    }
    if (quant_x8_dev(M, ts, xj.data(), x_f16, count, x8, s)) return -1;
    if (launches) ++*launches;
    if (fused_group_dev(M, ts, xj.data(), count, 1, 1, yj.data(), ldy, s, launches, x8.data())) return -1;
  }
  return 0;
}

int group_matmul(Model& M, Tensor* const* ts, const void* const* X, int count, int m, float* const* Y, const int* ldy,
                 hipStream_t s, int* launches = nullptr) {
  if (g_act8 && m <= 8) return act8_tokens(M, ts, X, 1, count, m, Y, ldy, s, launches);
  return fused_group_dev(M, ts, X, count, m, 1, Y, ldy, s, launches);
}

int fused_dev(Model& M, Tensor& t, const void* X16, int m, int per, float* Y, int ldy, hipStream_t s) {
  Tensor* tp = &t;
  return fused_group_dev(M, &tp, &X16, 1, m, per, &Y, &ldy, s);
}

// Prefill GEMM of path 2: 0 (default) = the hand-written MFMA GEMM over tiled codes for every K-quant format
// (k_gemm_prefill: scaled fp16 weights, Q4_K / Q5_K; k_gemm_prefill_sub: grid weights folded per sub-block, Q6_K /
// IQ4_XS); 1 = the older hand-written GEMM over row-major codes (k_gemm_codes_mfma, every format); 2 / 3 = rocBLAS,
// always the two-GEMM / the one-GEMM form over fp16 hi + lo weights; 4 = rocBLAS with the one-GEMM form up to
// g_prefill_one_max tokens, else two GEMMs. Kernel mode 1 keeps the SIMT GEMM.
int g_prefill = 0;

// Y[:, r0 : r0 + nr] = x . w^T for a chunk of rows through rocBLAS. WW is the column-major nr x 2K matrix [w hi |
// w lo] (ld nr), XX [m][2K] = [x hi | x hi] and XL [m][K] = x lo are the column-major 2K x m and K x m matrices of
// their transposes. Column-major view: Y^T (nr x m, ld ldy) = WW . XX over K' = 2K (x_hi w_hi + x_hi w_lo), then
// += WW[:, :K] . XL (x_lo w_hi).
int blas_chunk(Model& M, const uint16_t* WW, const uint16_t* XX, const uint16_t* XL, int nr, int m, int K, float* Y,
               int ldy) {
  const float one = 1.f, zero = 0.f;
  rocblas_status st = rocblas_gemm_ex(M.blas, rocblas_operation_none, rocblas_operation_none, nr, m, 2 * K, &one,
                                      WW, rocblas_datatype_f16_r, nr, XX, rocblas_datatype_f16_r, 2 * K, &zero, Y,
                                      rocblas_datatype_f32_r, ldy, Y, rocblas_datatype_f32_r, ldy,
                                      rocblas_datatype_f32_r, rocblas_gemm_algo_standard, 0, 0);
  if (st == rocblas_status_success)
    st = rocblas_gemm_ex(M.blas, rocblas_operation_none, rocblas_operation_none, nr, m, K, &one, WW,
                         rocblas_datatype_f16_r, nr, XL, rocblas_datatype_f16_r, K, &one, Y, rocblas_datatype_f32_r,
                         ldy, Y, rocblas_datatype_f32_r, ldy, rocblas_datatype_f32_r, rocblas_gemm_algo_standard, 0, 0);
  if (st != rocblas_status_success) {
    g_err = std::string("rocblas_gemm_ex: ") + rocblas_status_to_string(st);
    return -1;
  }
  return 0;
}

// The one-GEMM form for small m (memory-bound on the weights): T (column-major nr x 2m, ld nr) = WW . XB with XB the
// column-major 2K x 2m matrix of [x hi | x hi] (columns t < m) and [x lo | 0] (columns m + t): the weights are read
// once (4 B per weight instead of 6) and the launch has twice the output columns; a third of its products are with
// the zero half. Y[:, r0 : r0 + nr] = T[:m] + T[m:].
int blas_chunk_one(Model& M, const uint16_t* WW, const uint16_t* XB, int nr, int m, int K, float* Y, int ldy,
                   hipStream_t s) {
  const float one = 1.f, zero = 0.f;
  rocblas_status st = rocblas_gemm_ex(M.blas, rocblas_operation_none, rocblas_operation_none, nr, 2 * m, 2 * K, &one,
                                      WW, rocblas_datatype_f16_r, nr, XB, rocblas_datatype_f16_r, 2 * K, &zero, M.T32,
                                      rocblas_datatype_f32_r, nr, M.T32, rocblas_datatype_f32_r, nr,
                                      rocblas_datatype_f32_r, rocblas_gemm_algo_standard, 0, 0);
  if (st != rocblas_status_success) {
    g_err = std::string("rocblas_gemm_ex: ") + rocblas_status_to_string(st);
    return -1;
  }
  HIPCHECK(lw::launch_add_halves(M.T32, Y, m, nr, ldy, s));
  return 0;
}

// m up to this takes the one-GEMM form: measured faster at every m from 32 to 512 on a config-2 layer (0.76 vs
// 0.92 ms at m = 128, 1.38 vs 1.45 ms at m = 512); beyond, the third of its products that meet the zero half grows
// with m while the weight reads it saves do not
int g_prefill_one_max = 512;

// decode into scratch (tile-row chunks) + GEMM with the side bytes (path 2 / m > 8; llmrt.cu:1826-1841)
int decode_gemm_dev(Model& M, Tensor& t, const float* X, int m, float* Y, int ldy, hipStream_t s) {
  const bool kq = t.kqt >= lw::KQ_Q4_K && t.kqt <= lw::KQ_IQ4_XS;
  if (g_kernel_mode != 1 && g_prefill == 0 && kq && t.K % 256 == 0 && lw::decode_tiled_ok(t.dm)) {
    // the hand-written GEMM over tiled codes, x hi + lo (and, for the formats with mins, Sx hi + lo)
    const size_t row_bytes = (size_t)lw::TN * t.K;
    const size_t cap = std::max(row_bytes, std::min<size_t>((size_t)t.N * t.K, (size_t)64 << 20));
    if (grow(M.codes, M.codes_cap, cap) || grow(M.X16, M.X16_cap, lw::prefill_x_bytes(m, (int)t.K)) ||
        grow(M.SX, M.SX_cap, lw::prefill_sx_bytes(m, (int)t.K)))
      return -1;
    HIPCHECK(lw::launch_prefill_x(X, M.X16, M.SX, m, (int)t.K, s));
    const int rows_fit = (int)std::max<size_t>(1, M.codes_cap / row_bytes);
    for (int tr0 = 0; tr0 < t.dm.NT; tr0 += rows_fit) {
      const int tr1 = std::min(t.dm.NT, tr0 + rows_fit);
      HIPCHECK(lw::launch_decode_tiled(t.dm, M.codes, tr0, tr1, s));
      HIPCHECK(lw::launch_gemm_prefill(t.dm, M.codes, tr0 * lw::TN, (tr1 - tr0) * lw::TN, M.X16, M.SX, m, Y, ldy, s));
    }
    return 0;
  }
  const bool mfma = g_kernel_mode != 1 && g_prefill == 1;
  const bool blas = g_kernel_mode != 1 && !mfma;
  if (blas) {
    if (!M.blas && rocblas_create_handle(&M.blas) != rocblas_status_success) {
      M.blas = nullptr;
      g_err = "rocblas_create_handle failed";
      return -1;
    }
    if (rocblas_set_stream(M.blas, s) != rocblas_status_success) {
      g_err = "rocblas_set_stream failed";
      return -1;
    }
    // fp16 x: [m][2K] hi | hi, then [m][K] lo; weights [rows][2K] fp16 per chunk of tile rows (at most 256 MB)
    const size_t ww_row = (size_t)lw::TN * t.K * 4;
    const size_t cap = std::max(ww_row, std::min<size_t>((size_t)t.N * t.K * 4, (size_t)256 << 20));
    const bool one = g_prefill == 3 || ((g_prefill == 0 || g_prefill == 4) && m <= g_prefill_one_max);
    if (grow(M.X16, M.X16_cap, (size_t)(one ? 4 : 3) * m * t.K * 2) || grow(M.W16, M.W16_cap, cap)) return -1;
    if (one) HIPCHECK(lw::launch_split_x_gemm2(X, M.X16, m, (int)t.K, s));
    else HIPCHECK(lw::launch_split_x_gemm(X, M.X16, M.X16 + (size_t)2 * m * t.K, m, (int)t.K, s));
    const int rows_fit = (int)std::max<size_t>(1, M.W16_cap / ww_row);
    if (one && grow(M.T32, M.T32_cap, (size_t)2 * m * std::min<size_t>((size_t)rows_fit * lw::TN, t.N) * 4)) return -1;
    const bool fused = !t.dm.packed && t.dm.split;  // decode + dequant in one kernel
    if (!fused && grow(M.codes, M.codes_cap, (size_t)rows_fit * lw::TN * t.K)) return -1;
    for (int tr0 = 0; tr0 < t.dm.NT; tr0 += rows_fit) {
      const int tr1 = std::min(t.dm.NT, tr0 + rows_fit), nr = (tr1 - tr0) * lw::TN;
      if (fused) {
        HIPCHECK(lw::launch_decode_hilo(t.dm, tr0, tr1, M.W16, s));
      } else {
        HIPCHECK(lw::launch_decode(t.dm, M.codes, tr0, tr1, s));
        HIPCHECK(lw::launch_dequant_hilo(t.dm, M.codes, tr0 * lw::TN, nr, M.W16, s));
      }
      if (one ? blas_chunk_one(M, M.W16, M.X16, nr, m, (int)t.K, Y + (size_t)tr0 * lw::TN, ldy, s)
              : blas_chunk(M, M.W16, M.X16, M.X16 + (size_t)2 * m * t.K, nr, m, (int)t.K, Y + (size_t)tr0 * lw::TN, ldy))
        return -1;
    }
    return 0;
  }
  const size_t row_bytes = (size_t)lw::TN * t.K;
  const size_t cap = std::max(row_bytes, std::min<size_t>((size_t)t.N * t.K, (size_t)64 << 20));
  if (grow(M.codes, M.codes_cap, cap)) return -1;
  if (mfma) {
    if (grow(M.X16, M.X16_cap, (size_t)2 * m * t.K * 2)) return -1;
    HIPCHECK(lw::launch_split_x(X, M.X16, m, (int)t.K, s));
  }
  const int rows_fit = (int)std::max<size_t>(1, M.codes_cap / row_bytes);
  for (int tr0 = 0; tr0 < t.dm.NT; tr0 += rows_fit) {
    const int tr1 = std::min(t.dm.NT, tr0 + rows_fit);
    HIPCHECK(lw::launch_decode(t.dm, M.codes, tr0, tr1, s));
    if (mfma)
      HIPCHECK(lw::launch_gemm_codes_mfma(t.dm, M.codes, tr0 * lw::TN, (tr1 - tr0) * lw::TN, M.X16, m, Y, ldy, s));
    else
      HIPCHECK(lw::launch_gemm_codes(t.dm, M.codes, tr0 * lw::TN, (tr1 - tr0) * lw::TN, X, m, Y, ldy, s));
  }
  return 0;
}

// ── caller-allocation-free matmul: one static scratch array per device ──────────────────────────────────────
// lw_matmul_dev_noalloc keeps the partials, tile-row counters and split activations of its launches in `scratch`,
// which every GPU the library runs on holds from module load until the process ends. Host code never passes the
// array's name to a kernel (that is a host-side stand-in, not a device address): each device's copy is found once
// with hipGetSymbolAddress, with that device current (scratch_on_device, first called from rt_open), and only that
// address is used.
constexpr size_t kNoAllocScratchBytes = (size_t)16 << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];
std::mutex g_scratch_mu;
std::map<int, uint8_t*> g_scratch_addr;  // device -> address of its copy of `scratch`

uint8_t* scratch_on_device() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    g_err = "no current HIP device";
    return nullptr;
  }
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  const auto it = g_scratch_addr.find(dev);
  if (it != g_scratch_addr.end()) return it->second;
  void* p = nullptr;
  const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess || !p) {
    g_err = std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e);
    return nullptr;
  }
  g_scratch_addr[dev] = static_cast<uint8_t*>(p);
  return static_cast<uint8_t*>(p);
}

}  // namespace

// ── C-ABI ────────────────────────────────────────────────────────────────────────────────────────────────

extern "C" {

const char* lw_last_error(void) { return g_err.c_str(); }

void* rt_open(const char* dir, int max_ctx, int max_batch, long long budget_mb, int floor_mb, int verbose) {
  (void)max_ctx;
  (void)max_batch;
  g_err.clear();
  if (!dir) {
    fail("rt_open: null directory");
    return nullptr;
  }
  std::unique_ptr<Model> M(new Model());
  M->dir = dir;
  M->verbose = verbose;
  if (!parse_manifest(*M)) return nullptr;
  M->fd = open((M->dir + "/weights.bin").c_str(), O_RDONLY);
  if (M->fd < 0) {
    fail("cannot open " + M->dir + "/weights.bin");
    return nullptr;
  }
  struct stat st;
  if (fstat(M->fd, &st)) {
    fail("cannot stat weights.bin");
    release(M.release());
    return nullptr;
  }
  M->file_size = (uint64_t)st.st_size;
  if (!validate(*M)) {
    release(M.release());
    return nullptr;
  }
  const auto t0 = std::chrono::steady_clock::now();
  if (budget_mb != 0) {
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || ndev < 1) {
      (void)hipGetLastError();
      fail("rt_open: no GPU (open with budget_mb = 0 for CPU-only use)");
      release(M.release());
      return nullptr;
    }
    if (hipStreamCreateWithFlags(&M->stream, hipStreamNonBlocking) != hipSuccess) {
      fail("rt_open: stream creation failed");
      release(M.release());
      return nullptr;
    }
    M->gpu = true;
    // the no-allocation entry point's scratch on this device (its address, found once per device)
    if (!scratch_on_device()) {
      fail("rt_open: " + g_err);
      release(M.release());
      return nullptr;
    }
    const int threads = lw::default_threads();
    const long long floor_kb = (long long)floor_mb * 1024;
    size_t used = 0;
    for (auto& t : M->ts) {
      if (!t.matrix()) continue;
      if (budget_mb > 0 && used + t.nbytes > (size_t)budget_mb * 1048576ull) break;  // forward order: stop
      if (floor_mb > 0 && meminfo_kb("MemAvailable") - (long long)(t.nbytes >> 10) < floor_kb) break;
      if (!(t.packed() ? make_resident_packed(*M, t) : make_resident(*M, t, threads))) {
        release(M.release());
        return nullptr;
      }
      used += t.dev_bytes + t.side_bytes;
    }
  }
  M->avail_after_kb = meminfo_kb("MemAvailable");
  if (verbose)
    fprintf(stderr, "[lazyweights_amd] %s: %zu tensors, resident %.1f MB (coded %.1f MB, layout padding %.1f MB), "
                    "load %.2f s\n",
            dir, M->ts.size(), M->resident_bytes / 1e6, M->coded_bytes / 1e6, M->pad_bytes / 1e6,
            std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count());
  return M.release();
}

void rt_close(void* h) { release(static_cast<Model*>(h)); }

int rt_test_matmul(void* h, const char* name, const float* X, int m, float* Y, int path) {
  Model* M = static_cast<Model*>(h);
  if (!M || !X || !Y || m < 1) {
    g_err = "rt_test_matmul: bad arguments";
    return -1;
  }
  Tensor* t = M->find(name);
  if (check_matmul(t, name)) return -1;
  const size_t K = (size_t)t->K, N = (size_t)t->N;
  float *dx = nullptr, *dy = nullptr;
  void* dx16 = nullptr;
  int rc = 0;
  auto cleanup = [&]() {
    if (dx) (void)hipFree(dx);
    if (dy) (void)hipFree(dy);
    if (dx16) (void)hipFree(dx16);
  };
  if (hipMalloc(reinterpret_cast<void**>(&dy), (size_t)m * N * 4) != hipSuccess) {
    cleanup();
    g_err = "rt_test_matmul: device allocation failed";
    return -1;
  }
  if (g_act8 && m <= 8 && path != 2) {  // int8 activations quantized on the device from the fp32 x
    if (hipMalloc(reinterpret_cast<void**>(&dx), (size_t)m * K * 4) != hipSuccess ||
        hipMemcpy(dx, X, (size_t)m * K * 4, hipMemcpyHostToDevice) != hipSuccess) {
      cleanup();
      g_err = "rt_test_matmul: upload failed";
      return -1;
    }
    const void* xp = dx;
    float* yp = dy;
    const int ld = (int)N;
    rc = act8_tokens(*M, &t, &xp, 0, 1, m, &yp, &ld, M->stream, nullptr);
  } else if (m <= 8 && path != 2) {
    // fp32 activations as fp16 hi + lo pseudo-tokens (x = hi + lo to 2^-22 relative)
    std::vector<uint16_t> x16((size_t)2 * m * K);
    for (int j = 0; j < m; ++j)
      for (size_t k = 0; k < K; ++k) {
        const float x = X[(size_t)j * K + k];
        const uint16_t hi = lw::f32_to_f16(x);
        x16[(2 * j) * K + k] = hi;
        x16[(2 * j + 1) * K + k] = lw::f32_to_f16(x - lw::f16_to_f32(hi));
      }
    if (hipMalloc(&dx16, x16.size() * 2) != hipSuccess ||
        hipMemcpy(dx16, x16.data(), x16.size() * 2, hipMemcpyHostToDevice) != hipSuccess) {
      cleanup();
      g_err = "rt_test_matmul: upload failed";
      return -1;
    }
    rc = fused_dev(*M, *t, dx16, m, 2, dy, (int)N, M->stream);
  } else {
    if (hipMalloc(reinterpret_cast<void**>(&dx), (size_t)m * K * 4) != hipSuccess ||
        hipMemcpy(dx, X, (size_t)m * K * 4, hipMemcpyHostToDevice) != hipSuccess) {
      cleanup();
      g_err = "rt_test_matmul: upload failed";
      return -1;
    }
    rc = decode_gemm_dev(*M, *t, dx, m, dy, (int)N, M->stream);
  }
  if (rc == 0) {
    if (hipStreamSynchronize(M->stream) != hipSuccess ||
        hipMemcpy(Y, dy, (size_t)m * N * 4, hipMemcpyDeviceToHost) != hipSuccess) {
      g_err = std::string("rt_test_matmul: ") + hipGetErrorString(hipGetLastError());
      rc = -1;
    }
  }
  cleanup();
  return rc;
}

int lw_test_quant_x8(const void* X, int x_f16, int m, int K, int8_t* xq, float* dx, float* sx) {
  if (!X || !xq || !dx || !sx || m < 1 || K < 32 || K % 32) {
    g_err = "lw_test_quant_x8: bad arguments";
    return -1;
  }
  const size_t n = (size_t)m * K, nb = n / 32, xb = n * (x_f16 ? 2 : 4);
  uint8_t* d = nullptr;
  if (hipMalloc(reinterpret_cast<void**>(&d), xb + n + 8 * nb) != hipSuccess) {
    g_err = "lw_test_quant_x8: device allocation failed";
    return -1;
  }
  int8_t* q = reinterpret_cast<int8_t*>(d + xb);
  float* fd = reinterpret_cast<float*>(d + xb + n);
  int rc = 0;
  if (hipMemcpy(d, X, xb, hipMemcpyHostToDevice) != hipSuccess ||
      lw::launch_quant_x8(d, x_f16, m, K, q, fd, fd + nb, nullptr) != hipSuccess ||
      hipDeviceSynchronize() != hipSuccess || hipMemcpy(xq, q, n, hipMemcpyDeviceToHost) != hipSuccess ||
      hipMemcpy(dx, fd, nb * 4, hipMemcpyDeviceToHost) != hipSuccess ||
      hipMemcpy(sx, fd + nb, nb * 4, hipMemcpyDeviceToHost) != hipSuccess) {
    g_err = std::string("lw_test_quant_x8: ") + hipGetErrorString(hipGetLastError());
    rc = -1;
  }
  (void)hipFree(d);
  return rc;
}

int rt_test_decode(void* h, const char* name, uint8_t* out) {
  Model* M = static_cast<Model*>(h);
  if (!M || !out) {
    g_err = "rt_test_decode: bad arguments";
    return -1;
  }
  Tensor* t = M->find(name);
  if (!t) {
    g_err = std::string("no tensor ") + (name ? name : "(null)");
    return -1;
  }
  if (t->enc == "raw8") return pread_all(M->fd, out, t->nbytes, t->off) ? 0 : -1;
  if (!t->resident) {
    g_err = t->name + ": not resident";
    return -1;
  }
  uint8_t* d = nullptr;
  const size_t n = (size_t)t->N * t->K;
  HIPCHECK(hipMalloc(reinterpret_cast<void**>(&d), n));
  hipError_t e = lw::launch_decode(t->dm, d, 0, t->dm.NT, M->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(M->stream);
  if (e == hipSuccess) e = hipMemcpy(out, d, n, hipMemcpyDeviceToHost);
  (void)hipFree(d);
  if (e != hipSuccess) {
    g_err = std::string("rt_test_decode: ") + hipGetErrorString(e);
    return -1;
  }
  return 0;
}

double rt_gpu_decode_all(void* h, int reps) {
  Model* M = static_cast<Model*>(h);
  if (!M || !M->gpu || reps < 1) return -1;
  size_t need = 0;
  for (auto& t : M->ts)
    if (t.resident) need = std::max(need, std::min<size_t>((size_t)t.N * t.K, (size_t)256 << 20));
  if (!need || grow(M->codes, M->codes_cap, need)) return -1;
  hipEvent_t e0, e1;
  if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) return -1;
  std::vector<double> ts;
  for (int r = 0; r < reps; ++r) {
    (void)hipEventRecord(e0, M->stream);
    for (auto& t : M->ts) {
      if (!t.resident) continue;
      const size_t row_bytes = (size_t)lw::TN * t.K;
      const int rows_fit = (int)std::max<size_t>(1, M->codes_cap / row_bytes);
      for (int tr0 = 0; tr0 < t.dm.NT; tr0 += rows_fit)
        (void)lw::launch_decode(t.dm, M->codes, tr0, std::min(t.dm.NT, tr0 + rows_fit), M->stream);
    }
    (void)hipEventRecord(e1, M->stream);
    (void)hipEventSynchronize(e1);
    float ms = 0;
    (void)hipEventElapsedTime(&ms, e0, e1);
    ts.push_back(ms / 1e3);
  }
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  std::sort(ts.begin(), ts.end());
  return ts[ts.size() / 2];
}

int rt_test_cpu_decode(void* h, const char* name, int threads, uint8_t* out) {
  Model* M = static_cast<Model*>(h);
  if (!M || !out) return -1;
  Tensor* t = M->find(name);
  if (t && t->packed()) {  // the stored bytes are the symbols (kernels/llmrt.cu:2547)
    return pread_all(M->fd, out, (size_t)t->N * t->KS(), t->off) ? 0 : -1;
  }
  if (!t || !t->coded() || t->pre_il) {
    g_err = std::string(name ? name : "(null)") + ": not a raw coded tensor";
    return -1;
  }
  std::vector<uint8_t> blob(t->nbytes, 0);
  if (!pread_all(M->fd, blob.data(), t->nbytes, t->off)) return -1;
  std::string err;
  if (!lw::cpu_decode(blob.data(), blob.size(), (int)t->N, t->KS(), std::max(1, threads), out, nullptr, err)) {
    g_err = std::string(name) + ": " + err;
    return -1;
  }
  return 0;
}

double rt_cpu_decode_all(void* h, int threads, long long* symbols) {
  Model* M = static_cast<Model*>(h);
  if (!M) return -1;
  double total = 0;
  long long nsym = 0;
  std::vector<uint8_t> blob, out;
  for (auto& t : M->ts) {
    if (!t.coded() || t.pre_il) continue;
    blob.assign(t.nbytes, 0);
    if (!pread_all(M->fd, blob.data(), t.nbytes, t.off)) return -1;
    out.resize((size_t)t.N * t.KS());
    double s = 0;
    std::string err;
    if (!lw::cpu_decode(blob.data(), blob.size(), (int)t.N, t.KS(), std::max(1, threads), out.data(), &s, err)) {
      g_err = t.name + ": " + err;
      return -1;
    }
    total += s;
    nsym += (long long)t.N * t.KS();
  }
  if (symbols) *symbols = nsym;
  return total;
}

double rt_stat(void* h, const char* key) {
  Model* M = static_cast<Model*>(h);
  if (!M || !key) return -1;
  const std::string s(key);
  if (s == "resident_bytes") return (double)M->resident_bytes;
  if (s == "streamed_bytes" || s == "stream_wait_s" || s == "stream_bytes_moved" || s == "n_streamed" ||
      s == "graph_launches" || s == "graph_captures")
    return 0;
  if (s == "mem_available_mb") return M->avail_after_kb / 1024.0;
  if (s == "coded_bytes") return (double)M->coded_bytes;
  if (s == "device_bytes") return (double)M->device_bytes;
  if (s == "pad_bytes") return (double)M->pad_bytes;
  return -1;
}

int rt_forward(void* h, const int* ids, int n, float* logits, int all_logits) {
  (void)h;
  (void)ids;
  (void)n;
  (void)logits;
  (void)all_logits;
  g_err = "rt_forward: this library holds coded matrices only (no model runtime)";
  return -1;
}
void rt_reset(void* h) {
  if (h) static_cast<Model*>(h)->pos = 0;
}
void rt_set_window(void* h, int w) {
  if (h) static_cast<Model*>(h)->window = std::max(0, w);
}
void rt_set_pos(void* h, int p) {
  if (h) static_cast<Model*>(h)->pos = std::max(0, std::min(p, static_cast<Model*>(h)->pos));
}
int rt_pos(void* h) { return h ? static_cast<Model*>(h)->pos : 0; }
int rt_vocab(void* h) {
  (void)h;
  return 0;
}

int lw_tensor_info(void* h, const char* name, int64_t* out) {
  Model* M = static_cast<Model*>(h);
  if (!M || !out) return -1;
  Tensor* t = M->find(name);
  if (!t) {
    g_err = std::string("no tensor ") + (name ? name : "(null)");
    return -1;
  }
  out[0] = t->N;
  out[1] = t->K;
  out[2] = t->kqt;
  out[3] = t->symbits;
  out[4] = (int64_t)t->nbytes;
  out[5] = t->kqt ? (int64_t)M->ts[t->side_idx].nbytes : 0;
  out[6] = (int64_t)t->dev_bytes;
  out[7] = t->matrix() ? t->T() : 0;
  out[8] = t->resident ? 1 : 0;
  return 0;
}

int lw_matmul_dev(void* h, const char* name, const void* X, int x_f16, int m, float* Y, int ldy, void* stream) {
  Model* M = static_cast<Model*>(h);
  if (!M || !X || !Y) {
    g_err = "lw_matmul_dev: bad arguments";
    return -1;
  }
  Tensor* t = M->find(name);
  if (check_matmul(t, name)) return -1;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (g_act8 && m >= 1 && m <= 8) return act8_tokens(*M, &t, &X, x_f16, 1, m, &Y, &ldy, s, nullptr);
  if (x_f16) {
    if (m < 1 || m > 16) {
      g_err = "lw_matmul_dev: fp16 activations need 1 <= m <= 16";
      return -1;
    }
    return fused_dev(*M, *t, X, m, 1, Y, ldy, s);
  }
  if (m < 1) {
    g_err = "lw_matmul_dev: m < 1";
    return -1;
  }
  if (m > 8) return decode_gemm_dev(*M, *t, static_cast<const float*>(X), m, Y, ldy, s);  // prefill shapes
  if (grow(M->X16, M->X16_cap, (size_t)2 * m * t->K * 2)) return -1;
  HIPCHECK(lw::launch_split_x(static_cast<const float*>(X), M->X16, m, (int)t->K, s));
  return fused_dev(*M, *t, M->X16, m, 2, Y, ldy, s);
}

int lw_matmul_dev_noalloc(void* h, const char* name, const void* X, int x_f16, int m, float* Y, int ldy,
                          void* stream) {
  Model* M = static_cast<Model*>(h);
  if (!M || !X || !Y) {
    g_err = "lw_matmul_dev_noalloc: bad arguments";
    return -1;
  }
  Tensor* t = M->find(name);
  if (check_matmul(t, name)) return -1;
  if (g_act8) {
    g_err = "lw_matmul_dev_noalloc: int8 activations are not supported (lw_set_act8(0) first)";
    return -1;
  }
  if (x_f16 ? (m < 1 || m > 16) : (m < 1 || m > 8)) {
    g_err = "lw_matmul_dev_noalloc: needs 1 <= m <= 16 with fp16 activations, 1 <= m <= 8 with fp32";
    return -1;
  }
  uint8_t* base = scratch_on_device();
  if (!base) return -1;
  hipStream_t s = static_cast<hipStream_t>(stream);
  FixedScratch fx{base, kNoAllocScratchBytes};
  const void* X16 = X;
  int per = 1;
  if (!x_f16) {  // fp32 x split into fp16 hi + lo rows, at the end of the scratch
    const size_t xb = ((size_t)2 * m * t->K * sizeof(uint16_t) + 255) & ~(size_t)255;
    if (xb >= fx.bytes) {
      g_err = "lw_matmul_dev_noalloc: activations exceed the " + std::to_string(kNoAllocScratchBytes) +
              "-byte scratch";
      return -1;
    }
    fx.bytes -= xb;
    void* x16 = base + fx.bytes;
    HIPCHECK(lw::launch_split_x(static_cast<const float*>(X), x16, m, (int)t->K, s));
    X16 = x16;
    per = 2;
  }
  const int rc = fused_group_dev(*M, &t, &X16, 1, m, per, &Y, &ldy, s, nullptr, nullptr, &fx);
  if (rc) g_err = "lw_matmul_dev_noalloc: " + g_err;
  return rc;
}

int lw_group_matmul_dev(void* h, int count, const char* const* names, const void* const* X, int m,
                        float* const* Y, void* stream) {
  Model* M = static_cast<Model*>(h);
  if (!M || count < 1 || !names || !X || !Y || m < 1 || m > 16) {
    g_err = "lw_group_matmul_dev: bad arguments";
    return -1;
  }
  std::vector<Tensor*> ts(count);
  std::vector<int> ldy(count);
  for (int i = 0; i < count; ++i) {
    ts[i] = M->find(names[i]);
    if (check_matmul(ts[i], names[i])) return -1;
    if (!X[i] || !Y[i]) {
      g_err = "lw_group_matmul_dev: null buffer";
      return -1;
    }
    ldy[i] = (int)ts[i]->N;
  }
  return group_matmul(*M, ts.data(), X, count, m, Y, ldy.data(), static_cast<hipStream_t>(stream));
}

int lw_set_act8(int on) {
  if (on != 0 && on != 1) return -1;
  g_act8 = on;
  return 0;
}

int lw_set_kernel_mode(int mode) {
  if (mode < 0 || mode > 9) return -1;
  g_kernel_mode = mode;
  return 0;
}

int lw_set_prefill_gemm(int which) {
  if (which < 0 || which > 4) return -1;
  g_prefill = which;
  return 0;
}

int lw_bench_groups(void* h, int ngroups, const int* sizes, const char* const* names, const void* const* X, int m,
                    float* const* Y, int warmup, int iters, double* out) {
  Model* M = static_cast<Model*>(h);
  if (!M || ngroups < 1 || !sizes || !out || iters < 1) {
    g_err = "lw_bench_groups: bad arguments";
    return -1;
  }
  std::vector<int> first(ngroups + 1, 0);
  for (int g = 0; g < ngroups; ++g) first[g + 1] = first[g] + sizes[g];
  hipStream_t s = M->stream;
  for (int w = 0; w < warmup; ++w)
    for (int g = 0; g < ngroups; ++g)
      if (lw_group_matmul_dev(h, sizes[g], names + first[g], X + first[g], m, Y + first[g], s)) return -1;
  HIPCHECK(hipStreamSynchronize(s));
  hipEvent_t a, b;
  HIPCHECK(hipEventCreate(&a));
  HIPCHECK(hipEventCreate(&b));
  HIPCHECK(hipEventRecord(a, s));
  for (int it = 0; it < iters; ++it)
    for (int g = 0; g < ngroups; ++g)
      if (lw_group_matmul_dev(h, sizes[g], names + first[g], X + first[g], m, Y + first[g], s)) return -1;
  HIPCHECK(hipEventRecord(b, s));
  HIPCHECK(hipEventSynchronize(b));
  float ms = 0;
  HIPCHECK(hipEventElapsedTime(&ms, a, b));
  // the groups' launches alone: events around each pass of them (an event between two launches costs the stream
  // about 2 us, so not one around each group), host work excluded. The passes are enqueued back to back and
  // synchronized once, and the first is not counted: with the stream idle, its start event would be reached while
  // the host still plans the first launch
  const int kit = std::max(1, std::min(iters, 20));
  std::vector<hipEvent_t> ev(2 * (size_t)(kit + 1));
  for (auto& e : ev) HIPCHECK(hipEventCreate(&e));
  double kms = 0;
  int launches = 0;
  std::vector<int> ldys(first[ngroups]);
  for (int i = 0; i < first[ngroups]; ++i) {
    Tensor* t = M->find(names[i]);
    if (!t) {
      g_err = std::string("lw_bench_groups: unknown tensor ") + (names[i] ? names[i] : "(null)");
      return -1;
    }
    ldys[i] = (int)t->N;
  }
  for (int it = 0; it <= kit; ++it) {
    HIPCHECK(hipEventRecord(ev[2 * it], s));
    for (int g = 0; g < ngroups; ++g) {
      std::vector<Tensor*> ts;
      for (int i = first[g]; i < first[g + 1]; ++i) ts.push_back(M->find(names[i]));
      int nl = 0;
      if (group_matmul(*M, ts.data(), X + first[g], sizes[g], m, Y + first[g], ldys.data() + first[g], s, &nl))
        return -1;
      if (it == 0) launches += nl;
    }
    HIPCHECK(hipEventRecord(ev[2 * it + 1], s));
  }
  HIPCHECK(hipEventSynchronize(ev.back()));
  for (int it = 1; it <= kit; ++it) {
    float k = 0;
    HIPCHECK(hipEventElapsedTime(&k, ev[2 * it], ev[2 * it + 1]));
    kms += k;
  }
  for (auto& e : ev) (void)hipEventDestroy(e);
  (void)hipEventDestroy(a);
  (void)hipEventDestroy(b);
  out[0] = ms / iters;
  out[1] = kms / kit;
  out[2] = launches;
  return 0;
}

double lw_stream_read_gbps(long long bytes, int reps) {
  if (bytes < (1 << 20) || reps < 1) return -1;
  void* buf = nullptr;
  float* out = nullptr;
  const int blocks = 256 * 16;
  if (hipMalloc(&buf, (size_t)bytes) != hipSuccess) return -1;
  if (hipMalloc(reinterpret_cast<void**>(&out), (size_t)blocks * 256 * 4) != hipSuccess) {
    (void)hipFree(buf);
    return -1;
  }
  (void)hipMemset(buf, 1, (size_t)bytes);
  hipEvent_t a, b;
  (void)hipEventCreate(&a);
  (void)hipEventCreate(&b);
  std::vector<double> r;
  const size_t n16 = (size_t)bytes / 16;
  (void)lw::launch_stream_read(buf, n16, out, blocks, nullptr);
  for (int i = 0; i < reps; ++i) {
    (void)hipEventRecord(a, nullptr);
    (void)lw::launch_stream_read(buf, n16, out, blocks, nullptr);
    (void)hipEventRecord(b, nullptr);
    (void)hipEventSynchronize(b);
    float ms = 0;
    (void)hipEventElapsedTime(&ms, a, b);
    r.push_back(n16 * 16.0 / (ms * 1e-3) / 1e9);
  }
  (void)hipEventDestroy(a);
  (void)hipEventDestroy(b);
  (void)hipFree(buf);
  (void)hipFree(out);
  std::sort(r.begin(), r.end());
  return r[r.size() / 2];
}

}  // extern "C"
