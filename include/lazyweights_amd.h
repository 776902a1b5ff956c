/* lazyweights_amd — C-ABI of the MI355X-native decode-on-demand weight path.
 *
 * Drop-in for the reference runtime's matmul/decode exports (kernels/llmrt.cu extern "C" block, lines 1916-2575):
 * same names, argument meaning and return codes. Host buffers are caller-owned; the handle is opaque and owned
 * by the library until rt_close. Not thread-safe per handle (as the reference).
 *
 * Accepted bundles: a directory with manifest.txt + weights.bin (lazyweights/bundle.py:10-21). Coded matrices
 * enc huf8 / huf4p (and the reference's pre-interleaved huf8_il / huf8_ilc / huf4p_il / huf4p_ilc exports), each
 * with a K-quant side tensor <name>.kqs (enc kq_Q4_K | kq_Q5_K | kq_Q6_K | kq_IQ4_XS) for the fused GEMV.
 * Matrix-only bundles (no model cfg keys) open. Errors never exit the process: functions return nullptr / -1 and
 * lw_last_error() describes the failure.
 */
#ifndef LAZYWEIGHTS_AMD_H
#define LAZYWEIGHTS_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ── reference-compatible entry points ─────────────────────────────────────────────────────────────────── */

/* Replaces rt_open (kernels/llmrt.cu:1921). Opens a bundle; coded matrices are re-laid out for the GPU and made
 * resident while budget_mb (< 0: unlimited) and the host MemAvailable floor (floor_mb) allow. budget_mb == 0 keeps
 * everything on the host: no GPU is touched, CPU entry points still work. max_ctx / max_batch are accepted and
 * ignored (no model runtime). Returns nullptr on a missing or malformed manifest / weights.bin. */
void* rt_open(const char* dir, int max_ctx, int max_batch, long long budget_mb, int floor_mb, int verbose);

/* Replaces rt_close (kernels/llmrt.cu:2239). */
void rt_close(void* h);

/* Replaces rt_test_matmul (kernels/llmrt.cu:2441): Y[m, N] = X[m, K] @ dequant(W)^T for tensor `name`, host X (fp32)
 * and host Y. path 0 = auto (fused if m <= 8), 1 = fused, 2 = decode into scratch + GEMM. Returns 0, or -1 when the
 * tensor is missing, not resident or not a K-quant coded matrix. */
int rt_test_matmul(void* h, const char* name, const float* X, int m, float* Y, int path);

/* Replaces rt_test_decode (kernels/llmrt.cu:2461): GPU decode to host codes [N, K] (one byte per weight, pair
 * symbols unpacked low nibble first, no add for K-quants); raw8 tensors are copied. -1 if not resident. */
int rt_test_decode(void* h, const char* name, uint8_t* out);

/* Replaces rt_gpu_decode_all (kernels/llmrt.cu:2482): GPU decode of every resident coded matrix; median seconds of
 * `reps` event-timed passes. */
double rt_gpu_decode_all(void* h, int reps);

/* Replaces rt_test_cpu_decode (kernels/llmrt.cu:2543): CPU decode of the raw blob to symbols [N, KS]
 * (KS = K / 2 for huf4p), `threads` workers. -1 for pre-interleaved or non-coded tensors. */
int rt_test_cpu_decode(void* h, const char* name, int threads, uint8_t* out);

/* Replaces rt_cpu_decode_all (kernels/llmrt.cu:2558): CPU decode of every coded matrix, blobs read first (untimed);
 * returns decode seconds, *symbols = symbols decoded. */
double rt_cpu_decode_all(void* h, int threads, long long* symbols);

/* Replaces rt_stat (kernels/llmrt.cu:2276). Keys of the reference: resident_bytes, streamed_bytes, stream_wait_s,
 * stream_bytes_moved, mem_available_mb, n_streamed, graph_launches, graph_captures; plus coded_bytes (algorithmic
 * bytes of the resident coded matrices: blob + side tensor), device_bytes (their device layout), pad_bytes
 * (device layout bytes beyond the blob payload). Unknown keys: -1. */
double rt_stat(void* h, const char* key);

/* Model-runtime entries of the reference (kernels/llmrt.cu:2269-2291). This library holds matrices, not a model:
 * rt_forward returns -1; rt_vocab returns 0; the others keep a position counter only. */
int rt_forward(void* h, const int* ids, int n, float* logits, int all_logits);
void rt_reset(void* h);
void rt_set_window(void* h, int w);
void rt_set_pos(void* h, int p);
int rt_pos(void* h);
int rt_vocab(void* h);

/* ── extensions (no counterpart in the reference) ──────────────────────────────────────────────────────── */

/* Last error message of the calling thread ("" if none). */
const char* lw_last_error(void);

/* Shape and byte counts of a tensor: out[0] N, out[1] K, out[2] kqt (0 none, 1 Q4_K, 2 Q5_K, 3 Q6_K, 4 IQ4_XS),
 * out[3] symbol bits (4 or 8), out[4] blob bytes, out[5] side bytes, out[6] device layout bytes, out[7] tiles,
 * out[8] resident (0/1). Returns -1 if absent. */
int lw_tensor_info(void* h, const char* name, int64_t* out);

/* Device-pointer GEMV / skinny GEMM on `stream` (a hipStream_t; NULL = the null stream), no host copies, no
 * synchronisation: Y[m, N] (row stride ldy) = X[m, K] @ dequant(W)^T. X is fp16 (x_f16 = 1, the headline path,
 * m <= 16) or fp32 (x_f16 = 0: split into fp16 hi + lo; m <= 8 fused, any larger m the prefill path: decode into a
 * device scratch and GEMMs on the matrix cores, as rt_test_matmul's path 2, see lw_set_prefill_gemm). Returns 0 or
 * -1. */
int lw_matmul_dev(void* h, const char* name, const void* X, int x_f16, int m, float* Y, int ldy, void* stream);

/* lw_matmul_dev without any device allocation. No counterpart in the reference: it is for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). The launches' partials,
 * tile-row counters and (fp32 x) split activations live in a static 16 MiB device array held by every GPU the library
 * runs on until the process ends; the counters are cleared by a kernel on `stream` at each call. Fused path only:
 * fp16 X with 1 <= m <= 16 or fp32 X with 1 <= m <= 8, int8 activations off; -1 with an error text when the call
 * needs more than the 16 MiB (KT * m * N * 4 bytes of partials, 8 with fp32 X, + 8 * N / 64 of counters + 4 m K of
 * split x). Calls that overlap on one GPU (several streams or threads) race on the array. */
int lw_matmul_dev_noalloc(void* h, const char* name, const void* X, int x_f16, int m, float* Y, int ldy,
                          void* stream);

/* Several independent matmuls (e.g. the matrices of one decoder layer), each with its own fp16 activations X[i]
 * [m, K_i] and output Y[i] [m, N_i], launched back to back on `stream`. Returns 0 or -1. */
int lw_group_matmul_dev(void* h, int count, const char* const* names, const void* const* X, int m,
                        float* const* Y, void* stream);

/* Fused-kernel selection for all handles. 0 (default): m = 1 with fp16 activations, the whole-tile kernel (a tile
 * per wave copied to LDS, 8 chains per lane, every tile including exception tiles), or the half-tile kernel (two
 * buffered half-tile units per wave, the next one's copy in flight while one decodes) where the whole-tile kernel's
 * blocks would have fewer than 10 waves (few tiles per CU); m = 1 with int8 activations, the whole-tile kernel;
 * 2 <= m <= 8 with fp16 or int8 activations and every format, the whole-tile
 * kernel with its products on the matrix cores; otherwise the ring-staged kernels wherever a matrix has a ring
 * schedule (the block-per-column kernel). 1 = the whole-tile fallback kernel everywhere; 2 = the block-per-column ring
 * kernel for every m; 7 = the ring-staged kernels for every m (for m = 1 the flat, load-balanced ring kernel);
 * 3 = as 7, but exception tiles are never decoded inside the flat launch (always by the separate exception pass);
 * 4 = as 7, with the low-latency kernel (8 chains per lane) for every m = 1 launch; 5 = as 7, never the low-latency
 * kernel; 6 = as 0, but m = 1 always through the whole-tile kernel and int8 activations one m = 1 pass per token;
 * 8 = as 0, but m = 1 with fp16 activations always through the half-tile kernel; 9 = as 6, with the whole-tile
 * kernel (m = 1, fp16 activations) looking each code up by the comparator over the canonical code's per-length
 * limits (the reference's hw/huff/huff_engine.h:54-77 lookup) and a 256-entry table in canonical order instead of
 * the 2048-entry table: the same bits, about 3x slower (returns -1 for a matrix whose codes are not the canonical
 * code of their lengths). Returns 0 or -1. */
int lw_set_kernel_mode(int mode);

/* Prefill GEMM (path 2, and fp32 X with m > 8) for every handle. The reference dequantizes to fp32 and runs its own
 * fp32 GEMM (kernels/llmrt.cu:201-343, 1826-1841). 0 (default) = the hand-written matrix-core GEMM for Q4_K / Q5_K
 * (codes decoded to a device scratch, each scaled by its 6-bit sub-block scale into an exact fp16 weight, x split into
 * fp16 hi + lo, v_mfma_f32_32x32x16_f16 with fp32 accumulation, super-block scales and mins applied in registers) and
 * rocBLAS for Q6_K / IQ4_XS; 1 = hand-written for every format (Q6_K / IQ4_XS through a per-sub-block-scaled MFMA
 * GEMM); 2 / 3 = rocBLAS always, over the decoded weights w = s f(q) - o split into fp16 hi + lo (two fp16 GEMMs with
 * fp32 accumulation, x_hi w_hi + x_hi w_lo, then + x_lo w_hi / one GEMM over 2m columns [x_hi | x_hi] and [x_lo | 0]);
 * 4 = rocBLAS with the one-GEMM form up to 512 tokens. Kernel mode 1 overrides all with the SIMT GEMM. Returns 0 or
 * -1. */
int lw_set_prefill_gemm(int which);

/* Int8 activations for 1 <= m <= 8 (on = 1; default 0 = fp16 hi + lo activations): rt_test_matmul, lw_matmul_dev
 * and lw_group_matmul_dev quantize x per block of 32 (d = max|x| / 127, q = x / d rounded to nearest even, plus
 * d sum q) and the fused kernels take integer dot products per sub-block, y += s d acc - o d sum q. Replaces the
 * reference's act8 switch (kernels/llmrt.cu:2221, LLMRT_FP_ACT; kernels k_quant_x8 / k_gemvm_kq8 at
 * kernels/llmrt.cu:1035-1169), which is on by default there. m > 1 runs one pass over the weights for all tokens:
 * with kernel mode 0 on the matrix cores (each token within fp32 rounding of its m = 1 result), with modes 3, 4, 5
 * and 7 by the ring kernels (the same bits per token as an m = 1 call); with kernel mode 6 or a packed matrix, one
 * m = 1 pass per token. Needs kernel mode 0, 3, 4, 5, 6, 7 or 9 (as 6). Returns 0 or -1. */
int lw_set_act8(int on);

/* The int8 quantization of lw_set_act8 on host buffers (test entry, runs the device kernel): X [m, K] fp32 or fp16
 * (x_f16) -> xq [m, K] int8, dx [m, K / 32] = max|x| / 127 per block, sx [m, K / 32] = dx * sum of the block's q
 * (kernels/llmrt.cu:1035-1055). Returns 0 or -1. */
int lw_test_quant_x8(const void* X, int x_f16, int m, int K, int8_t* xq, float* dx, float* sx);

/* Times `iters` repetitions (after `warmup`) of lw_group_matmul_dev over `ngroups` groups laid out back to back in
 * names/X/Y (group g has sizes[g] matrices), cycling through the groups, with HIP events on the launch stream.
 * out[0] = mean ms per pass over all groups, out[1] = mean ms per pass of the groups' kernels alone (events around
 * each pass of the groups' launches, host work excluded: min(iters, 20) passes enqueued back to back after one that
 * is not counted), out[2] = number of kernel launches per pass. */
int lw_bench_groups(void* h, int ngroups, const int* sizes, const char* const* names, const void* const* X, int m,
                    float* const* Y, int warmup, int iters, double* out);

/* Achievable HBM read bandwidth (GB/s): streaming 16-byte reads over `bytes` of device memory, median of reps. */
double lw_stream_read_gbps(long long bytes, int reps);

/* Synthetic data and bundles (test / bench inputs). */
/* codes [N, K] (one byte per weight) and side bytes [N, K / 256 * SB]; seeded; independent of `threads`. */
int lw_synth_matrix(int kqt, int N, int K, double entropy, uint64_t seed, uint8_t* codes, uint8_t* side, int threads);
/* codes -> symbols [N, KS] (pairs for Q4_K / IQ4_XS). */
int lw_form_symbols(int kqt, const uint8_t* codes, int N, int K, uint8_t* sym);
/* Encode symbols [N, KS] as a huf8/huf4p blob (lazyweights/bundle.py:57-85). Returns the blob size; writes it
 * to `blob` when cap is large enough; *bits = payload bits. -1 on bad shapes. */
long long lw_encode(const uint8_t* sym, int N, int KS, uint8_t* blob, long long cap, uint64_t* bits);
/* Incremental bundle-directory writer (the format of lazyweights/bundle.py:10-21, 114-136: weights.bin with every
 * tensor at a 256-byte boundary, manifest.txt with `cfg <key> <value>` and
 * `t <name> <enc> <N> <K> <scale> <zp> <offset> <nbytes>` lines). lw_bundle_create returns NULL if the directory
 * cannot be written. Names, encodings, keys and values are single words (no white space): lw_bundle_cfg /
 * lw_bundle_add return -1 and write nothing otherwise. lw_bundle_finish writes the manifest, frees the handle and
 * returns 0, or -1 if any file write failed. */
void* lw_bundle_create(const char* dir);
int lw_bundle_cfg(void* w, const char* key, const char* value);
int lw_bundle_add(void* w, const char* name, const char* enc, long long N, long long K, double scale, int zp,
                  const void* data, long long nbytes);
int lw_bundle_finish(void* w);
/* Write a bundle directory of `count` synthetic K-quant matrices (each with its .kqs side tensor). */
int lw_write_bundle(const char* dir, int count, const char* const* names, const int* kqts, const int* Ns,
                    const int* Ks, const double* entropies, const uint64_t* seeds, int threads);

/* Huffman code lengths of a histogram (n <= 256 symbols): lmax > 0 gives the length-limited lengths of
 * lazyweights/lanecodecs.py:28-38, lmax <= 0 the plain heap lengths of lazyweights/huffman.py:8-26. */
int lw_huffman_lengths(const int64_t* hist, int n, int lmax, uint8_t* L);

/* The comparator table kernel mode 9 looks codes up in (built at load time for every K-quant matrix; host-side, for
 * tests): from a bundle decode table lut [2048] (sym | len << 8) and K-quant type kqt (1..4), out [288] = the limits
 * of code lengths 1..10 (a window value v of 11 bits, first code bit most significant, holds a code longer than k
 * when v >= out[k - 1]), for l = 1..11 out[9 + l] = (4 (base_l - first_l)) << 16 | (11 - l), and out[32 ..] the
 * kernels' table entries of the symbols in canonical order; the reference builds the same limits / first / base in
 * hw/huff/huff_engine.h:39-52 (build_canon). Returns 0, or -1 when the table's codes are not the canonical code of
 * their lengths (or bad arguments). */
int lw_canon_table(int kqt, const uint16_t* lut, uint32_t* out);

/* The device layout this library builds from a blob at load time (host-side, for inspection and tests): fills tbase
 * [T], mid [T * 32], split [T * 16 * 32] (bit offsets of symbols 32 k per lane: the chain starts of the
 * low-latency and whole-tile kernels), rows [T], sched [2 T] (ring staging schedule), *ring_rows and, when words_cap is large enough, words;
 * returns the word count (-1 on a bad or corrupt blob). Any output pointer may be NULL. pre_il / compact select the
 * reference's pre-interleaved export formats (_il / _ilc). */
long long lw_build_layout(const uint8_t* blob, long long len, int N, int KS, int pre_il, int compact, uint32_t* tbase,
                          uint16_t* mid, uint16_t* split, uint16_t* rows, uint64_t* sched, int* ring_rows,
                          uint32_t* words, long long words_cap);

#ifdef __cplusplus
}
#endif

#endif /* LAZYWEIGHTS_AMD_H */
