/* kvf_oracle.h - CPU restatement of KVForge's host-side arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker the parity tests,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg compare the HIP
 * path against. Nothing in kvforge_amd/ links, loads or calls it.
 *
 * Every function restates one piece of the reference (paths relative to the
 * reference checkout):
 *   kvfo_make_data              runtime/kvf_host.h:51-61
 *   kvfo_quantize               runtime/kvf_host.h:72-121
 *   kvfo_page_table             runtime/kvf_host.h:156-165 (std::shuffle of iota)
 *   kvfo_row_of                 runtime/kvf_host.h:124-135
 *   kvfo_place                  runtime/kvf_host.h:149-197 (host scatter part)
 *   kvfo_reference_attention    runtime/kvf_host.h:202-234 (and _mt: the
 *                               same per-head arithmetic over host threads)
 *   kvfo_rel_l2                 runtime/kvf_host.h:236-244
 *   kvfo_reference_partials     runtime/kvf_kernels.cuh:147-153,276-281 (split
 *                               chunking, per-split max/sum in the log2 domain)
 *   kvfo_merge_partials         runtime/kvf_kernels.cuh:288-306
 *   kvfo_scale_log2             runtime/kvf_host.h:292
 * Extensions that the reference does not have (outlier channels, variable
 * lengths, the shared block pool) are this build's own definitions and are
 * marked as such where they are defined.
 *
 * Pinning (see tests/test_oracle.py): binary16 conversion against numpy over
 * every half and a dense float sweep; mt19937_64 against the C++ standard's
 * known answer; quantizer against hand-checked rows and invariants; the
 * attention reference against closed forms and scipy's softmax; placement by
 * brute-force bijection checks; the merge against the unsplit reference;
 * log-uniform lengths against a numpy restatement of libstdc++'s
 * generate_canonical over the raw mt19937_64 stream; ragged data against
 * make_data for equal lengths and against its own draw order.
 */
#ifndef KVF_ORACLE_H
#define KVF_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* formats and orders use the reference's numbering (kvf_kernels.cuh:26-27) */
enum { KVFO_F16 = 0, KVFO_INT8 = 1, KVFO_INT4 = 2 };
enum { KVFO_HEAD = 0, KVFO_TOKEN = 1 };

uint16_t kvfo_f2h(float f);
float kvfo_h2f(uint16_t h);
void kvfo_f2h_array(const float *x, uint16_t *out, long long n);
void kvfo_h2f_array(const uint16_t *x, float *out, long long n);

/* The 10000th output of a default-seeded std::mt19937_64 (for the KAT). */
uint64_t kvfo_mt64_10000th(void);
/* First `count` raw outputs of mt19937_64(seed). */
void kvfo_mt64_raw(uint64_t seed, uint64_t *out, long long count);
/* `count` draws of std::normal_distribution<float>(0,1) on mt19937_64(seed). */
void kvfo_normal(uint64_t seed, float *out, long long count);

/* q [B][H][D], K and V [B][Hkv][n][D] in logical order, drawn in that order. */
void kvfo_make_data(int B, int H, int Hkv, int D, int n, uint64_t seed,
                    float *q, float *K, float *V);

/* Quantize `rows` logical rows of D floats.
 *   data: rows * D*bits/8 bytes;  meta: rows * (D/group) * 2 halves laid out
 *   as (scale, zero) pairs;  deq: rows * D dequantised floats.
 * meta may be NULL for f16. */
void kvfo_quantize(int fmt, int group, int D, const float *X, long long rows,
                   uint8_t *data, uint16_t *meta, float *deq);

/* perm = iota(pages) shuffled by std::shuffle with mt19937_64(seed). */
void kvfo_page_table(long long pages, uint64_t seed, int32_t *perm);

/* Physical row of (b, h, t). table may be NULL when bt == 0 (contiguous). */
long long kvfo_row_of(int order, int bt, const int32_t *table, int max_blocks,
                      int n, int Hkv, int b, int h, int t);

/* Scatter logical quantized rows into the physical layout (zero elsewhere).
 * rows_alloc: B*Hkv*n for contiguous, pages*Hkv*bt for paged. */
void kvfo_place(int B, int Hkv, int n, int row_bytes, int meta_words,
                int order, int bt, const int32_t *table, int max_blocks,
                const uint8_t *data, const uint32_t *meta,
                uint8_t *pdata, uint32_t *pmeta);

/* Exact attention in double over logical K/V, out [B][H][D] floats. */
void kvfo_reference_attention(int B, int H, int Hkv, int D, int n,
                              const float *q, const float *K, const float *V,
                              float scale, float *out);

/* As kvfo_reference_attention, over `threads` host threads (same output). */
void kvfo_reference_attention_mt(int B, int H, int Hkv, int D, int n,
                                 const float *q, const float *K, const float *V,
                                 float scale, float *out, int threads);
/* Variable-length extension (this build's definition): sequence b uses the
 * first lens[b] tokens of its rows; K/V are [B][Hkv][n_max][D]. */
void kvfo_reference_attention_varlen(int B, int H, int Hkv, int D, int n_max,
                                     const int32_t *lens, const float *q,
                                     const float *K, const float *V,
                                     float scale, float *out);
/* As kvfo_reference_attention_varlen, over `threads` host threads. */
void kvfo_reference_attention_varlen_mt(int B, int H, int Hkv, int D, int n_max,
                                        const int32_t *lens, const float *q,
                                        const float *K, const float *V, float scale,
                                        float *out, int threads);
/* The varlen reference over ragged arrays (kvfo_make_data_ragged's layout):
 * sequence b's rows start at Hkv * (lens[0] + ... + lens[b-1]), head by head.
 * Pinned against kvfo_reference_attention_varlen on the padded arrays. */
void kvfo_reference_attention_ragged_mt(int B, int H, int Hkv, int D, const int32_t *lens,
                                        const float *q, const float *K, const float *V,
                                        float scale, float *out, int threads);

double kvfo_rel_l2(const float *a, const float *ref, long long n);
float kvfo_scale_log2(int D);

/* Per-split results in double: for split s of head (b,h) over tokens
 * [s*chunk, min(n,(s+1)*chunk)), chunk = ceil(n/S):
 *   o_norm [B][H][S][D]  normalised partial output (0 when empty)
 *   lse2   [B][H][S]     log2-domain log-sum-exp of the scores scaled by
 *                        scale_log2 (-inf when empty)
 *   m2     [B][H][S]     log2-domain max score (-inf when empty) */
void kvfo_reference_partials(int B, int H, int Hkv, int D, int n, int S,
                             const float *q, const float *K, const float *V,
                             float scale_log2, float *o_norm, double *lse2,
                             double *m2);

/* Log-sum-exp merge of unnormalised partials in the reference's layout
 * (part_o [B][H][S][D], part_ml [B][H][S][2]), computed in double. */
void kvfo_merge_partials(int B, int H, int D, int S, const float *part_o,
                         const float *part_ml, float *out);

/* Outlier extension (this build's definition): shuffle iota(Hkv*D) with
 * mt19937_64(seed), take the first ceil(frac*Hkv*D) entries (kv_head*D +
 * channel) and multiply those K and V columns by `factor` for every b and t.
 * Returns the number of channels written to `chosen` (may be NULL). */
int kvfo_inject_outliers(int B, int Hkv, int D, int n, uint64_t seed,
                         double frac, float factor, float *K, float *V,
                         int32_t *chosen);

/* Variable lengths (this build's definition): lens[b] = lo + U{0..hi-lo}
 * drawn with std::uniform_int_distribution<int> on mt19937_64(seed). */
void kvfo_varlen_lengths(int B, int lo, int hi, uint64_t seed, int32_t *lens);

/* Shared block pool (this build's definition): pool pages are
 * iota(pool) shuffled with mt19937_64(seed); sequence b takes the next
 * ceil(lens[b]/bt) pages in order. table is [B][max_blocks] with
 * max_blocks = ceil(max(lens)/bt); unused entries are -1. Returns the number
 * of pages handed out, or -1 if the pool is too small. */
int kvfo_pool_table(int B, const int32_t *lens, int bt, int pool,
                    uint64_t seed, int max_blocks, int32_t *table);

/* Log-uniform lengths (this build's definition):
 * lens[b] = clamp(lround(exp(u)), lo, hi) with u drawn in order by
 * std::uniform_real_distribution<double>(ln lo, ln hi) on mt19937_64(seed). */
void kvfo_lengths_loguniform(int B, int lo, int hi, uint64_t seed, int32_t *lens);

/* Ragged data (this build's definition): make_data's draws (q, then K, then
 * V) over the tokens each sequence holds only; K and V rows (b, h, t <
 * lens[b]) are packed in that order, so equal lengths give make_data's
 * arrays. */
void kvfo_make_data_ragged(int B, int H, int Hkv, int D, const int32_t *lens,
                           uint64_t seed, float *q, float *K, float *V);

#ifdef __cplusplus
}
#endif
#endif
