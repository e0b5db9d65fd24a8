/* kvf_abi.h - the drop-in boundary of KVForge's decode-attention path, MI355X.
 *
 * This header replaces the ABI part of the reference's
 * runtime/kvf_kernels.cuh (Args, Fmt, Ord: lines 26-46) and the extern "C"
 * launcher that src/codegen.cpp:79-91 emits. A plan compiled for the
 * reference drops in unchanged: the same Args layout (9 pointers, 9 ints, one
 * float, in the same order), the same variant ids, the same plan-override
 * semantics (a launcher overwrites splits, warps, group_shift, block_shift),
 * the same error behaviour (the launch error is returned, faults surface at
 * the caller's next synchronisation, nothing is allocated and no host sync is
 * made), with hipError_t / hipStream_t in place of the CUDA types.
 *
 * MI355X meaning of the scheduling fields: `warps` is the number of 64-lane
 * wavefronts per workgroup (4 or 8), not 32-thread warps.
 */
#ifndef KVF_ABI_H
#define KVF_ABI_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
#include <hip/hip_fp16.h>
namespace kvf {

/* runtime/kvf_kernels.cuh:26-27 */
enum Fmt { FMT_F16 = 0, FMT_INT8 = 1, FMT_INT4 = 2 };
enum Ord { ORD_HEAD = 0, ORD_TOKEN = 1 };

/* runtime/kvf_kernels.cuh:29-46, field for field. */
struct Args {
  const float *q;          /* [B][H][D], fp32 */
  const unsigned char *k;  /* K payload, rows of D*bits/8 bytes */
  const unsigned char *v;  /* V payload */
  const __half2 *k_meta;   /* [rows][D/group] (scale, zero), quantized only */
  const __half2 *v_meta;
  const int *block_table;  /* [B][max_blocks] page ids, paged layouts only */
  float *out;              /* [B][H][D], fp32 */
  float *part_o;           /* [B][H][splits][D] unnormalised partial output */
  float *part_ml;          /* [B][H][splits][2] running max (log2) and sum */
  int B, H, Hkv, n;
  int splits;              /* chunks of the KV length per head */
  int warps;               /* 64-lane wavefronts per workgroup (4 or 8) */
  int group_shift;         /* log2(quantization group), quantized only */
  int block_shift;         /* log2(tokens per page), paged only */
  int max_blocks;          /* pages per sequence in the block table */
  float scale_log2;        /* softmax scale * log2(e) */
};

/* Additive extension for variable-length batches out of a shared block pool
 * with optional f16 query/output (no counterpart in the reference's Args,
 * which has one n for every sequence and fp32 q/out only,
 * runtime/kvf_kernels.cuh:30-39). Args stays byte-identical; these fields
 * travel beside it. With per-sequence lengths split s of a sequence takes
 * its 32-token tiles s, s + splits, s + 2 * splits, ... (uniform lengths keep
 * the reference's contiguous chunks), so part_o / part_ml hold different
 * partials than a contiguous split would; the merged output agrees to
 * rounding. */
struct VarlenArgs {
  const int *seq_lens;     /* [B] tokens per sequence; Args::n is the maximum */
  const void *q16;         /* [B][H][D] binary16 query, or NULL to use Args::q */
  void *out16;             /* [B][H][D] binary16 output, or NULL to use Args::out */
  int flags;               /* KVF_VARLEN_* bits; 0 by default */
};

} /* namespace kvf */
typedef kvf::Args kvf_args_t;
typedef kvf::VarlenArgs kvf_varlen_args_t;
#else
/* The same layout for C callers. */
typedef struct kvf_args {
  const float *q;
  const unsigned char *k, *v;
  const void *k_meta, *v_meta;
  const int *block_table;
  float *out, *part_o, *part_ml;
  int B, H, Hkv, n, splits, warps, group_shift, block_shift, max_blocks;
  float scale_log2;
} kvf_args_t;
typedef struct kvf_varlen_args {
  const int *seq_lens;
  const void *q16;
  void *out16;
  int flags;
} kvf_varlen_args_t;
#endif

/* Version of this C ABI, also returned by kvf_abi_version(). 2: the one-launch
 * (kvf_launch_fused_variant), persistent and timed-step entry points take
 * the sizes of their counter and queue buffers, in 32-bit words, and reject
 * buffers that are too small; VarlenArgs carries `flags`. Version 1 took the
 * buffers without sizes, and its VarlenArgs had three fields (24 bytes).
 * A caller built against another version checks kvf_abi_version() at load. */
#define KVF_ABI_VERSION 2

/* VarlenArgs::flags. LONGEST_FIRST (batches of 2..64 sequences): workgroups
 * take sequences in decreasing length, so the longest sequences' workgroups
 * are dispatched first and the short ones fill the tail. The output is
 * identical either way; it pays when lengths are very unequal (a log-uniform
 * batch of 16 sequences: 95 -> 78 us) and costs a dependent load at the start
 * otherwise (8 sequences within 3x of each other: +2 %). */
#define KVF_VARLEN_LONGEST_FIRST 1

#ifdef __cplusplus
extern "C" {
#endif

/* ---- dispatch by variant id ------------------------------------------------
 * Variant ids are the reference's: "{fmt}_{hm|tm}_{c|p}_g{G}_u{U}_d{D}"
 * (src/codegen.cpp:59-65), e.g. "int8_hm_c_g4_u2_d128". These entry points
 * are the C-ABI face of kvf::Registry (runtime/kvf_registry.h:15-24) for
 * callers outside C++ (ctypes, cgo); the registry lookup plus
 * `fn(a, st)` is exactly what bench/sweep.cu:180-186 does. */

/* Launch one decode step (partial kernel, plus the merge when a->splits > 1)
 * with the caller's Args unchanged. Returns hipErrorNotFound for an unknown
 * id, hipErrorInvalidValue for arguments the kernels cannot run (for
 * example warps outside {4, 8} or a group the format does not offer),
 * otherwise the launch status. */
hipError_t kvf_launch_variant(const char *variant_id, const kvf_args_t *a,
                              hipStream_t stream);

/* As kvf_launch_variant, for the variable-length / block-pool extension. */
hipError_t kvf_launch_varlen_variant(const char *variant_id, const kvf_args_t *a,
                                     const kvf_varlen_args_t *va,
                                     hipStream_t stream);

/* Unsigned ints per merge counter of the one-launch step: each counter has a
 * 128-byte line of its own, so the arrivals of different head groups do not
 * serialise on one line. A step of B sequences needs
 * KVF_COUNTER_WORDS(B, head groups) of them, head groups = Hkv for GQA-packed
 * variants ("_g2_" and up) and H otherwise. */
#define KVF_COUNTER_STRIDE 32
#define KVF_COUNTER_WORDS(B, head_groups) ((size_t)(B) * (size_t)(head_groups) * KVF_COUNTER_STRIDE)
/* Unsigned ints of the persistent step's work queue. */
#define KVF_QUEUE_WORDS (2 * KVF_COUNTER_STRIDE)

/* One decode step in a single kernel launch: the last workgroup of each
 * (sequence, head group) merges the splits, which removes the reference's
 * second (merge) launch (runtime/kvf_kernels.cuh:315-318). `counters` is
 * caller-owned device memory of `counter_words` unsigned ints, at least
 * KVF_COUNTER_WORDS(B, pack > 1 ? Hkv : H) (hipErrorInvalidValue otherwise,
 * before anything is launched), zero before the first call; every call
 * leaves it zero again. Calls that run concurrently (on different streams)
 * need distinct counters, exactly as they need distinct part_o / part_ml.
 * `va` may be NULL. Outputs match kvf_launch_variant to rounding. */
hipError_t kvf_launch_fused_variant(const char *variant_id, const kvf_args_t *a,
                                    const kvf_varlen_args_t *va, unsigned *counters,
                                    size_t counter_words, hipStream_t stream);

/* The persistent step: one launch whose workgroups, at most as many as are
 * resident at once (`workgroups` > 0 caps them further), work through a
 * queue of the step's B * head groups * splits items, claiming the next item
 * with one atomic while the current one's last tiles are in flight; the
 * work queue over (head, split) that the reference's cost model prices as
 * T_merge, T_launch and imbalance (src/cost.cpp:163-188, 212-231). Items go
 * sequence by sequence (longest first with KVF_VARLEN_LONGEST_FIRST), head
 * group by head group, split by split. With `counters` (as in
 * kvf_launch_fused_variant) the last workgroup of each head group merges its
 * splits inside the launch; with counters == NULL the merge kernel follows,
 * as in kvf_launch_varlen_variant. `counter_words` is the size of `counters` (0
 * with no counters), checked as for kvf_launch_fused_variant. `queue` is
 * caller-owned device memory of `queue_words` >= KVF_QUEUE_WORDS unsigned
 * ints, zero before the first call; every call leaves it zero again, and
 * concurrent calls need distinct queues.
 * `va` may be NULL. Outputs equal kvf_launch_fused_variant's (counters) or
 * kvf_launch_varlen_variant's (no counters) bit for bit. Unroll-2 variants
 * only ("_u2_" ids); others return hipErrorInvalidValue. No counterpart in
 * the reference, which launches one block per (split, head). */
hipError_t kvf_launch_persistent_variant(const char *variant_id, const kvf_args_t *a,
                                         const kvf_varlen_args_t *va, unsigned *counters,
                                         size_t counter_words, unsigned *queue,
                                         size_t queue_words, int workgroups, hipStream_t stream);

/* Bytes of the device scratch array behind kvf_launch_fused_variant_noalloc. */
#define KVF_SCRATCH_BYTES (16u << 20)

/* As kvf_launch_fused_variant, but allocating nothing and taking no
 * workspace: the merge counters and the split partials live in a file-scope
 * device array of KVF_SCRATCH_BYTES (16 MiB) that each GPU holds until the
 * process ends, so Args::part_o and Args::part_ml are ignored. No counterpart
 * in the reference; it is for callers that cannot allocate (code under HIP
 * graph capture, tight serving loops). Returns hipErrorInvalidValue when the
 * step's counters (KVF_COUNTER_WORDS(B, pack > 1 ? Hkv : H) unsigned ints, at
 * most 64 KiB) or partials (B*H*splits*(d+2) floats) do not fit. The first
 * call on a device (and the first of each variant) sets up: it looks up the
 * array's device address and the device's CU and XCD counts and queries the
 * kernel's occupancy, none of which allocates; make one call per variant
 * before capturing a graph, after which a call only enqueues the kernel (no
 * memset: the kernel returns its counters to zero itself). Calls that overlap
 * on one GPU share the array and race; run them on one stream. */
hipError_t kvf_launch_fused_variant_noalloc(const char *variant_id, const kvf_args_t *a,
                                            const kvf_varlen_args_t *va,
                                            hipStream_t stream);

/* Only the partial (split) kernel of a variant, writing part_o / part_ml
 * even when splits == 1; for measuring the streaming kernel by itself. */
hipError_t kvf_launch_partial_variant(const char *variant_id, const kvf_args_t *a,
                                      hipStream_t stream);

/* As kvf_launch_partial_variant, with `start` and `stop` (created by the
 * caller with timing enabled) bound to the split kernel's own dispatch, so
 * hipEventElapsedTime(start, stop) is that kernel's execution time, the
 * figure a kernel trace reports. Harness use (the reference's time_launch,
 * runtime/kvf_host.h:302-331, brackets the launch with events instead). */
hipError_t kvf_launch_partial_variant_timed(const char *variant_id, const kvf_args_t *a,
                                            hipStream_t stream, hipEvent_t start,
                                            hipEvent_t stop);

/* As kvf_launch_partial_variant_timed, for the variable-length / block-pool
 * extension (`va` as in kvf_launch_varlen_variant; may be NULL). Harness use,
 * no counterpart in the reference. */
hipError_t kvf_launch_partial_varlen_variant_timed(const char *variant_id, const kvf_args_t *a,
                                                   const kvf_varlen_args_t *va,
                                                   hipStream_t stream, hipEvent_t start,
                                                   hipEvent_t stop);

/* One whole decode step, as kvf_launch_varlen_variant (`va` may be NULL) or,
 * when `counters` is not NULL, as kvf_launch_fused_variant (`counter_words`
 * its size, checked the same way), with `start` and
 * `stop` (created by the caller with timing enabled) bound to the split
 * kernel's own dispatch: hipEventElapsedTime(start, stop) is that kernel's
 * execution time inside the step, the merge launch (if any) following it as
 * it does in every step. Harness use, no counterpart in the reference. */
hipError_t kvf_launch_step_timed(const char *variant_id, const kvf_args_t *a,
                                 const kvf_varlen_args_t *va, unsigned *counters,
                                 size_t counter_words, hipStream_t stream, hipEvent_t start,
                                 hipEvent_t stop);

/* Only the log-sum-exp merge (runtime/kvf_kernels.cuh:288-306) of the
 * partials named by `a` (B, H, splits, part_o, part_ml, out) for head
 * dimension d. */
hipError_t kvf_launch_merge(int d, const kvf_args_t *a, hipStream_t stream);

/* Number of registered variants and the id of the i-th one. */
int kvf_variant_count(void);
const char *kvf_variant_id(int i);

/* ---- KV append / quantize (the step before the path) ----------------------
 * Quantize `rows` logical rows of `d` fp32 values (device memory, row r is
 * sequence b = r / (Hkv*n), head h = (r / n) % Hkv, token t = r % n) in the
 * format (fmt, group) and write each row to its physical row of the
 * (order, paged) layout: codes into `data`, (scale, zero) binary16 pairs
 * into `meta` (NULL for f16). Bit-exact with the reference's host quantizer
 * (runtime/kvf_host.h:72-121) and placement (runtime/kvf_host.h:124-135,
 * 166-184). `block_table` is [B][max_blocks] when block_tokens > 0. */
hipError_t kvf_quantize_place(int fmt, int group, int d, const float *x,
                              int B, int Hkv, int n, int order,
                              int block_tokens, const int *block_table,
                              int max_blocks, unsigned char *data, void *meta,
                              hipStream_t stream);

/* Append one token per sequence: quantize the B*Hkv rows of `x`
 * ([B][Hkv][d] fp32, device memory) and write row (b, h) to token
 * positions[b] (device int32 [B]) of the same layouts as kvf_quantize_place,
 * whose arithmetic it shares, so appending every token of a cache one call
 * at a time produces the same bytes as placing it whole. A position outside
 * [0, n) (contiguous) or [0, max_blocks*block_tokens) (paged) writes nothing.
 * No counterpart in the reference, which quantizes on the host
 * (runtime/kvf_host.h:72-121); it is the per-step form of that step. */
hipError_t kvf_append_tokens(int fmt, int group, int d, const float *x,
                             int B, int Hkv, int n, const int *positions,
                             int order, int block_tokens,
                             const int *block_table, int max_blocks,
                             unsigned char *data, void *meta,
                             hipStream_t stream);

/* Library version string. */
const char *kvf_version(void);

/* KVF_ABI_VERSION of the library's build. */
int kvf_abi_version(void);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* KVF_ABI_H */
