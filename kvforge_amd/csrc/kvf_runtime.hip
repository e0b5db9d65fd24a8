// kvf_runtime.hip - C-ABI entry points of libkvf_hip.so.
//
//   kvf_launch_variant / kvf_launch_varlen_variant / kvf_launch_partial_variant
//       dispatch a decode step by the reference's variant id
//       (src/codegen.cpp:59-65), the way bench/sweep.cu:180-186 does through
//       kvf::Registry;
//   kvf_launch_merge
//       the log-sum-exp merge alone;
//   kvf_quantize_place, kvf_append_tokens
//       the KV append step: quantize fp32 rows on the GPU and scatter them to
//       their physical rows, bit-exact with runtime/kvf_host.h:72-135,166-184.
#include "kvf_kernels.hpp"

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

namespace kvf {
namespace gfx950 {
namespace {

Registry &registry() {
  static Registry reg;
  static std::once_flag once;
  std::call_once(once, [] { kvf_register_all(reg); });
  return reg;
}

LaunchXFn extended(const char *id) { return id ? registry().findx(id) : nullptr; }

// GQA pack size of a variant id ("_g{G}_"), 1 when absent.
int pack_of(const char *id) {
  const char *g = std::strstr(id, "_g");
  return g ? std::max(1, std::atoi(g + 2)) : 1;
}

// Whether `words` unsigned ints hold the fused step's merge counters for `a`
// (one KVF_COUNTER_STRIDE line per (sequence, head group)).
bool counters_fit(const char *id, const kvf_args_t &a, size_t words) {
  if (a.B < 1 || a.H < 1 || a.Hkv < 1) return false;
  const size_t groups = pack_of(id) > 1 ? (size_t)a.Hkv : (size_t)a.H;
  return words >= KVF_COUNTER_WORDS(a.B, groups);
}

Ext ext_of(const kvf_varlen_args_t *va) {
  Ext x;
  if (va) {
    x.seq_lens = va->seq_lens;
    x.q16 = static_cast<const _Float16 *>(va->q16);
    x.out16 = static_cast<_Float16 *>(va->out16);
    x.longest_first = (va->flags & KVF_VARLEN_LONGEST_FIRST) != 0;
  }
  return x;
}

std::vector<std::string> &variant_ids() {
  static std::vector<std::string> ids;
  static std::once_flag once;
  std::call_once(once, [] {
    for (const auto &kv : registry().fn) ids.push_back(kv.first);
    std::sort(ids.begin(), ids.end());
  });
  return ids;
}

// ---------------------------------------------------------------- quantizer
template <int FMT>
__global__ void __launch_bounds__(256)
quantize_place_kernel(const float *__restrict__ x, long long rows, int d, int group, int Hkv,
                      int n, int order, int bt, const int *table, int max_blocks,
                      unsigned char *data, uint32_t *meta, const int *positions) {
  const int lane = threadIdx.x & 63;
  const long long row = (long long)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (row >= rows) return; // whole wavefronts leave together
  // bulk: row r is token r % n of head (r / n) % Hkv of sequence r / (n Hkv);
  // append: row r is head r % Hkv of sequence r / Hkv at token positions[b],
  // and a position outside the layout writes nothing
  int t, h, b;
  if (positions) {
    h = (int)(row % Hkv);
    b = (int)(row / Hkv);
    t = positions[b];
    if (t < 0 || t >= (bt ? max_blocks * bt : n)) return;
  } else {
    t = (int)(row % n);
    h = (int)((row / n) % Hkv);
    b = (int)(row / ((long long)n * Hkv));
  }
  long long prow;
  if (bt == 0) {
    prow = order == ORD_HEAD ? ((long long)b * Hkv + h) * n + t : ((long long)b * n + t) * Hkv + h;
  } else {
    const long long page = table[(long long)b * max_blocks + t / bt];
    const long long base = page * Hkv * bt;
    prow = order == ORD_HEAD ? base + (long long)h * bt + t % bt
                             : base + (long long)(t % bt) * Hkv + h;
  }
  const float *xr = x + row * d;
  const int per = d / 64; // elements per lane: column = e*64 + lane
  if constexpr (FMT == FMT_F16) {
    for (int e = 0; e < per; ++e) {
      const int col = e * 64 + lane;
      const _Float16 hv = (_Float16)xr[col];
      reinterpret_cast<_Float16 *>(data)[prow * d + col] = hv;
    }
    return;
  } else {
    const int levels = FMT == FMT_INT8 ? 255 : 15;
    const int rb = FMT == FMT_INT8 ? d : d / 2;
    const int gpr = d / group;
    float xv[2];
    for (int e = 0; e < per; ++e) xv[e] = xr[e * 64 + lane];
    // min/max over each group: groups of 32 are lane halves, 64 one slot,
    // 128 both slots of a 64-wide row pair
    const int span = group < 64 ? group : 64;
    float lo[2], hi[2];
    for (int e = 0; e < per; ++e) {
      lo[e] = xv[e];
      hi[e] = xv[e];
      for (int m = 1; m < span; m <<= 1) {
        lo[e] = fminf(lo[e], __shfl_xor(lo[e], m));
        hi[e] = fmaxf(hi[e], __shfl_xor(hi[e], m));
      }
    }
    if (group == 128 && per == 2) {
      lo[0] = lo[1] = fminf(lo[0], lo[1]);
      hi[0] = hi[1] = fmaxf(hi[0], hi[1]);
    }
    for (int e = 0; e < per; ++e) {
      const int col = e * 64 + lane;
      const _Float16 zero_h = (_Float16)lo[e];
      float scale = __fdiv_rn(hi[e] - lo[e], (float)levels);
      if (scale <= 0.f) scale = 1.f;
      const _Float16 scale_h = (_Float16)scale;
      const float zero = (float)zero_h;
      const float sc = (float)scale_h;
      const float qf = roundf(__fdiv_rn(xv[e] - zero, sc)); // half away from zero
      const int qv = (int)fminf(fmaxf(qf, 0.f), (float)levels);
      const int gi = col / group;
      if (col % group == 0) {
        const uint32_t w = (uint32_t)__builtin_bit_cast(uint16_t, scale_h) |
                           ((uint32_t)__builtin_bit_cast(uint16_t, zero_h) << 16);
        meta[prow * gpr + gi] = w;
      }
      if constexpr (FMT == FMT_INT8) {
        data[prow * rb + col] = (unsigned char)qv;
      } else {
        const int hi_code = __shfl_down(qv, 1);
        if ((col & 1) == 0)
          data[prow * rb + col / 2] = (unsigned char)(qv | (hi_code << 4));
      }
    }
  }
}

} // namespace
} // namespace gfx950
} // namespace kvf

using namespace kvf;
using namespace kvf::gfx950;

extern "C" hipError_t kvf_launch_variant(const char *id, const kvf_args_t *a, hipStream_t st) {
  if (!a) return hipErrorInvalidValue;
  const LaunchFn fn = registry().find(id ? id : "");
  if (!fn) return hipErrorNotFound;
  return fn(*a, st);
}

extern "C" hipError_t kvf_launch_varlen_variant(const char *id, const kvf_args_t *a,
                                                const kvf_varlen_args_t *va, hipStream_t st) {
  if (!a) return hipErrorInvalidValue;
  const LaunchXFn fx = extended(id);
  if (!fx) return hipErrorNotFound;
  return fx(*a, ext_of(va), Launch{}, st);
}

extern "C" hipError_t kvf_launch_fused_variant(const char *id, const kvf_args_t *a,
                                               const kvf_varlen_args_t *va, unsigned *counters,
                                               size_t counter_words, hipStream_t st) {
  if (!a || !counters) return hipErrorInvalidValue;
  const LaunchXFn fx = extended(id);
  if (!fx) return hipErrorNotFound;
  if (!counters_fit(id, *a, counter_words)) return hipErrorInvalidValue;
  Ext x = ext_of(va);
  x.counters = counters;
  return fx(*a, x, Launch{}, st);
}

extern "C" hipError_t kvf_launch_persistent_variant(const char *id, const kvf_args_t *a,
                                                    const kvf_varlen_args_t *va, unsigned *counters,
                                                    size_t counter_words, unsigned *queue,
                                                    size_t queue_words, int workgroups, hipStream_t st) {
  if (!a || !queue || workgroups < 0) return hipErrorInvalidValue;
  const LaunchXFn fx = extended(id);
  if (!fx) return hipErrorNotFound;
  if (queue_words < KVF_QUEUE_WORDS) return hipErrorInvalidValue;
  if (counters && !counters_fit(id, *a, counter_words)) return hipErrorInvalidValue;
  Ext x = ext_of(va);
  x.counters = counters;
  x.queue = queue;
  x.slots = workgroups;
  return fx(*a, x, Launch{}, st);
}

// ---- the entry point that allocates nothing ----------------------------------
// The one-launch step's device memory beyond inputs and outputs (its merge
// counters and the split partials) lives in `scratch`, a file-scope device
// array of KVF_SCRATCH_BYTES that every GPU holds from module load until the
// process ends. In host code `scratch` names a host-side stand-in, not a
// device address: its address on each device comes from hipGetSymbolAddress,
// called once per device with that device current, and only that address is
// handed to kernels. Layout: [0, 64 KiB) merge counters (zero at load, and
// every completed step leaves them at zero again), then part_ml, then part_o,
// each 256-byte aligned. Calls that overlap on one GPU share the array and
// race.
static __device__ __align__(256) unsigned char scratch[KVF_SCRATCH_BYTES];

namespace {
constexpr size_t SCRATCH_COUNTERS = 64 * 1024;
constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[MAX_DEVICES] = {};

hipError_t scratch_of_current_device(unsigned char **out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= MAX_DEVICES) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void *p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (!p) return hipErrorInvalidSymbol;
    g_scratch_ptr[dev] = p;
  }
  *out = static_cast<unsigned char *>(g_scratch_ptr[dev]);
  return hipSuccess;
}

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }
} // namespace

extern "C" hipError_t kvf_launch_fused_variant_noalloc(const char *id, const kvf_args_t *a,
                                                       const kvf_varlen_args_t *va,
                                                       hipStream_t st) {
  if (!a || a->B < 1 || a->H < 1 || a->Hkv < 1 || a->splits < 1) return hipErrorInvalidValue;
  const LaunchXFn fx = extended(id);
  if (!fx) return hipErrorNotFound;
  // counters: one per (sequence, head group); the pack size comes from the id
  const size_t counters = KVF_COUNTER_WORDS(a->B, pack_of(id) > 1 ? a->Hkv : a->H) * sizeof(unsigned);
  const size_t heads = (size_t)a->B * a->H * a->splits;
  const size_t d = std::strstr(id, "_d64") ? 64 : 128;
  const size_t ml_bytes = align256(heads * 2 * sizeof(float));
  const size_t o_bytes = align256(heads * d * sizeof(float));
  if (counters > SCRATCH_COUNTERS || SCRATCH_COUNTERS + ml_bytes + o_bytes > KVF_SCRATCH_BYTES)
    return hipErrorInvalidValue;
  unsigned char *base = nullptr;
  const hipError_t e = scratch_of_current_device(&base);
  if (e != hipSuccess) return e;
  kvf_args_t b = *a;
  b.part_ml = reinterpret_cast<float *>(base + SCRATCH_COUNTERS);
  b.part_o = reinterpret_cast<float *>(base + SCRATCH_COUNTERS + ml_bytes);
  Ext x = ext_of(va);
  x.counters = reinterpret_cast<unsigned *>(base);
  return fx(b, x, Launch{}, st);
}

extern "C" hipError_t kvf_launch_partial_variant(const char *id, const kvf_args_t *a,
                                                 hipStream_t st) {
  if (!a) return hipErrorInvalidValue;
  const LaunchXFn fx = extended(id);
  if (!fx) return hipErrorNotFound;
  if (!a->part_o || !a->part_ml) return hipErrorInvalidValue;
  Launch l;
  l.partial_only = true;
  return fx(*a, Ext{}, l, st);
}

extern "C" hipError_t kvf_launch_partial_variant_timed(const char *id, const kvf_args_t *a,
                                                       hipStream_t st, hipEvent_t start,
                                                       hipEvent_t stop) {
  if (!a) return hipErrorInvalidValue;
  const LaunchXFn fx = extended(id);
  if (!fx) return hipErrorNotFound;
  if (!a->part_o || !a->part_ml || !start || !stop) return hipErrorInvalidValue;
  Launch l;
  l.partial_only = true;
  l.ev_start = start;
  l.ev_stop = stop;
  return fx(*a, Ext{}, l, st);
}

extern "C" hipError_t kvf_launch_partial_varlen_variant_timed(const char *id, const kvf_args_t *a,
                                                              const kvf_varlen_args_t *va,
                                                              hipStream_t st, hipEvent_t start,
                                                              hipEvent_t stop) {
  if (!a) return hipErrorInvalidValue;
  const LaunchXFn fx = extended(id);
  if (!fx) return hipErrorNotFound;
  if (!a->part_o || !a->part_ml || !start || !stop) return hipErrorInvalidValue;
  Launch l;
  l.partial_only = true;
  l.ev_start = start;
  l.ev_stop = stop;
  return fx(*a, ext_of(va), l, st);
}

extern "C" hipError_t kvf_launch_step_timed(const char *id, const kvf_args_t *a,
                                            const kvf_varlen_args_t *va, unsigned *counters,
                                            size_t counter_words, hipStream_t st, hipEvent_t start,
                                            hipEvent_t stop) {
  if (!a || !start || !stop) return hipErrorInvalidValue;
  const LaunchXFn fx = extended(id);
  if (!fx) return hipErrorNotFound;
  if (counters && !counters_fit(id, *a, counter_words)) return hipErrorInvalidValue;
  Ext x = ext_of(va);
  x.counters = counters;
  Launch l;
  l.ev_start = start;
  l.ev_stop = stop;
  return fx(*a, x, l, st);
}

extern "C" hipError_t kvf_launch_merge(int d, const kvf_args_t *a, hipStream_t st) {
  if (!a || a->splits < 1 || a->B < 1 || a->H < 1 || !a->part_o || !a->part_ml || !a->out)
    return hipErrorInvalidValue;
  if (d == 128) return launch_merge_kernel<128>(*a, Ext{}, st);
  if (d == 64) return launch_merge_kernel<64>(*a, Ext{}, st);
  return hipErrorInvalidValue;
}

extern "C" int kvf_variant_count(void) { return (int)variant_ids().size(); }

extern "C" const char *kvf_variant_id(int i) {
  const auto &ids = variant_ids();
  return (i >= 0 && i < (int)ids.size()) ? ids[i].c_str() : nullptr;
}

namespace {
hipError_t quantize_rows(int fmt, int group, int d, const float *x, int B, int Hkv, int n,
                         const int *positions, int order, int block_tokens,
                         const int *block_table, int max_blocks, unsigned char *data,
                         void *meta, hipStream_t st) {
  if (!x || !data || B < 1 || Hkv < 1 || n < 1 || (d != 64 && d != 128)) return hipErrorInvalidValue;
  if (order != ORD_HEAD && order != ORD_TOKEN) return hipErrorInvalidValue;
  if (block_tokens < 0 || (block_tokens > 0 && (!block_table || max_blocks * block_tokens < n)))
    return hipErrorInvalidValue;
  if (fmt != FMT_F16) {
    if (!meta || (group != 32 && group != 64 && group != 128) || group > d) return hipErrorInvalidValue;
  }
  const long long rows = (long long)B * Hkv * (positions ? 1 : n);
  const dim3 block(256);
  const dim3 grid((unsigned)((rows + 3) / 4));
  uint32_t *m = static_cast<uint32_t *>(meta);
  switch (fmt) {
  case FMT_F16:
    hipLaunchKernelGGL(quantize_place_kernel<FMT_F16>, grid, block, 0, st, x, rows, d, group, Hkv,
                       n, order, block_tokens, block_table, max_blocks, data, m, positions);
    break;
  case FMT_INT8:
    hipLaunchKernelGGL(quantize_place_kernel<FMT_INT8>, grid, block, 0, st, x, rows, d, group,
                       Hkv, n, order, block_tokens, block_table, max_blocks, data, m, positions);
    break;
  case FMT_INT4:
    hipLaunchKernelGGL(quantize_place_kernel<FMT_INT4>, grid, block, 0, st, x, rows, d, group,
                       Hkv, n, order, block_tokens, block_table, max_blocks, data, m, positions);
    break;
  default:
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}
} // namespace

extern "C" hipError_t kvf_quantize_place(int fmt, int group, int d, const float *x, int B,
                                         int Hkv, int n, int order, int block_tokens,
                                         const int *block_table, int max_blocks,
                                         unsigned char *data, void *meta, hipStream_t st) {
  return quantize_rows(fmt, group, d, x, B, Hkv, n, nullptr, order, block_tokens, block_table,
                       max_blocks, data, meta, st);
}

extern "C" hipError_t kvf_append_tokens(int fmt, int group, int d, const float *x, int B, int Hkv,
                                        int n, const int *positions, int order,
                                        int block_tokens, const int *block_table,
                                        int max_blocks, unsigned char *data, void *meta,
                                        hipStream_t st) {
  if (!positions) return hipErrorInvalidValue;
  return quantize_rows(fmt, group, d, x, B, Hkv, n, positions, order, block_tokens, block_table,
                       max_blocks, data, meta, st);
}

extern "C" const char *kvf_version(void) { return "kvforge-mi355x 0.3 (gfx950, ABI 2)"; }

extern "C" int kvf_abi_version(void) { return KVF_ABI_VERSION; }
