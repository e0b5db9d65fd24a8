// bw_probe - the machine-file figures of the CDNA cost model, measured on the
// GPU it runs on with the decode kernels' own access pattern: 16-byte raw
// buffer loads through a per-workgroup descriptor, issued in batches, each
// workgroup walking its own contiguous run of memory once.
//
// Its output is a machine file in the reference's format (src/machine.cpp
// reads the same `key = value` lines). The experiments:
//
//   stream  HBM read rate. A 4 GiB buffer is read in 1 GiB windows, each rep
//           a different window, so no rep finds its bytes in the 256 MiB
//           memory-side cache (MALL). Workgroups per CU x waves x loads in
//           flight per lane; the best is bw_peak_gbs.
//   curve   rate against bytes in flight per CU, one workgroup per CU, for
//           1 .. all CUs; the best one-CU rate is bw_sm_gbs. The table is the
//           cost model's Little's-law data.
//   chase   one lane follows a random cycle through the 128-byte lines of a
//           2 GiB buffer, a MALL-sized read in front of every rep and every
//           rep continuing where the previous one stopped, so each hop is to
//           a line no rep has touched: lat_ns. The same hops again behind a
//           read that clears L2 but not the MALL: lat_mall_ns.
//   trip    event-bound (hipExtLaunchKernelGGL) duration of a full-chip grid
//           of empty workgroups, kernel_floor_us, and, printed beside it, of
//           one whose lanes each load 16 bytes of cold memory and store them
//           (a kernel's fixed cost hides that round trip; the latency of a
//           memory round trip is the chase's lat_ns).
//   cached  repeated reads of a set that fits one XCD's L2 and of one that
//           fits the MALL: bw_l2_gbs, bw_mall_gbs.
//   grain   one dword per S bytes of cold memory: bytes each access costs at
//           the peak rate; the stride past which that stops growing is the
//           transaction size, sector_bytes.
//   fma     FP32 multiply-add rate, f32_gflops; launch: stream-ordered empty
//           kernel between events, launch_us; copy: a read+write kernel,
//           bw_copy_gbs.
//
//   bw_probe [--name NAME] [--out FILE] [--device N] [--quick] [--resources CSV]
//                              (CSV: the kernel resource table the machine
//                              file names, kvforge_amd/tools/dump_resources.py)
//   bw_probe --copy MIB        one copy of MIB MiB and nothing else: the
//                              kernel of known traffic that calibrates the
//                              FETCH_SIZE / WRITE_SIZE counters
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <numeric>
#include <random>
#include <string>
#include <vector>

namespace {

#define CK(call)                                                                                   \
  do {                                                                                             \
    const hipError_t e_ = (call);                                                                  \
    if (e_ != hipSuccess) {                                                                        \
      std::fprintf(stderr, "%s:%d: %s: %s\n", __FILE__, __LINE__, #call, hipGetErrorString(e_));   \
      std::exit(1);                                                                                \
    }                                                                                              \
  } while (0)

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kWord3 = 0x00020000; // raw buffer, 32-bit data format
constexpr int kStream = 2;         // nontemporal: every byte is read once

// Descriptor over `bytes` from `p`; every field is wave-uniform.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t desc(const void *p, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
  return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void *>(((uint64_t)hi << 32) | lo), 0,
                                           (int)__builtin_amdgcn_readfirstlane(bytes), kWord3);
}

// Workgroup w reads run bytes from base + w * run: the waves take 1 KiB rows
// in turn, each lane 16 bytes of a row, DEPTH rows per wave issued before any
// is consumed. `run` is a multiple of waves * DEPTH KiB. CPOL is the loads'
// cache policy: nontemporal streams, 0 allocates in L2 (to evict it).
template <int DEPTH, int CPOL = kStream>
__global__ void __launch_bounds__(1024) run_read(const char *base, uint32_t run, int *sink) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, waves = blockDim.x >> 6;
  const __amdgpu_buffer_rsrc_t rs = desc(base + (size_t)blockIdx.x * run, run);
  const uint32_t step = (uint32_t)waves * DEPTH * 1024;
  v4i acc = {0, 0, 0, 0};
  for (uint32_t o = (uint32_t)wave * 1024 + lane * 16; o < run; o += step) {
    v4i v[DEPTH];
#pragma unroll
    for (int d = 0; d < DEPTH; ++d)
      v[d] = __builtin_amdgcn_raw_buffer_load_b128(rs, o + (uint32_t)d * waves * 1024, 0, CPOL);
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) acc ^= v[d];
  }
  const int r = acc.x ^ acc.y ^ acc.z ^ acc.w;
  if (r == 0x5bd1e995) sink[threadIdx.x] = r; // keeps the loads; the data never holds it
}

// Every workgroup reads the same `bytes` (a cache-resident set, a multiple
// of 4 x 4 KiB) `passes` times, starting at a different row so the
// workgroups spread over it.
__global__ void __launch_bounds__(256) reread(const char *base, uint32_t bytes, int passes, int *sink) {
  const __amdgpu_buffer_rsrc_t rs = desc(base, bytes);
  const uint32_t lanes = blockDim.x * 16;
  uint32_t o = (blockIdx.x * lanes + threadIdx.x * 16) % bytes;
  v4i acc = {0, 0, 0, 0};
  const uint32_t n = bytes / lanes;
  for (int p = 0; p < passes; ++p)
    for (uint32_t i = 0; i < n; i += 4) {
      v4i v[4];
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        v[d] = __builtin_amdgcn_raw_buffer_load_b128(rs, o, 0, 0);
        o += lanes;
        if (o >= bytes) o -= bytes;
      }
#pragma unroll
      for (int d = 0; d < 4; ++d) acc ^= v[d];
    }
  const int r = acc.x ^ acc.y ^ acc.z ^ acc.w;
  if (r == 0x5bd1e995) sink[threadIdx.x] = r;
}

// One lane: `hops` dependent loads, line index i -> next[i * 32].
__global__ void follow(const uint32_t *next, uint32_t from, int hops, uint32_t *end) {
  uint32_t i = from;
  for (int h = 0; h < hops; ++h) i = __builtin_nontemporal_load(next + (size_t)i * 32);
  *end = i;
}

__global__ void nothing() {}

// Each lane: one 16-byte load of cold memory, one store.
__global__ void __launch_bounds__(256) one_trip(const v4i *src, v4i *dst) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  dst[i] = __builtin_nontemporal_load(src + i);
}

// One dword per `stride` bytes, each lane `per` accesses `stride` * lanes apart.
__global__ void __launch_bounds__(256) sparse_read(const char *base, uint32_t stride, int per, int *sink) {
  const size_t lanes = (size_t)gridDim.x * blockDim.x;
  size_t at = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * stride;
  int acc = 0;
  for (int k = 0; k < per; ++k, at += lanes * stride)
    acc ^= __builtin_nontemporal_load(reinterpret_cast<const int *>(base + at));
  if (acc == 0x5bd1e995) sink[threadIdx.x] = acc;
}

// Sixteen independent multiply-add chains per lane.
__global__ void __launch_bounds__(256) fma_rate(float *out, int iters) {
  float x[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) x[j] = threadIdx.x * 0.001f + j;
  const float m = 0.999999f, c = 0.5f;
  for (int i = 0; i < iters; ++i) {
#pragma unroll
    for (int j = 0; j < 16; ++j) x[j] = __builtin_fmaf(x[j], m, c);
  }
  float s = 0;
#pragma unroll
  for (int j = 0; j < 16; ++j) s += x[j];
  out[(size_t)blockIdx.x * blockDim.x + threadIdx.x] = s;
}

// Reads and writes n 16-byte words, both nontemporal.
__global__ void __launch_bounds__(256) copy16(const v4i *src, v4i *dst, size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    __builtin_nontemporal_store(__builtin_nontemporal_load(src + i), dst + i);
}

// ----------------------------------------------------------------- timing
struct Events {
  hipEvent_t a, b;
  Events() {
    CK(hipEventCreate(&a));
    CK(hipEventCreate(&b));
  }
  ~Events() {
    (void)hipEventDestroy(a);
    (void)hipEventDestroy(b);
  }
  double us() {
    CK(hipEventSynchronize(b));
    float ms = 0;
    CK(hipEventElapsedTime(&ms, a, b));
    return ms * 1e3;
  }
};

// Median over reps of the stream-ordered time of body(rep), with prep(rep)
// run untimed before each.
template <class Prep, class Body> double median_us(int reps, Prep &&prep, Body &&body) {
  Events e;
  std::vector<double> t;
  for (int r = 0; r < reps + 2; ++r) {
    prep(r);
    CK(hipEventRecord(e.a, 0));
    body(r);
    CK(hipGetLastError());
    CK(hipEventRecord(e.b, 0));
    const double us = e.us();
    if (r >= 2) t.push_back(us);
  }
  std::sort(t.begin(), t.end());
  return t[t.size() / 2];
}

// Median of the event-bound duration of a kernel launch (the events are
// recorded by the dispatch itself, as a kernel trace times it).
template <class Launch> double bound_us(int reps, Launch &&launch) {
  Events e;
  std::vector<double> t;
  for (int r = 0; r < reps + 5; ++r) {
    launch(e.a, e.b, r);
    CK(hipGetLastError());
    const double us = e.us();
    if (r >= 5) t.push_back(us);
  }
  std::sort(t.begin(), t.end());
  return t[t.size() / 2];
}

struct Device {
  hipDeviceProp_t prop;
  int cus = 0, wave = 64, xcds = 1;
  long long l2 = 0;
};

template <int DEPTH>
void launch_run(int wgs, int threads, const char *base, uint32_t run, int *sink) {
  hipLaunchKernelGGL(run_read<DEPTH>, dim3(wgs), dim3(threads), 0, 0, base, run, sink);
}

// Rate of `wgs` workgroups each reading `run` bytes. Rep r reads window
// r % windows of the buffer; with as many windows as fit (64 at most), at
// least 512 MiB of other windows are read before one comes round again, so
// no rep finds its bytes in the MALL.
double run_rate(int depth, int wgs, int threads, const char *buf, size_t buf_bytes, uint32_t run, int *sink,
                int reps) {
  const size_t span = (size_t)wgs * run;
  const size_t windows = std::max<size_t>(1, std::min<size_t>(64, buf_bytes / span));
  if ((windows - 1) * span < (512ull << 20)) {
    std::fprintf(stderr, "run_rate: %zu bytes per rep leave no room to evict the MALL\n", span);
    std::exit(1);
  }
  const size_t stride = buf_bytes / windows;
  const double us = median_us(
      reps, [](int) {},
      [&](int r) {
        const char *b = buf + (size_t)(r % windows) * stride;
        switch (depth) {
        case 2: launch_run<2>(wgs, threads, b, run, sink); break;
        case 4: launch_run<4>(wgs, threads, b, run, sink); break;
        case 8: launch_run<8>(wgs, threads, b, run, sink); break;
        default: launch_run<16>(wgs, threads, b, run, sink); break;
        }
      });
  return span / (us * 1e3);
}

int copy_only(int mib) {
  const size_t bytes = (size_t)mib << 20;
  v4i *src, *dst;
  CK(hipMalloc(&src, bytes));
  CK(hipMalloc(&dst, bytes));
  CK(hipMemset(src, 3, bytes));
  hipLaunchKernelGGL(copy16, dim3(2048), dim3(256), 0, 0, src, dst, bytes / 16);
  CK(hipGetLastError());
  CK(hipDeviceSynchronize());
  std::printf("copy16: %d MiB read and %d MiB written (%zu KiB each)\n", mib, mib, bytes >> 10);
  CK(hipFree(src));
  CK(hipFree(dst));
  return 0;
}

} // namespace

int main(int argc, char **argv) {
  std::string name = "mi355x", out_path, resources;
  int dev = 0, copy_mib = 0;
  bool quick = false;
  for (int i = 1; i < argc; ++i) {
    const std::string a = argv[i];
    if (a == "--name" && i + 1 < argc) name = argv[++i];
    else if (a == "--out" && i + 1 < argc) out_path = argv[++i];
    else if (a == "--device" && i + 1 < argc) dev = std::atoi(argv[++i]);
    else if (a == "--copy" && i + 1 < argc) copy_mib = std::atoi(argv[++i]);
    else if (a == "--resources" && i + 1 < argc) resources = argv[++i];
    else if (a == "--quick") quick = true;
    else {
      std::fprintf(stderr, "usage: bw_probe [--name N] [--out FILE] [--device N] [--quick] [--resources CSV] | "
                           "--copy MIB\n");
      return 2;
    }
  }
  CK(hipSetDevice(dev));
  if (copy_mib > 0) return copy_only(copy_mib);

  Device d;
  CK(hipGetDeviceProperties(&d.prop, dev));
  d.cus = d.prop.multiProcessorCount;
  d.wave = d.prop.warpSize;
  d.l2 = d.prop.l2CacheSize;
  (void)hipDeviceGetAttribute(&d.xcds, hipDeviceAttributeNumberOfXccs, dev);
  int max_wg_cu = 32;
  (void)hipDeviceGetAttribute(&max_wg_cu, hipDeviceAttributeMaxBlocksPerMultiProcessor, dev);
  // The MALL's size is not a device attribute; 256 MiB is MI355X's. It only
  // sizes working sets here (reads of 1 GiB windows, a 128 MiB cached set).
  const long long mall = 256LL << 20;
  const int reps = quick ? 5 : 15;
  std::printf("device %s (%s): %d CUs in %d XCDs, %d-lane waves, L2 %lld KiB per XCD, %.1f GB\n", d.prop.name,
              d.prop.gcnArchName, d.cus, d.xcds, d.wave, d.l2 / 1024, d.prop.totalGlobalMem / 1e9);
  std::fflush(stdout);

  int *sink;
  CK(hipMalloc(&sink, 1024 * sizeof(int)));
  const size_t buf_bytes = 4ull << 30;
  char *buf;
  CK(hipMalloc(&buf, buf_bytes));
  CK(hipMemset(buf, 0x11, buf_bytes));

  // ---- stream: the best sustained read rate ---------------------------------------------
  double bw_peak = 0;
  std::printf("stream: 1 GiB windows, GB/s by workgroups/CU x waves x loads in flight per lane\n");
  for (int per_cu : {1, 2, 4})
    for (int waves : {4, 8, 16}) {
      if (per_cu * waves * d.wave > d.prop.maxThreadsPerMultiProcessor) continue;
      std::printf("  %d x %2d waves:", per_cu, waves);
      for (int depth : {2, 4, 8, 16}) {
        const int wgs = d.cus * per_cu;
        const uint32_t quantum = (uint32_t)waves * depth * 1024;
        const uint32_t run = (uint32_t)((1ull << 30) / wgs / quantum * quantum);
        const double g = run_rate(depth, wgs, waves * d.wave, buf, buf_bytes, run, sink, reps);
        std::printf("  d%-2d %7.1f", depth, g);
        bw_peak = std::max(bw_peak, g);
      }
      std::printf("\n");
      std::fflush(stdout);
    }
  std::printf("  bw_peak_gbs = %.1f\n", bw_peak);

  // ---- curve: rate against bytes in flight per CU ------------------------------------------
  double bw_cu = 0;
  std::vector<int> counts = {1, 4, 16, 64, 128, d.cus};
  if (quick) counts = {1, d.cus};
  std::printf("curve: one workgroup of 16 waves per CU, GB/s by active CUs x KiB in flight per CU\n");
  for (int n : counts) {
    std::printf("  %4d CUs:", n);
    for (int depth : {2, 4, 8, 16}) {
      const uint32_t quantum = 16u * depth * 1024;
      const uint32_t run = std::max<uint32_t>(quantum, (uint32_t)std::min<size_t>(64ull << 20, (256ull << 20) / n) /
                                                           quantum * quantum);
      const double g = run_rate(depth, n, 1024, buf, buf_bytes, run, sink, reps);
      std::printf("  %4d KiB %7.1f", 16 * depth, g);
      if (n == 1) bw_cu = std::max(bw_cu, g);
    }
    std::printf("\n");
    std::fflush(stdout);
  }
  std::printf("  bw_sm_gbs = %.2f (one CU)\n", bw_cu);

  // ---- chase: dependent loads to lines nothing has touched -----------------------------------
  double lat = 0, lat_mall = 0;
  {
    const size_t region = 2ull << 30, lines = region / 128;
    std::vector<uint32_t> order(lines);
    std::iota(order.begin(), order.end(), 0u);
    std::mt19937_64 g(20260);
    std::shuffle(order.begin(), order.end(), g);
    std::vector<uint32_t> next(lines * 32, 0);
    for (size_t i = 0; i < lines; ++i) next[(size_t)order[i] * 32] = order[(i + 1) % lines];
    uint32_t *dnext, *dend;
    CK(hipMalloc(&dnext, next.size() * 4));
    CK(hipMalloc(&dend, 4));
    CK(hipMemcpy(dnext, next.data(), next.size() * 4, hipMemcpyHostToDevice));
    const int hops = quick ? 4000 : 16000;
    // the flush reads 1 GiB of the stream buffer: four times the MALL
    auto flush_all = [&](int) { launch_run<8>(d.cus * 2, 512, buf, (uint32_t)((1ull << 30) / (d.cus * 2)), sink); };
    size_t pos = 0;
    std::vector<double> cold, warm;
    Events e;
    for (int r = 0; r < (quick ? 4 : 10); ++r) {
      flush_all(r);
      CK(hipEventRecord(e.a, 0));
      hipLaunchKernelGGL(follow, dim3(1), dim3(1), 0, 0, dnext, order[pos], hops, dend);
      CK(hipEventRecord(e.b, 0));
      cold.push_back(e.us() * 1e3 / hops);
      // the same hops: L2 cleared by a 64 MiB read that allocates there
      // (8 MiB per XCD, twice its L2), the MALL keeps them
      hipLaunchKernelGGL((run_read<8, 0>), dim3(d.cus), dim3(512), 0, 0, buf + (1ull << 30),
                         (uint32_t)((64ull << 20) / d.cus), sink);
      CK(hipEventRecord(e.a, 0));
      hipLaunchKernelGGL(follow, dim3(1), dim3(1), 0, 0, dnext, order[pos], hops, dend);
      CK(hipEventRecord(e.b, 0));
      warm.push_back(e.us() * 1e3 / hops);
      pos = (pos + hops) % lines;
    }
    std::sort(cold.begin(), cold.end());
    std::sort(warm.begin(), warm.end());
    lat = cold[cold.size() / 2];
    lat_mall = warm[warm.size() / 2];
    std::printf("chase: %d hops per rep over 2 GiB; HBM %.0f ns, MALL %.0f ns per hop\n", hops, lat, lat_mall);
    CK(hipFree(dnext));
    CK(hipFree(dend));
  }
  std::fflush(stdout);

  // ---- trip: the floor of a kernel and of one memory round trip ----------------------------------
  double floor_us = 0, trip_us = 0;
  {
    const int wgs = d.cus;
    v4i *dst;
    CK(hipMalloc(&dst, (size_t)wgs * 256 * 16));
    floor_us = bound_us(100, [&](hipEvent_t a, hipEvent_t b, int) {
      hipExtLaunchKernelGGL(nothing, dim3(wgs), dim3(256), 0, 0, a, b, 0);
    });
    // each rep loads from a different 4 MiB of the stream buffer's last GiB,
    // which the chase's flushes never read
    const size_t slab = (size_t)wgs * 256 * 16;
    trip_us = bound_us(100, [&](hipEvent_t a, hipEvent_t b, int r) {
      const v4i *src = reinterpret_cast<const v4i *>(buf + (3ull << 30) + (size_t)(r % 200) * slab);
      hipExtLaunchKernelGGL(one_trip, dim3(wgs), dim3(256), 0, 0, a, b, 0, src, dst);
    });
    std::printf("trip: empty %d x 256 grid %.2f us, one cold load + store per lane %.2f us\n", wgs, floor_us,
                trip_us);
    CK(hipFree(dst));
  }

  // ---- cached: L2- and MALL-resident sets ------------------------------------------------------------
  const uint32_t l2_set = (uint32_t)std::max<long long>(1 << 20, d.l2 / 2);
  const int l2_passes = 100;
  const double l2_us = median_us(
      reps, [](int) {},
      [&](int) { hipLaunchKernelGGL(reread, dim3(d.cus * 4), dim3(256), 0, 0, buf, l2_set, l2_passes, sink); });
  // each workgroup reads the whole set `passes` times
  const double bw_l2 = (double)l2_set * l2_passes * d.cus * 4 / (l2_us * 1e3);
  const uint32_t mall_set = 128u << 20;
  const int mall_passes = 2;
  const double mall_us = median_us(
      reps, [](int) {},
      [&](int) { hipLaunchKernelGGL(reread, dim3(d.cus * 4), dim3(256), 0, 0, buf, mall_set, mall_passes, sink); });
  const double bw_mall = (double)mall_set * mall_passes * d.cus * 4 / (mall_us * 1e3);
  std::printf("cached: %u KiB set %.0f GB/s, %u MiB set %.0f GB/s\n", l2_set >> 10, bw_l2, mall_set >> 20, bw_mall);

  // ---- grain: bytes per access against stride --------------------------------------------------------
  int sector = 0;
  {
    std::printf("grain: bytes per dword access of cold memory at %.0f GB/s:", bw_peak);
    double prev = 0;
    const int lanes = d.cus * 8 * 256;
    for (uint32_t s : {16u, 32u, 64u, 128u, 256u, 512u}) {
      const int per = (int)std::min<size_t>(64, (1ull << 30) / ((size_t)lanes * s));
      const size_t span = (size_t)lanes * s * per;
      const double us = median_us(
          reps, [](int) {},
          [&](int r) {
            hipLaunchKernelGGL(sparse_read, dim3(d.cus * 8), dim3(256), 0, 0,
                               buf + (size_t)(r % 3) * (1ull << 30), s, per, sink);
          });
      const double bytes = us * 1e3 * bw_peak / ((double)lanes * per);
      std::printf("  %uB:%.0f", s, bytes);
      if (!sector && prev > 0 && bytes < 1.2 * prev) sector = (int)(s / 2);
      prev = bytes;
      (void)span;
    }
    if (!sector) sector = 512;
    std::printf("\n  sector_bytes = %d\n", sector);
  }

  // ---- fma, launch, copy ---------------------------------------------------------------------------------
  float *fout;
  CK(hipMalloc(&fout, (size_t)d.cus * 8 * 256 * 4));
  const int iters = 8192;
  const double f_us = median_us(
      reps, [](int) {}, [&](int) { hipLaunchKernelGGL(fma_rate, dim3(d.cus * 8), dim3(256), 0, 0, fout, iters); });
  const double gflops = 2.0 * 16 * iters * (double)d.cus * 8 * 256 / (f_us * 1e3);
  const double launch_us = median_us(200, [](int) {}, [&](int) { hipLaunchKernelGGL(nothing, dim3(1), dim3(64), 0, 0); });
  const size_t cbytes = 512ull << 20;
  const double c_us = median_us(reps, [](int) {}, [&](int r) {
    const v4i *src = reinterpret_cast<const v4i *>(buf + (size_t)(r % 2) * (1ull << 30));
    hipLaunchKernelGGL(copy16, dim3(d.cus * 8), dim3(256), 0, 0, src,
                       reinterpret_cast<v4i *>(buf + (2ull << 30) + (size_t)(r % 2) * cbytes), cbytes / 16);
  });
  const double bw_copy = 2.0 * cbytes / (c_us * 1e3);
  std::printf("fma %.0f GFLOP/s, launch %.2f us, copy %.0f GB/s (read + written)\n", gflops, launch_us, bw_copy);

  FILE *f = out_path.empty() ? stdout : std::fopen(out_path.c_str(), "w");
  if (!f) {
    std::fprintf(stderr, "cannot write %s\n", out_path.c_str());
    return 1;
  }
  std::fprintf(f, "# %s (%s), measured by kvforge_amd/bin/bw_probe\n", d.prop.name[0] ? d.prop.name : "GPU",
               d.prop.gcnArchName);
  std::fprintf(f, "# latency: HBM %.0f ns per dependent hop to an untouched line; MALL-resident %.0f ns\n", lat,
               lat_mall);
  std::fprintf(f, "name = %s\n", name.c_str());
  std::fprintf(f, "compute_capability = %d.%d\n", d.prop.major, d.prop.minor);
  std::fprintf(f, "dram_gb = %.1f\n", d.prop.totalGlobalMem / 1e9);
  std::fprintf(f, "sms = %d\n", d.cus);
  std::fprintf(f, "bw_peak_gbs = %.1f\n", bw_peak);
  std::fprintf(f, "bw_sm_gbs = %.2f\n", bw_cu);
  std::fprintf(f, "lat_ns = %.0f\n", lat);
  std::fprintf(f, "bw_l2_gbs = %.0f\n", bw_l2);
  std::fprintf(f, "l2_bytes = %lld\n", d.l2);
  std::fprintf(f, "sector_bytes = %d\n", sector);
  std::fprintf(f, "line_bytes = 128\n");
  std::fprintf(f, "f32_gflops = %.0f\n", gflops);
  std::fprintf(f, "launch_us = %.2f\n", launch_us);
  std::fprintf(f, "max_warps_per_sm = %d\n", d.prop.maxThreadsPerMultiProcessor / d.wave);
  std::fprintf(f, "max_blocks_per_sm = %d\n", max_wg_cu);
  std::fprintf(f, "regs_per_sm = %d\n", d.prop.regsPerMultiprocessor);
  std::fprintf(f, "wave_size = %d\n", d.wave);
  std::fprintf(f, "mall_bytes = %lld\n", mall);
  std::fprintf(f, "bw_mall_gbs = %.0f\n", bw_mall);
  std::fprintf(f, "lat_mall_ns = %.0f\n", lat_mall);
  std::fprintf(f, "bw_copy_gbs = %.0f\n", bw_copy);
  std::fprintf(f, "kernel_floor_us = %.2f\n", floor_us);
  if (!resources.empty()) std::fprintf(f, "resources = %s\n", resources.c_str());
  if (f != stdout) {
    std::fclose(f);
    std::printf("wrote %s\n", out_path.c_str());
  }
  CK(hipFree(fout));
  CK(hipFree(buf));
  CK(hipFree(sink));
  return 0;
}
