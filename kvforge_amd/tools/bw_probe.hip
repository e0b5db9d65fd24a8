// bw_probe - measure the MI355X parameters the KVForge cost model depends on.
//
// The counterpart of the reference's bench/bw_probe.cu (machine-file writer,
// bench/bw_probe.cu:140-262), written for CDNA: 64-lane wavefronts, compute
// units (CUs) grouped into XCDs with a private L2 each, and a memory-side
// Infinity Cache (MALL) in front of HBM. Every figure is measured, none is
// taken from a datasheet:
//
//   bw_peak_gbs   sustained HBM read bandwidth over a region 8x the MALL
//   bw_sm_gbs     read bandwidth of ONE CU with ample waves in flight
//   lat_ns        HBM load-to-use latency (dependent pointer chase, idle)
//   bw_l2_gbs     aggregate read bandwidth of a working set that fits L2
//   bw_mall_gbs   aggregate read bandwidth of a working set that fits the
//                 MALL but not L2 (new key)
//   f32_gflops    sustained FP32 FMA throughput
//   launch_us     event-measured duration of an empty kernel
//   sector_bytes  transaction granularity, from a strided-read test
//   bif table     bandwidth against bytes in flight per CU and active CUs,
//                 printed for the cost model's Little's-law term
//
// The kernels are pure streaming reads, because that is what decode attention
// does to the KV cache: touch every byte once, in order, never come back.
//
//   bw_probe [--name NAME] [--out machines/mi355x.gpu] [--device N] [--quick]
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <numeric>
#include <random>
#include <string>
#include <vector>

#define CK(call)                                                                   \
  do {                                                                             \
    hipError_t e__ = (call);                                                       \
    if (e__ != hipSuccess) {                                                       \
      std::fprintf(stderr, "HIP error %s at %s:%d\n", hipGetErrorString(e__),      \
                   __FILE__, __LINE__);                                            \
      std::exit(1);                                                                \
    }                                                                              \
  } while (0)

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// ------------------------------------------------------------------ kernels
// Grid-stride read of 16-byte vectors, UNROLL independent loads in flight per
// lane; NT selects nontemporal loads. The xor is a sink so the loads stay.
template <int UNROLL, bool NT>
__global__ void stream_read(const u32x4 *__restrict__ p, size_t n_vec, unsigned *sink) {
  unsigned acc = 0;
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  for (; i + (UNROLL - 1) * stride < n_vec; i += UNROLL * stride) {
    u32x4 v[UNROLL];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u)
      v[u] = NT ? __builtin_nontemporal_load(p + i + (size_t)u * stride) : p[i + (size_t)u * stride];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  if (acc == 0x9e3779b9u) *sink = acc; // practically never true
}

// Each block streams its own contiguous slice (no grid stride), so the bytes
// in flight per CU are exactly blocks_per_cu * threads * UNROLL * 16.
template <int UNROLL>
__global__ void slice_read(const u32x4 *__restrict__ p, size_t vec_per_block, unsigned *sink) {
  unsigned acc = 0;
  const u32x4 *q = p + (size_t)blockIdx.x * vec_per_block;
  for (size_t i = threadIdx.x; i + (UNROLL - 1) * blockDim.x < vec_per_block;
       i += UNROLL * blockDim.x) {
    u32x4 v[UNROLL];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) v[u] = __builtin_nontemporal_load(q + i + (size_t)u * blockDim.x);
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  if (acc == 0x9e3779b9u) *sink = acc;
}

// One lane chases a random cycle of 128-byte lines.
__global__ void chase(const unsigned *next, unsigned start, int steps, unsigned *out) {
  unsigned i = start;
  for (int s = 0; s < steps; ++s) i = next[(size_t)i * 32];
  *out = i;
}

// Repeated reads of a small region (L2 or MALL resident).
__global__ void cached_read(const u32x4 *__restrict__ p, size_t n_vec, int passes, unsigned *sink) {
  unsigned acc = 0;
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (int r = 0; r < passes; ++r)
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n_vec; i += stride) {
      const u32x4 v = p[i];
      acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
  if (acc == 0x9e3779b9u) *sink = acc;
}

// Eight independent FMA chains per lane.
__global__ void fma_chain(float *out, int iters) {
  float a0 = threadIdx.x, a1 = a0 + 1, a2 = a0 + 2, a3 = a0 + 3;
  float a4 = a0 + 4, a5 = a0 + 5, a6 = a0 + 6, a7 = a0 + 7;
  const float m = 1.0000001f, c = 1e-7f;
  for (int i = 0; i < iters; ++i) {
    a0 = fmaf(a0, m, c); a1 = fmaf(a1, m, c); a2 = fmaf(a2, m, c); a3 = fmaf(a3, m, c);
    a4 = fmaf(a4, m, c); a5 = fmaf(a5, m, c); a6 = fmaf(a6, m, c); a7 = fmaf(a7, m, c);
  }
  out[(size_t)blockIdx.x * blockDim.x + threadIdx.x] = a0 + a1 + a2 + a3 + a4 + a5 + a6 + a7;
}

__global__ void empty_kernel() {}

// Plain copy of n_vec 16-byte vectors: the calibration kernel for the
// FETCH_SIZE / WRITE_SIZE counters (known bytes read and written).
__global__ void copy_kernel(const u32x4 *__restrict__ src, u32x4 *__restrict__ dst, size_t n_vec) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n_vec; i += stride)
    __builtin_nontemporal_store(__builtin_nontemporal_load(src + i), dst + i);
}

// One 16-byte load and one store per lane: a single memory round trip.
__global__ void one_trip(const u32x4 *__restrict__ p, unsigned *out) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const u32x4 v = __builtin_nontemporal_load(p + i);
  out[i] = v.x ^ v.w;
}

// 4-byte reads at a byte stride: time per access grows with the number of
// distinct transactions and stops once every access owns one.
__global__ void stride_read(const char *p, size_t n_access, int stride, unsigned *sink) {
  unsigned acc = 0;
  const size_t step = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n_access; i += step)
    acc ^= __builtin_nontemporal_load(reinterpret_cast<const unsigned *>(p + i * (size_t)stride));
  if (acc == 0x9e3779b9u) *sink = acc;
}

// ------------------------------------------------------------------ helpers
struct Timer {
  hipEvent_t a, b;
  Timer() { CK(hipEventCreate(&a)); CK(hipEventCreate(&b)); }
  ~Timer() { (void)hipEventDestroy(a); (void)hipEventDestroy(b); }
  void start() { CK(hipEventRecord(a, 0)); }
  double stop_us() {
    CK(hipEventRecord(b, 0));
    CK(hipEventSynchronize(b));
    float ms = 0;
    CK(hipEventElapsedTime(&ms, a, b));
    return ms * 1000.0;
  }
};

template <class F> double best_us(F &&f, int warm, int reps) {
  Timer t;
  double best = 1e30;
  for (int i = 0; i < warm + reps; ++i) {
    t.start();
    f();
    CK(hipGetLastError());
    const double us = t.stop_us();
    if (i >= warm) best = std::min(best, us);
  }
  return best;
}

template <class F> double median_us(F &&f, int warm, int reps) {
  Timer t;
  std::vector<double> v;
  for (int i = 0; i < warm + reps; ++i) {
    t.start();
    f();
    CK(hipGetLastError());
    const double us = t.stop_us();
    if (i >= warm) v.push_back(us);
  }
  std::sort(v.begin(), v.end());
  return v[v.size() / 2];
}

template <int U>
double slice_gbs(const u32x4 *big, size_t big_vec, int blocks, int threads, unsigned *sink) {
  // every block gets the same slice length; the total stays inside `big`
  const size_t per = std::min<size_t>(big_vec / blocks, (size_t)threads * U * 64);
  const double us = best_us(
      [&] { hipLaunchKernelGGL((slice_read<U>), dim3(blocks), dim3(threads), 0, 0, big, per, sink); },
      1, 3);
  return (double)per * 16 * blocks / (us * 1e3);
}

int main(int argc, char **argv) {
  std::string name = "mi355x", out_path;
  int dev = 0;
  bool quick = false;
  for (int i = 1; i < argc; ++i) {
    const std::string a = argv[i];
    if (a == "--name" && i + 1 < argc) name = argv[++i];
    else if (a == "--out" && i + 1 < argc) out_path = argv[++i];
    else if (a == "--device" && i + 1 < argc) dev = std::atoi(argv[++i]);
    else if (a == "--quick") quick = true;
    else {
      std::fprintf(stderr, "usage: bw_probe [--name N] [--out FILE] [--device N] [--quick]\n");
      return 2;
    }
  }
  CK(hipSetDevice(dev));
  hipDeviceProp_t prop;
  CK(hipGetDeviceProperties(&prop, dev));
  const int cus = prop.multiProcessorCount;
  const int wave = prop.warpSize;
  const int max_waves_cu = prop.maxThreadsPerMultiProcessor / wave;
  int max_blocks_cu = 32;
  (void)hipDeviceGetAttribute(&max_blocks_cu, hipDeviceAttributeMaxBlocksPerMultiProcessor, dev);
  const long long l2 = prop.l2CacheSize;
  // The Infinity Cache (MALL) size is not in hipDeviceProp_t; 256 MiB is the
  // MI355X's. It only sizes the working sets below (region >> MALL).
  const long long mall = 256LL << 20;
  std::printf("probing %s (%s): %d CUs, wave %d, %.1f GB HBM, L2 %lld KiB per XCD, %d MHz\n",
              prop.name, prop.gcnArchName, cus, wave, prop.totalGlobalMem / 1e9, l2 / 1024,
              prop.clockRate / 1000);
  std::fflush(stdout);

  unsigned *sink;
  CK(hipMalloc(&sink, 4));

  // ---- peak HBM bandwidth: 2 GiB, far past the MALL, several launch shapes ---------
  const size_t big_bytes = 2ull << 30;
  const size_t big_vec = big_bytes / 16;
  u32x4 *big;
  CK(hipMalloc(&big, big_bytes));
  CK(hipMemset(big, 1, big_bytes));
  double bw_peak = 0;
  int best_bpc = 0, best_thr = 0;
  for (int bpc : {1, 2, 4, 8})
    for (int threads : {256, 512, 1024}) {
      if (bpc * threads > prop.maxThreadsPerMultiProcessor) continue;
      const int blocks = cus * bpc;
      const double us = best_us(
          [&] { hipLaunchKernelGGL((stream_read<8, true>), dim3(blocks), dim3(threads), 0, 0, big, big_vec, sink); },
          2, quick ? 3 : 6);
      const double g = big_bytes / (us * 1e3);
      std::printf("  stream nt u8  blocks/CU %d x %4d threads: %7.1f GB/s\n", bpc, threads, g);
      if (g > bw_peak) { bw_peak = g; best_bpc = bpc; best_thr = threads; }
    }
  {
    const double us = best_us(
        [&] { hipLaunchKernelGGL((stream_read<8, false>), dim3(cus * best_bpc), dim3(best_thr), 0, 0, big, big_vec, sink); },
        2, quick ? 3 : 6);
    std::printf("  stream plain  (best shape)        : %7.1f GB/s\n", big_bytes / (us * 1e3));
    const double us16 = best_us(
        [&] { hipLaunchKernelGGL((stream_read<16, true>), dim3(cus * best_bpc), dim3(best_thr), 0, 0, big, big_vec, sink); },
        2, quick ? 3 : 6);
    const double g16 = big_bytes / (us16 * 1e3);
    std::printf("  stream nt u16 (best shape)        : %7.1f GB/s\n", g16);
    bw_peak = std::max(bw_peak, g16);
  }
  std::printf("  bw_peak  = %.1f GB/s\n", bw_peak);
  std::fflush(stdout);

  // ---- bytes in flight: bandwidth against active CUs and bytes in flight per CU ----
  std::printf("  bif table: active CUs x KiB in flight per CU -> GB/s\n");
  double bw_cu = 0;
  {
    const int thr = 1024;
    std::vector<int> cu_counts = {1, 8, 32, 64, 128, cus};
    if (quick) cu_counts = {1, cus};
    for (int ncu : cu_counts) {
      std::printf("   %4d CUs:", ncu);
      for (int u : {1, 2, 4, 8}) {
        double g = 0;
        switch (u) {
        case 1: g = slice_gbs<1>(big, big_vec, ncu, thr, sink); break;
        case 2: g = slice_gbs<2>(big, big_vec, ncu, thr, sink); break;
        case 4: g = slice_gbs<4>(big, big_vec, ncu, thr, sink); break;
        default: g = slice_gbs<8>(big, big_vec, ncu, thr, sink); break;
        }
        std::printf("  %4d KiB %7.1f", thr * u * 16 / 1024, g);
        if (ncu == 1) bw_cu = std::max(bw_cu, g);
      }
      std::printf("\n");
      std::fflush(stdout);
    }
  }
  std::printf("  bw_sm    = %.2f GB/s (one CU)\n", bw_cu);

  // ---- HBM latency: one lane chasing a random cycle over 1 GiB --------------------------
  double lat_ns = 0, lat_mall_ns = 0;
  {
    const size_t region = 1ull << 30;
    const size_t lines = region / 128;
    std::vector<unsigned> perm(lines);
    std::iota(perm.begin(), perm.end(), 0u);
    std::mt19937_64 rng(7);
    std::shuffle(perm.begin(), perm.end(), rng);
    std::vector<unsigned> nxt(lines * 32, 0);
    for (size_t i = 0; i < lines; ++i) nxt[(size_t)perm[i] * 32] = perm[(i + 1) % lines];
    unsigned *dnext, *dout;
    CK(hipMalloc(&dnext, nxt.size() * 4));
    CK(hipMalloc(&dout, 4));
    CK(hipMemcpy(dnext, nxt.data(), nxt.size() * 4, hipMemcpyHostToDevice));
    const int steps = quick ? 20000 : 100000;
    const double us = best_us(
        [&] { hipLaunchKernelGGL(chase, dim3(1), dim3(1), 0, 0, dnext, perm[0], steps, dout); }, 1, 3);
    lat_ns = us * 1e3 / steps;
    std::printf("  lat      = %.0f ns (HBM, idle)\n", lat_ns);
    // a 64 MiB cycle: resident in the MALL after the first pass
    const size_t mlines = (64ull << 20) / 128;
    std::vector<unsigned> mp(mlines);
    std::iota(mp.begin(), mp.end(), 0u);
    std::shuffle(mp.begin(), mp.end(), rng);
    std::vector<unsigned> mn(mlines * 32, 0);
    for (size_t i = 0; i < mlines; ++i) mn[(size_t)mp[i] * 32] = mp[(i + 1) % mlines];
    CK(hipMemcpy(dnext, mn.data(), mn.size() * 4, hipMemcpyHostToDevice));
    const int msteps = (int)std::min<size_t>(mlines * 2, 200000);
    const double mus = best_us(
        [&] { hipLaunchKernelGGL(chase, dim3(1), dim3(1), 0, 0, dnext, mp[0], msteps, dout); }, 1, 3);
    lat_mall_ns = mus * 1e3 / msteps;
    std::printf("  lat_mall = %.0f ns (64 MiB cycle, cache resident)\n", lat_mall_ns);
    CK(hipFree(dnext));
    CK(hipFree(dout));
  }
  std::fflush(stdout);

  // ---- copy: 512 MiB read + 512 MiB written (counter calibration) ---------------------
  double bw_copy = 0;
  {
    const size_t cbytes = 512ull << 20;
    const double us = best_us(
        [&] { hipLaunchKernelGGL(copy_kernel, dim3(cus * 4), dim3(256), 0, 0, big, big + (cbytes / 16), cbytes / 16); },
        1, 3);
    bw_copy = 2.0 * cbytes / (us * 1e3);
    std::printf("  copy     = %.0f GB/s (512 MiB read + 512 MiB written per launch)\n", bw_copy);
  }

  // ---- L2 and MALL bandwidth: working sets that fit each level ---------------------------
  const size_t l2_ws = (size_t)std::max<long long>(1 << 20, l2 / 2);
  const int l2_passes = 200;
  const double l2_us = best_us(
      [&] { hipLaunchKernelGGL(cached_read, dim3(cus * 4), dim3(256), 0, 0, big, l2_ws / 16, l2_passes, sink); },
      1, 4);
  const double bw_l2 = l2_ws * (double)l2_passes / (l2_us * 1e3);
  std::printf("  bw_l2    = %.0f GB/s (%zu KiB working set)\n", bw_l2, l2_ws / 1024);
  const size_t mall_ws = 128ull << 20;
  const int mall_passes = 8;
  const double mall_us = best_us(
      [&] { hipLaunchKernelGGL(cached_read, dim3(cus * 4), dim3(1024), 0, 0, big, mall_ws / 16, mall_passes, sink); },
      1, 4);
  const double bw_mall = mall_ws * (double)mall_passes / (mall_us * 1e3);
  std::printf("  bw_mall  = %.0f GB/s (%zu MiB working set)\n", bw_mall, mall_ws >> 20);

  // ---- FP32 throughput -----------------------------------------------------------------
  float *fout;
  CK(hipMalloc(&fout, (size_t)cus * 8 * 256 * 4));
  const int fiters = 20000;
  const double f_us = best_us(
      [&] { hipLaunchKernelGGL(fma_chain, dim3(cus * 8), dim3(256), 0, 0, fout, fiters); }, 1, 4);
  const double gflops = 2.0 * 8 * fiters * (double)cus * 8 * 256 / (f_us * 1e3);
  std::printf("  f32      = %.0f GFLOP/s\n", gflops);

  // ---- launch overhead: an empty kernel timed with events -------------------------------
  const double launch_us = median_us([&] { hipLaunchKernelGGL(empty_kernel, dim3(1), dim3(64), 0, 0); }, 20, 200);
  std::printf("  launch   = %.2f us\n", launch_us);
  // the same, timed by events bound to the kernel's own dispatch (what a
  // kernel trace reports), for a full-chip grid: the floor of any kernel
  double floor_us = 0, trip_us = 0;
  {
    hipEvent_t e0, e1;
    CK(hipEventCreate(&e0));
    CK(hipEventCreate(&e1));
    unsigned *tout;
    CK(hipMalloc(&tout, (size_t)cus * 256 * 4));
    std::vector<double> v, w;
    for (int i = 0; i < 120; ++i) {
      hipExtLaunchKernelGGL(empty_kernel, dim3(cus), dim3(256), 0, 0, e0, e1, 0);
      CK(hipEventSynchronize(e1));
      float ms = 0;
      CK(hipEventElapsedTime(&ms, e0, e1));
      if (i >= 20) v.push_back(ms * 1e3);
      hipExtLaunchKernelGGL(one_trip, dim3(cus), dim3(256), 0, 0, e0, e1, 0, (const u32x4 *)big + (size_t)(i % 64) * cus * 256, tout);
      CK(hipEventSynchronize(e1));
      CK(hipEventElapsedTime(&ms, e0, e1));
      if (i >= 20) w.push_back(ms * 1e3);
    }
    std::sort(v.begin(), v.end());
    std::sort(w.begin(), w.end());
    floor_us = v[v.size() / 2];
    trip_us = w[w.size() / 2];
    std::printf("  kernel floor = %.2f us (empty, %d x 256), one round trip = %.2f us\n", floor_us, cus, trip_us);
    CK(hipFree(tout));
    CK(hipEventDestroy(e0));
    CK(hipEventDestroy(e1));
  }

  // ---- transaction size: time per 4-byte access against byte stride -----------------------
  const size_t n_acc = 8u << 20;
  std::vector<std::pair<int, double>> st;
  for (int s : {4, 8, 16, 32, 64, 128, 256}) {
    const double us = best_us(
        [&] { hipLaunchKernelGGL(stride_read, dim3(cus * 8), dim3(256), 0, 0, (const char *)big, n_acc, s, sink); },
        1, 4);
    st.push_back({s, us * 1e3 / n_acc});
  }
  const double ref = st.back().second;
  int sector = 256;
  for (auto &p : st)
    if (p.second >= 0.9 * ref) { sector = p.first; break; }
  std::printf("  stride test (ns per 4 B access):");
  for (auto &p : st) std::printf("  %dB:%.4f", p.first, p.second);
  std::printf("\n  sector   = %d B\n", sector);

  const char *path = out_path.empty() ? nullptr : out_path.c_str();
  FILE *f = path ? std::fopen(path, "w") : stdout;
  if (!f) { std::fprintf(stderr, "cannot write %s\n", path); return 1; }
  std::fprintf(f, "# Measured by kvforge_amd/tools/bw_probe on %s (%s)\n", prop.name, prop.gcnArchName);
  std::fprintf(f, "# stride test, ns per 4-byte access:");
  for (auto &p : st) std::fprintf(f, "  %dB=%.4f", p.first, p.second);
  std::fprintf(f, "\n# HBM latency %.0f ns idle; MALL-resident chase %.0f ns\n", lat_ns, lat_mall_ns);
  std::fprintf(f, "name = %s\n", name.c_str());
  std::fprintf(f, "compute_capability = %d.%d\n", prop.major, prop.minor);
  std::fprintf(f, "dram_gb = %.1f\n", prop.totalGlobalMem / 1e9);
  std::fprintf(f, "sms = %d\n", cus);
  std::fprintf(f, "bw_peak_gbs = %.1f\n", bw_peak);
  std::fprintf(f, "bw_sm_gbs = %.2f\n", bw_cu);
  std::fprintf(f, "lat_ns = %.0f\n", lat_ns);
  std::fprintf(f, "bw_l2_gbs = %.0f\n", bw_l2);
  std::fprintf(f, "l2_bytes = %lld\n", l2);
  std::fprintf(f, "sector_bytes = %d\n", sector);
  std::fprintf(f, "line_bytes = 128\n");
  std::fprintf(f, "f32_gflops = %.0f\n", gflops);
  std::fprintf(f, "launch_us = %.2f\n", launch_us);
  std::fprintf(f, "max_warps_per_sm = %d\n", max_waves_cu);
  std::fprintf(f, "max_blocks_per_sm = %d\n", max_blocks_cu);
  std::fprintf(f, "regs_per_sm = %d\n", prop.regsPerMultiprocessor);
  std::fprintf(f, "wave_size = %d\n", wave);
  std::fprintf(f, "mall_bytes = %lld\n", mall);
  std::fprintf(f, "bw_mall_gbs = %.0f\n", bw_mall);
  std::fprintf(f, "lat_mall_ns = %.0f\n", lat_mall_ns);
  std::fprintf(f, "bw_copy_gbs = %.0f\n", bw_copy);
  std::fprintf(f, "kernel_floor_us = %.2f\n", floor_us);
  std::fprintf(f, "round_trip_us = %.2f\n", trip_us);
  if (path) {
    std::fclose(f);
    std::printf("wrote %s\n", path);
  }
  CK(hipFree(big));
  CK(hipFree(fout));
  CK(hipFree(sink));
  return 0;
}
