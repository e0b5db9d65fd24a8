// kvf_hostdata.cpp - host-side test-data generation of the harness
// (libkvf_hostdata.so), the counterpart of the data and placement helpers in
// the reference's runtime/kvf_host.h:51-61 (make_data) and :156-165 (page
// table). The sweep, the driver and bench.py build their inputs with it.
//
// The definitions the reference does not have (outlier channels, variable
// lengths, a shared block pool) are this build's:
//   outliers  : iota(Hkv*D) shuffled by mt19937_64(seed), first
//               ceil(frac*Hkv*D) (kv_head*D + channel) entries, those K and V
//               columns multiplied by `factor`;
//   lengths   : lo + std::uniform_int_distribution<int>(0, hi-lo) on
//               mt19937_64(seed);
//   pool      : iota(pool) shuffled by mt19937_64(seed); sequence b takes the
//               next ceil(len_b/bt) pages in order, unused entries -1.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <numeric>
#include <random>
#include <vector>

extern "C" {

void kvfh_make_data(int B, int H, int Hkv, int D, int n, uint64_t seed, float *q, float *K,
                    float *V) {
  std::mt19937_64 rng(seed);
  std::normal_distribution<float> nd(0.f, 1.f);
  const long long nq = (long long)B * H * D, nk = (long long)B * Hkv * n * D;
  for (long long i = 0; i < nq; ++i) q[i] = nd(rng);
  for (long long i = 0; i < nk; ++i) K[i] = nd(rng);
  for (long long i = 0; i < nk; ++i) V[i] = nd(rng);
}

void kvfh_page_table(long long pages, uint64_t seed, int32_t *out) {
  std::vector<int> perm((size_t)pages);
  std::iota(perm.begin(), perm.end(), 0);
  std::mt19937_64 rng(seed);
  std::shuffle(perm.begin(), perm.end(), rng);
  std::copy(perm.begin(), perm.end(), out);
}

int kvfh_inject_outliers(int B, int Hkv, int D, int n, uint64_t seed, double frac, float factor,
                         float *K, float *V) {
  const int total = Hkv * D;
  const int count = (int)std::ceil(frac * total - 1e-9);
  std::vector<int> idx(total);
  std::iota(idx.begin(), idx.end(), 0);
  std::mt19937_64 rng(seed);
  std::shuffle(idx.begin(), idx.end(), rng);
  for (int i = 0; i < count; ++i) {
    const int h = idx[i] / D, c = idx[i] % D;
    for (int b = 0; b < B; ++b) {
      const long long base = ((long long)b * Hkv + h) * n * D + c;
      for (int t = 0; t < n; ++t) {
        K[base + (long long)t * D] *= factor;
        V[base + (long long)t * D] *= factor;
      }
    }
  }
  return count;
}

void kvfh_varlen_lengths(int B, int lo, int hi, uint64_t seed, int32_t *lens) {
  std::mt19937_64 rng(seed);
  std::uniform_int_distribution<int> u(0, hi - lo);
  for (int b = 0; b < B; ++b) lens[b] = lo + u(rng);
}

int kvfh_pool_table(int B, const int32_t *lens, int bt, int pool, uint64_t seed, int max_blocks,
                    int32_t *table) {
  std::vector<int> pages(pool);
  std::iota(pages.begin(), pages.end(), 0);
  std::mt19937_64 rng(seed);
  std::shuffle(pages.begin(), pages.end(), rng);
  int next = 0;
  for (int b = 0; b < B; ++b) {
    const int need = (lens[b] + bt - 1) / bt;
    for (int i = 0; i < max_blocks; ++i) {
      int32_t v = -1;
      if (i < need) {
        if (next >= pool) return -1;
        v = pages[next++];
      }
      table[(long long)b * max_blocks + i] = v;
    }
  }
  return next;
}

} // extern "C"
