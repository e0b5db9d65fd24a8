// kvf_merge.hip - the stand-alone split merge (decode_merge, and
// decode_merge_sliced past one chunk of splits) and its launcher.
//
// This translation unit is built with -amdgpu-kernarg-preload-count=10: the
// merge kernels' arguments (two partial-buffer pointers, two output pointers,
// H, splits: 10 dwords) arrive in SGPRs when the wave starts, so its first
// loads do not wait for the kernel-argument segment. (The split kernels take
// the fields their first loads need as 14 leading dwords ahead of Args, built
// with a preload count of 14; preloading Args' own first fields, pointers
// only, had measured no gain.) Measured on MI355X (three alternating rounds), the
// decode step went from 9.02 to 8.73 us at n = 4096 and from 18.40 to 18.18 us
// at GQA 32/8, d128, n 32768, int8:64, 32 splits.
#include "kvf_kernels.hpp"

namespace kvf {
namespace gfx950 {

template <int D> hipError_t launch_merge_kernel(const Args &a, const Ext &x, hipStream_t st) {
  const dim3 grid(a.H, a.B);
  const float *po = (const float *)a.part_o, *pml = (const float *)a.part_ml;
  // one chunk of MERGE_CHUNK splits: one slice; more: up to 8 slices, one
  // chunk each while the splits fit
  const int chunks = (a.splits + MERGE_CHUNK - 1) / MERGE_CHUNK;
  if (chunks <= 1)
    hipLaunchKernelGGL((decode_merge<D>), grid, dim3(D), 0, st, po, pml, a.out, x.out16, a.H, a.splits);
  else if (chunks == 2)
    hipLaunchKernelGGL((decode_merge_sliced<D, 2>), grid, dim3(2 * D), 0, st, po, pml, a.out, x.out16, a.H,
                       a.splits);
  else if (chunks <= 4)
    hipLaunchKernelGGL((decode_merge_sliced<D, 4>), grid, dim3(4 * D), 0, st, po, pml, a.out, x.out16, a.H,
                       a.splits);
  else
    hipLaunchKernelGGL((decode_merge_sliced<D, 8>), grid, dim3(8 * D), 0, st, po, pml, a.out, x.out16, a.H,
                       a.splits);
  return hipGetLastError();
}

template hipError_t launch_merge_kernel<64>(const Args &, const Ext &, hipStream_t);
template hipError_t launch_merge_kernel<128>(const Args &, const Ext &, hipStream_t);

} // namespace gfx950
} // namespace kvf
