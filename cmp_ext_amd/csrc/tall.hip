// Instantiations of the strips-of-W kernel with swapped roles (gemm_skinny_nk_kernel,
// SWAP): C = A B (+ bias) with N <= 128 and many rows of A, which stream through the
// workgroups in strips while the small B is re-read from L2 by each of them.
#include <stdint.h>

#include "kernels.h"
#include "skinny_kernel.h"

namespace cmpext3 {
namespace {
// KS = 128 k per stage: strip rows of 256 bytes, B k-rows of 64 or 128 columns; 32-row
// strips with B of 64 columns (chosen when there are few strips) take 256 k per stage in a
// ring of three 48 KiB stages (MI355X, B as [K, N]: 2048 x 64 x 2048 10.0 -> 8.8 us, 8192
// x 64 x 2048 10.5 -> 9.8 against 128 k in three 24 KiB stages, two workgroups per CU).
// B as [N, K] with N <= 16 or <= 32 (routers, low-rank adapters): one or two 16-row blocks
// of it and 256 k per stage (x[16384, 4096] W[8, 4096]^T 27.7 -> 23.6 us against four).
template <typename T, bool XKN, bool NT>
hipError_t launch_tall_t(int mb, int strip, const GemmParams& p, dim3 grid, hipStream_t s) {
  const dim3 block(256);
  if (mb == 4 && strip == 32)
    return launch_kernel((gemm_skinny_nk_kernel<T, 4, 32, 256, NT, 3, true, XKN>), grid, block, 0, s, p);
  if (mb == 4 && strip == 64)
    return launch_kernel((gemm_skinny_nk_kernel<T, 4, 64, 128, NT, 8, true, XKN>), grid, block, 0, s, p);
  if (!XKN && mb == 1 && strip == 32)
    return launch_kernel((gemm_skinny_nk_kernel<T, 1, 32, 256, NT, 3, true, false>), grid, block, 0, s, p);
  if (!XKN && mb == 1 && strip == 64)
    return launch_kernel((gemm_skinny_nk_kernel<T, 1, 64, 256, NT, 8, true, false>), grid, block, 0, s, p);
  if (!XKN && mb == 2 && strip == 32)
    return launch_kernel((gemm_skinny_nk_kernel<T, 2, 32, 256, NT, 3, true, false>), grid, block, 0, s, p);
  if (!XKN && mb == 2 && strip == 64)
    return launch_kernel((gemm_skinny_nk_kernel<T, 2, 64, 256, NT, 8, true, false>), grid, block, 0, s, p);
  if (mb == 8 && strip == 32)
    return launch_kernel((gemm_skinny_nk_kernel<T, 8, 32, 128, NT, 8, true, XKN>), grid, block, 0, s, p);
  if (mb == 8 && strip == 64)
    return launch_kernel((gemm_skinny_nk_kernel<T, 8, 64, 128, NT, 8, true, XKN>), grid, block, 0, s, p);
  return hipErrorInvalidValue;
}
template <typename T>
hipError_t launch_tall_t(BLayout lay, int mb, int strip, const GemmParams& p, dim3 grid, hipStream_t s) {
  const bool nt = stream_once(p.M, p.K, p.stride_a, grid.z);
  if (lay == kKN) return nt ? launch_tall_t<T, true, true>(mb, strip, p, grid, s) : launch_tall_t<T, true, false>(mb, strip, p, grid, s);
  return nt ? launch_tall_t<T, false, true>(mb, strip, p, grid, s) : launch_tall_t<T, false, false>(mb, strip, p, grid, s);
}
}  // namespace

hipError_t launch_tall(DType dt, BLayout lay, int mb, int strip, const GemmParams& p, dim3 grid, hipStream_t s) {
  // every column of C in the workgroup's block, one workgroup per strip of A's rows
  if (p.N > 16 * mb || grid.y != 1 || (int64_t)grid.x * strip < p.M) return hipErrorInvalidValue;
  if (dt == kF16) return launch_tall_t<_Float16>(lay, mb, strip, p, grid, s);
  if (dt == kBF16) return launch_tall_t<__bf16>(lay, mb, strip, p, grid, s);
  return hipErrorInvalidValue;
}

}  // namespace cmpext3
