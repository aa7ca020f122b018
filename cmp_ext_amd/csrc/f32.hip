// Instantiations of the fp32 MFMA GEMM.
#include "f32_kernel.h"
#include "kernels.h"

namespace cmpext3 {
namespace {
template <bool KN, bool SPLITK>
hipError_t launch(KernelId id, const GemmParams& p, dim3 grid, hipStream_t s) {
  switch (id) {
    case kF32Tile128:
      hipLaunchKernelGGL((gemm_f32_kernel<KN, 128, 128, 2, 4, SPLITK>), grid, dim3(256), 0, s, p);
      break;
    case kF32Tile96x64:
      hipLaunchKernelGGL((gemm_f32_kernel<KN, 96, 64, 2, 8, SPLITK>), grid, dim3(256), 0, s, p);
      break;
    case kF32Tile64:
      hipLaunchKernelGGL((gemm_f32_kernel<KN, 64, 64, 2, 8, SPLITK>), grid, dim3(256), 0, s, p);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}
}  // namespace

// p.splits > 1: grid.z = batch * splits, fp32 partials into p.partials.
hipError_t launch_f32(KernelId id, BLayout lay, const GemmParams& p, dim3 grid, hipStream_t s) {
  if (p.splits > 1) return lay == kKN ? launch<true, true>(id, p, grid, s) : launch<false, true>(id, p, grid, s);
  return lay == kKN ? launch<true, false>(id, p, grid, s) : launch<false, false>(id, p, grid, s);
}
}  // namespace cmpext3
