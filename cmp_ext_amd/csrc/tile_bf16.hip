// Instantiations of the tiled MFMA GEMM for bf16.
#include "kernels.h"
#include "tile16_kernel.h"
#include "tile_kernel.h"

namespace cmpext3 {
namespace {
template <bool KN>
hipError_t launch(KernelId id, const GemmParams& p, dim3 grid, hipStream_t s) {
  switch (id) {
    case kTile256x256:
      launch_tile16<__bf16, KN, 256, 256>(p, grid, s);
      break;
    case kTile256x224:
      launch_tile16<__bf16, KN, 256, 224>(p, grid, s);
      break;
    case kTile128x128:
      hipLaunchKernelGGL((gemm_tile_kernel<__bf16, KN, 128, 128, 2, 2, 5>), grid, dim3(256), 0, s, p);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}
}  // namespace

hipError_t launch_tile_bf16(KernelId id, BLayout lay, const GemmParams& p, dim3 grid, hipStream_t s) {
  return lay == kKN ? launch<true>(id, p, grid, s) : launch<false>(id, p, grid, s);
}
}  // namespace cmpext3
