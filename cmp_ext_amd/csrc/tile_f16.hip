// Instantiations of the tiled MFMA GEMM for fp16: 256 x 256 and 256 x 224
// tiles with 8 waves and one workgroup per CU (128 KB of LDS); 128 x 128 tiles
// with 4 waves and two workgroups per CU; 64 x 256 tiles (M <= 64, short K) with
// 4 waves and two workgroups per CU.
#include "kernels.h"
#include "tile16_kernel.h"

namespace cmpext3 {
namespace {
template <bool KN>
hipError_t launch(KernelId id, const GemmParams& p, dim3 grid, hipStream_t s) {
  switch (id) {
    case kTile256x256:
      launch_tile16<_Float16, KN, 256, 256, 4, 2, 1>(p, grid, s);
      break;
    case kTile256x224:
      launch_tile16<_Float16, KN, 256, 224, 4, 2, 1>(p, grid, s);
      break;
    case kTile128x128:
      launch_tile16<_Float16, KN, 128, 128, 2, 2, 2>(p, grid, s);
      break;
    case kTile64x256:
      launch_tile16<_Float16, KN, 64, 256, 1, 4, 2>(p, grid, s);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}
}  // namespace

hipError_t launch_tile_f16(KernelId id, BLayout lay, const GemmParams& p, dim3 grid, hipStream_t s) {
  return lay == kKN ? launch<true>(id, p, grid, s) : launch<false>(id, p, grid, s);
}
}  // namespace cmpext3
