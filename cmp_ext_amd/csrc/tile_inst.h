// Instantiation of the four f16/bf16 tile shapes for one (element type, B layout,
// K check) -- one translation unit per combination, so that they build in
// parallel: 256 x 256 and 256 x 224 tiles with 8 waves and one workgroup per CU
// (128 KiB of LDS); 128 x 128 tiles with 4 waves and two workgroups per CU;
// 64 x 256 tiles (M <= 64, short K) with 4 waves and two workgroups per CU.
#pragma once

#include "kernels.h"
#include "tile16_kernel.h"

namespace cmpext3 {

template <typename T, bool KN, bool KCHECK>
hipError_t launch_tiles(KernelId id, const GemmParams& p, dim3 grid, hipStream_t s) {
  switch (id) {
    case kTile256x256:
      return launch_tile16_k<T, KN, 256, 256, 4, 2, 1, KCHECK>(p, grid, s);
    case kTile256x224:
      return launch_tile16_k<T, KN, 256, 224, 4, 2, 1, KCHECK>(p, grid, s);
    case kTile128x128:
      return launch_tile16_k<T, KN, 128, 128, 2, 2, 2, KCHECK>(p, grid, s);
    case kTile64x256:
      return launch_tile16_k<T, KN, 64, 256, 1, 4, 2, KCHECK>(p, grid, s);
    default:
      return hipErrorInvalidValue;
  }
}

}  // namespace cmpext3

#define CMPEXT3_TILE_TU(NAME, T, KN, KCHECK)                                               \
  namespace cmpext3 {                                                                      \
  hipError_t NAME(KernelId id, const GemmParams& p, dim3 grid, hipStream_t s) {            \
    return launch_tiles<T, KN, KCHECK>(id, p, grid, s);                                    \
  }                                                                                        \
  }
