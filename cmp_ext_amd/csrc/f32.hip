// Instantiations of the fp32 MFMA GEMM.
#include "f32_kernel.h"
#include "f32_kwave_kernel.h"
#include "kernels.h"

namespace cmpext3 {
namespace {
template <bool KN, bool SPLITK, bool DMA16>
hipError_t launch(KernelId id, const GemmParams& p, dim3 grid, hipStream_t s) {
  switch (id) {
    case kF32Tile128:
      return launch_kernel((gemm_f32_kernel<KN, 128, 128, 2, 4, SPLITK, DMA16>), grid, dim3(256), 0, s, p);
    case kF32Tile96x64:
      return launch_kernel((gemm_f32_kernel<KN, 96, 64, 2, 8, SPLITK, DMA16>), grid, dim3(256), 0, s, p);
    case kF32Tile64:
      return launch_kernel((gemm_f32_kernel<KN, 64, 64, 2, 8, SPLITK, DMA16>), grid, dim3(256), 0, s, p);
    case kF32Tile64K4:
      return launch_kernel((gemm_f32_kwave_kernel<64, KN, 2, SPLITK, DMA16>), grid, dim3(256), 0, s, p);
    case kF32Tile16K4:
      return launch_kernel((gemm_f32_kwave_kernel<16, KN, 2, SPLITK, DMA16>), grid, dim3(256), 0, s, p);
    default:
      return hipErrorInvalidValue;
  }
}

template <bool DMA16>
hipError_t launch_dma(KernelId id, BLayout lay, const GemmParams& p, dim3 grid, hipStream_t s) {
  if (p.splits > 1)
    return lay == kKN ? launch<true, true, DMA16>(id, p, grid, s) : launch<false, true, DMA16>(id, p, grid, s);
  return lay == kKN ? launch<true, false, DMA16>(id, p, grid, s) : launch<false, false, DMA16>(id, p, grid, s);
}
}  // namespace

// p.splits > 1: grid.z = batch * splits, fp32 partials into p.partials.  dma16: the
// operands meet the 16-byte LDS-DMA conditions (checked by the selector).
hipError_t launch_f32(KernelId id, BLayout lay, bool dma16, const GemmParams& p, dim3 grid, hipStream_t s) {
  return dma16 ? launch_dma<true>(id, lay, p, grid, s) : launch_dma<false>(id, lay, p, grid, s);
}
}  // namespace cmpext3
