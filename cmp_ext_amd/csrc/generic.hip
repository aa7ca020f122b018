// Instantiations of the any-shape f16/bf16 GEMM.
#include "generic_kernel.h"
#include "kernels.h"

namespace cmpext3 {
namespace {
template <typename T>
hipError_t launch(BLayout lay, const GemmParams& p, dim3 grid, hipStream_t s) {
  if (lay == kKN) return launch_kernel((gemm_generic_kernel<T, true>), grid, dim3(256), 0, s, p);
  return launch_kernel((gemm_generic_kernel<T, false>), grid, dim3(256), 0, s, p);
}
}  // namespace

hipError_t launch_generic(DType dt, BLayout lay, const GemmParams& p, dim3 grid, hipStream_t s) {
  if (dt == kF16) return launch<_Float16>(lay, p, grid, s);
  if (dt == kBF16) return launch<__bf16>(lay, p, grid, s);
  return hipErrorInvalidValue;
}
}  // namespace cmpext3
