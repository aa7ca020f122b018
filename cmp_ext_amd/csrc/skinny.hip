// Instantiations of the skinny-M GEMM (M <= 64, B is [K, N]).
#include "kernels.h"
#include "skinny_kernel.h"

namespace cmpext3 {
namespace {
constexpr int kPF = 4;  // K steps of loads in flight per wave

template <typename T>
hipError_t launch(int mb, const GemmParams& p, dim3 grid, hipStream_t s) {
  const dim3 block(kSkinnyWaves * 64);
  switch (mb) {
    case 1: hipLaunchKernelGGL((gemm_skinny_kernel<T, 1, kPF>), grid, block, 0, s, p); break;
    case 2: hipLaunchKernelGGL((gemm_skinny_kernel<T, 2, kPF>), grid, block, 0, s, p); break;
    case 3: hipLaunchKernelGGL((gemm_skinny_kernel<T, 3, kPF>), grid, block, 0, s, p); break;
    case 4: hipLaunchKernelGGL((gemm_skinny_kernel<T, 4, kPF>), grid, block, 0, s, p); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}
}  // namespace

hipError_t launch_skinny(DType dt, int mb, const GemmParams& p, dim3 grid, hipStream_t s) {
  if (dt == kF16) return launch<_Float16>(mb, p, grid, s);
  if (dt == kBF16) return launch<__bf16>(mb, p, grid, s);
  return hipErrorInvalidValue;
}
}  // namespace cmpext3
