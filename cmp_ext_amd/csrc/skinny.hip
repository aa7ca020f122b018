// Instantiations of the skinny-M GEMM (M <= 64; B is [K, N], or [N, K] for the
// strips-of-W kernel).
#include "kernels.h"
#include "skinny_kernel.h"
#include "skinny_wide_kernel.h"

namespace cmpext3 {
namespace {
template <typename T>
hipError_t launch(int mb, const GemmParams& p, dim3 grid, hipStream_t s) {
  const dim3 block(256);
  switch (mb) {
    case 1: hipLaunchKernelGGL((gemm_skinny_narrow_kernel<T, 1>), grid, block, 0, s, p); break;
    case 2: hipLaunchKernelGGL((gemm_skinny_narrow_kernel<T, 2>), grid, block, 0, s, p); break;
    case 3: hipLaunchKernelGGL((gemm_skinny_narrow_kernel<T, 3>), grid, block, 0, s, p); break;
    case 4: hipLaunchKernelGGL((gemm_skinny_narrow_kernel<T, 4>), grid, block, 0, s, p); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}
}  // namespace

template <typename T, int SW>
hipError_t launch_nk(int mb, const GemmParams& p, dim3 grid, hipStream_t s) {
  const dim3 block(256);
  switch (mb) {  // 1 KB of each W row per stage for one 16-row block of A, 512 bytes otherwise
    case 1: hipLaunchKernelGGL((gemm_skinny_nk_kernel<T, 1, SW, 512>), grid, block, 0, s, p); break;
    case 2: hipLaunchKernelGGL((gemm_skinny_nk_kernel<T, 2, SW, 256>), grid, block, 0, s, p); break;
    case 3: hipLaunchKernelGGL((gemm_skinny_nk_kernel<T, 3, SW, 256>), grid, block, 0, s, p); break;
    case 4: hipLaunchKernelGGL((gemm_skinny_nk_kernel<T, 4, SW, 256>), grid, block, 0, s, p); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_skinny(DType dt, int mb, const GemmParams& p, dim3 grid, hipStream_t s) {
  if (dt == kF16) return launch<_Float16>(mb, p, grid, s);
  if (dt == kBF16) return launch<__bf16>(mb, p, grid, s);
  return hipErrorInvalidValue;
}

namespace {
template <typename T>
hipError_t launch_wide(int mb, const GemmParams& p, float* ws, int splits, int ksplit, dim3 grid, hipStream_t s) {
  const dim3 block(256);
  switch (mb) {
    case 1: hipLaunchKernelGGL((gemm_skinny_wide_kernel<T, 1>), grid, block, 0, s, p, ws, splits, ksplit); break;
    case 2: hipLaunchKernelGGL((gemm_skinny_wide_kernel<T, 2>), grid, block, 0, s, p, ws, splits, ksplit); break;
    case 3: hipLaunchKernelGGL((gemm_skinny_wide_kernel<T, 3>), grid, block, 0, s, p, ws, splits, ksplit); break;
    case 4: hipLaunchKernelGGL((gemm_skinny_wide_kernel<T, 4>), grid, block, 0, s, p, ws, splits, ksplit); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}
}  // namespace

hipError_t launch_skinny_wide(DType dt, int mb, const GemmParams& p, float* ws, int splits, int ksplit, dim3 grid,
                              hipStream_t s) {
  if (dt == kF16) return launch_wide<_Float16>(mb, p, ws, splits, ksplit, grid, s);
  if (dt == kBF16) return launch_wide<__bf16>(mb, p, ws, splits, ksplit, grid, s);
  return hipErrorInvalidValue;
}

hipError_t launch_skinny_reduce(DType dt, const GemmParams& p, const float* ws, int splits, int batch,
                                hipStream_t s) {
  const int64_t quads = (int64_t)batch * p.M * (p.N / 4);
  const dim3 grid((unsigned)((quads + 255) / 256));
  if (dt == kF16)
    hipLaunchKernelGGL((skinny_reduce_kernel<_Float16>), grid, dim3(256), 0, s, p, ws, splits, batch);
  else if (dt == kBF16)
    hipLaunchKernelGGL((skinny_reduce_kernel<__bf16>), grid, dim3(256), 0, s, p, ws, splits, batch);
  else
    hipLaunchKernelGGL((skinny_reduce_kernel<float>), grid, dim3(256), 0, s, p, ws, splits, batch);
  return hipGetLastError();
}
hipError_t launch_skinny_nk(DType dt, int mb, int strip, const GemmParams& p, dim3 grid, hipStream_t s) {
  if (dt == kF16) return strip == 16 ? launch_nk<_Float16, 16>(mb, p, grid, s) : launch_nk<_Float16, 32>(mb, p, grid, s);
  if (dt == kBF16) return strip == 16 ? launch_nk<__bf16, 16>(mb, p, grid, s) : launch_nk<__bf16, 32>(mb, p, grid, s);
  return hipErrorInvalidValue;
}
}  // namespace cmpext3
