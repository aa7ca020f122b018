// Launcher of the short-K streaming kernel (f16/bf16, M <= 128, bias none or per row).
#include "kernels.h"
#include "selector.h"
#include "stream_kernel.h"

namespace cmpext3 {

template <typename T, int MT>
static void launch_stream_t(const GemmParams& p, int total, unsigned wgs, hipStream_t s) {
  if (p.bias != nullptr)
    hipLaunchKernelGGL((gemm_stream_kernel<T, 2, MT>), dim3(wgs), dim3(256), 0, s, p, total);
  else
    hipLaunchKernelGGL((gemm_stream_kernel<T, 0, MT>), dim3(wgs), dim3(256), 0, s, p, total);
}

hipError_t launch_stream(DType dt, const GemmParams& p, dim3 grid, hipStream_t s) {
  // grid.x = 128-column tiles of one product, grid.z = batch entries: one persistent
  // workgroup per CU walks all of them
  const int64_t total = (int64_t)grid.x * grid.z;
  if (total <= 0) return hipSuccess;
  if (total > 0x7FFFFFFF || (p.bias != nullptr && !p.bias_row) || p.M > 128) return hipErrorInvalidValue;
  const unsigned wgs = (unsigned)std::min<int64_t>(total, kNumCUs);
  if (dt == kF16)
    p.M <= 64 ? launch_stream_t<_Float16, 64>(p, (int)total, wgs, s) : launch_stream_t<_Float16, 128>(p, (int)total, wgs, s);
  else
    p.M <= 64 ? launch_stream_t<__bf16, 64>(p, (int)total, wgs, s) : launch_stream_t<__bf16, 128>(p, (int)total, wgs, s);
  return hipGetLastError();
}

}  // namespace cmpext3
