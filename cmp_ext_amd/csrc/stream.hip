// Launcher of the short-K streaming kernel (f16/bf16; M <= 128 with K <= 128, or M <= 64
// with K <= 256; bias none or per row).
#include "kernels.h"
#include "selector.h"
#include "stream_kernel.h"

namespace cmpext3 {

// B read non-temporally for K >= 160 (two chunks per tile, the second at least a quarter
// full).  MI355X, 64 images of 128 x 128 pixels, us per call without / with: 64 <- 256
// channels 134.5 / 129.4, 64 <- 160 91.6 / 86.8, 48 <- 200 102.0 / 98.2; but 64 <- 136
// 71.3 / 76.2, and with one chunk (K <= 128) it is always slower: 64 <- 128 62.7 / 75.4,
// 16 <- 128 51.7 / 57.8, 32 <- 64 37.5 / 38.0.
static bool stream_nt(const GemmParams& p) { return p.K >= 160; }

template <typename T, int MT, int KC, bool NT>
static void launch_stream_t(const GemmParams& p, int total, unsigned wgs, hipStream_t s) {
  if (p.bias != nullptr)
    hipLaunchKernelGGL((gemm_stream_kernel<T, 2, MT, KC, NT>), dim3(wgs), dim3(256), 0, s, p, total);
  else
    hipLaunchKernelGGL((gemm_stream_kernel<T, 0, MT, KC, NT>), dim3(wgs), dim3(256), 0, s, p, total);
}

template <typename T>
static void launch_stream_shape(const GemmParams& p, int total, unsigned wgs, hipStream_t s) {
  if (p.M > 64)
    launch_stream_t<T, 128, 1, false>(p, total, wgs, s);
  else if (p.K > kStreamKC)
    stream_nt(p) ? launch_stream_t<T, 64, 2, true>(p, total, wgs, s) : launch_stream_t<T, 64, 2, false>(p, total, wgs, s);
  else
    launch_stream_t<T, 64, 1, false>(p, total, wgs, s);
}

hipError_t launch_stream(DType dt, const GemmParams& p, dim3 grid, hipStream_t s) {
  // grid.x = 128-column tiles of one product, grid.z = batch entries: one persistent
  // workgroup per CU walks all of them
  const int64_t total = (int64_t)grid.x * grid.z;
  if (total <= 0) return hipSuccess;
  if (total > 0x7FFFFFFF || (p.bias != nullptr && !p.bias_row) || p.M > 128 ||
      p.K > (p.M > 64 ? 1 : 2) * kStreamKC)
    return hipErrorInvalidValue;
  const unsigned wgs = (unsigned)std::min<int64_t>(total, kNumCUs);
  if (dt == kF16)
    launch_stream_shape<_Float16>(p, (int)total, wgs, s);
  else
    launch_stream_shape<__bf16>(p, (int)total, wgs, s);
  return hipGetLastError();
}

}  // namespace cmpext3
