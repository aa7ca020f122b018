// Launcher of the short-K streaming kernel (f16/bf16, M <= 2048 in row blocks of 64 or 128,
// K <= 256, bias none or per row).
#include "kernels.h"
#include "selector.h"
#include "stream_kernel.h"

namespace cmpext3 {

// B read non-temporally for K >= 160 (two chunks per tile, the second at least a quarter
// full).  MI355X, 64 images of 128 x 128 pixels, us per call without / with: 64 <- 256
// channels 134.5 / 129.4, 64 <- 160 91.6 / 86.8, 48 <- 200 102.0 / 98.2; but 64 <- 136
// 71.3 / 76.2, and with one chunk (K <= 128) it is always slower: 64 <- 128 62.7 / 75.4,
// 16 <- 128 51.7 / 57.8, 32 <- 64 37.5 / 38.0.
// With several row blocks the later blocks read each B chunk from L2, which the
// non-temporal policy would give up: only for M <= 128.
static bool stream_nt(const GemmParams& p) { return p.K >= 160 && p.M <= 128; }

template <typename T, int WG, int KC, bool NT>
static void launch_stream_t(const GemmParams& p, int total, unsigned wgs, hipStream_t s) {
  if (p.bias != nullptr)
    hipLaunchKernelGGL((gemm_stream_kernel<T, 2, WG, KC, NT>), dim3(wgs), dim3(256 * WG), 0, s, p, total);
  else
    hipLaunchKernelGGL((gemm_stream_kernel<T, 0, WG, KC, NT>), dim3(wgs), dim3(256 * WG), 0, s, p, total);
}

template <typename T, int WG>
static void launch_stream_rows(const GemmParams& p, int total, unsigned wgs, hipStream_t s) {
  if (p.K <= kStreamKC)
    launch_stream_t<T, WG, 1, false>(p, total, wgs, s);
  else if (stream_nt(p))
    launch_stream_t<T, WG, 2, true>(p, total, wgs, s);
  else
    launch_stream_t<T, WG, 2, false>(p, total, wgs, s);
}

// 65..128 rows: two groups of 4 waves, 64 rows each (MI355X, 64 images of 128 x 128
// pixels, against one group of 4 waves of 128 rows each: 128 <- 128 channels 85.3 ->
// 83.6 us, 128 <- 64 63.7 -> 61.1 us, 72 <- 32 59.7 -> 51.5 us; and K up to 256 fits).
template <typename T>
static void launch_stream_shape(const GemmParams& p, int total, unsigned wgs, hipStream_t s) {
  if (p.M > 64)
    launch_stream_rows<T, 2>(p, total, wgs, s);
  else
    launch_stream_rows<T, 1>(p, total, wgs, s);
}

hipError_t launch_stream(DType dt, const GemmParams& p, dim3 grid, hipStream_t s) {
  // grid.x = 128-column tiles of one product (all of M: the kernel covers the rows itself),
  // grid.z = batch entries: persistent workgroups, a set per row block of 64 (M <= 64) or 128
  // rows, walk all of them.  A grid that does not match N would send the walk past the
  // operands, so it is an error.
  if (grid.y != 1 || (int64_t)grid.x != ((int64_t)p.N + kStreamN - 1) / kStreamN || (int)grid.x != p.tiles_n)
    return hipErrorInvalidValue;
  const int64_t total = (int64_t)grid.x * grid.z;
  if (total <= 0) return hipSuccess;
  if (total > 0x7FFFFFFF || (p.bias != nullptr && !p.bias_row) || p.M > kStreamMaxRows || p.K > 2 * kStreamKC)
    return hipErrorInvalidValue;
  const int mt = p.M > 64 ? 128 : 64;
  const int row_blocks = (p.M + mt - 1) / mt;
  // workgroups per row block: a multiple of 8 (one per XCD and round) when there are 8 or more
  int64_t per_block = std::min<int64_t>(total, kNumCUs / row_blocks);
  if (per_block >= 8) per_block -= per_block % 8;
  const unsigned wgs = (unsigned)(per_block * row_blocks);
  if (dt == kF16)
    launch_stream_shape<_Float16>(p, (int)total, wgs, s);
  else
    launch_stream_shape<__bf16>(p, (int)total, wgs, s);
  return hipGetLastError();
}

}  // namespace cmpext3
