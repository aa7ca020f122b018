// Launcher of the short-K streaming kernel (f16/bf16, M <= 2048 in row blocks of 64 or 128,
// K <= 256, B as [K, N] or [N, K], bias none or per row); the [K, N] instantiations.
#include "stream_launch.h"

namespace cmpext3 {

hipError_t launch_stream(DType dt, BLayout lay, const GemmParams& p, dim3 grid, hipStream_t s) {
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
  if (lay == kNK) return launch_stream_nk(dt, p, (int)total, wgs, s);
  return launch_stream_layout<false>(dt, p, (int)total, wgs, s);
}

}  // namespace cmpext3
