// Launch helpers of the short-K streaming kernel, shared by the translation unit of B as
// [K, N] (stream.hip) and that of B as [N, K] (stream_nk.hip).
#pragma once

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
inline bool stream_nt(const GemmParams& p) { return p.K >= 160 && p.M <= 128; }

template <typename T, int WG, int KC, bool NT, bool BNK>
hipError_t launch_stream_t(const GemmParams& p, int total, unsigned wgs, hipStream_t s) {
  if (p.bias != nullptr)
    return launch_kernel((gemm_stream_kernel<T, 2, WG, KC, NT, BNK>), dim3(wgs), dim3(256 * WG), 0, s, p, total);
  return launch_kernel((gemm_stream_kernel<T, 0, WG, KC, NT, BNK>), dim3(wgs), dim3(256 * WG), 0, s, p, total);
}

template <typename T, int WG, bool BNK>
hipError_t launch_stream_rows(const GemmParams& p, int total, unsigned wgs, hipStream_t s) {
  if (p.K <= kStreamKC) return launch_stream_t<T, WG, 1, false, BNK>(p, total, wgs, s);
  if (stream_nt(p)) return launch_stream_t<T, WG, 2, true, BNK>(p, total, wgs, s);
  return launch_stream_t<T, WG, 2, false, BNK>(p, total, wgs, s);
}

// 65..128 rows: two groups of 4 waves, 64 rows each (MI355X, 64 images of 128 x 128
// pixels, against one group of 4 waves of 128 rows each: 128 <- 128 channels 85.3 ->
// 83.6 us, 128 <- 64 63.7 -> 61.1 us, 72 <- 32 59.7 -> 51.5 us; and K up to 256 fits).
template <typename T, bool BNK>
hipError_t launch_stream_shape(const GemmParams& p, int total, unsigned wgs, hipStream_t s) {
  if (p.M > 64) return launch_stream_rows<T, 2, BNK>(p, total, wgs, s);
  return launch_stream_rows<T, 1, BNK>(p, total, wgs, s);
}

// All instantiations for one B layout (one translation unit each, built in parallel).
template <bool BNK>
hipError_t launch_stream_layout(DType dt, const GemmParams& p, int total, unsigned wgs, hipStream_t s) {
  if (dt == kF16) return launch_stream_shape<_Float16, BNK>(p, total, wgs, s);
  return launch_stream_shape<__bf16, BNK>(p, total, wgs, s);
}

hipError_t launch_stream_nk(DType dt, const GemmParams& p, int total, unsigned wgs, hipStream_t s);

}  // namespace cmpext3
