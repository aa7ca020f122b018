// Instantiations of the skinny-M GEMM (M <= 64; B is [K, N], or [N, K] for the
// strips-of-W kernel).
#include <stdint.h>

#include <algorithm>

#include "kernels.h"
#include "skinny_kernel.h"
#include "skinny_wide_kernel.h"

namespace cmpext3 {
namespace {
template <typename T>
hipError_t launch(int mb, const GemmParams& p, dim3 grid, hipStream_t s) {
  const dim3 block(256);
  switch (mb) {
    case 1: return launch_kernel((gemm_skinny_narrow_kernel<T, 1>), grid, block, 0, s, p);
    case 2: return launch_kernel((gemm_skinny_narrow_kernel<T, 2>), grid, block, 0, s, p);
    case 3: return launch_kernel((gemm_skinny_narrow_kernel<T, 3>), grid, block, 0, s, p);
    case 4: return launch_kernel((gemm_skinny_narrow_kernel<T, 4>), grid, block, 0, s, p);
    default: return hipErrorInvalidValue;
  }
}
}  // namespace

namespace {
template <typename T, int SW, bool NT>
hipError_t launch_nk(int mb, const GemmParams& p, dim3 grid, hipStream_t s) {
  const dim3 block(256);
  // 1 KiB of each W row per stage for one 16-row block of A, 512 bytes otherwise; 64-row
  // strips: 512 bytes for one or two blocks, 256 for three or four (the ring keeps >= 3
  // stages).  32-row strips with one block (more than 256 of them): 512-byte stages in a
  // ring of 3 (72 KiB), so that two workgroups share a CU and all strips run at once
  // instead of in 1.75 rounds (MI355X, x[1, 4096] W[14336, 4096]^T 21.4 -> 19.7 us,
  // x[16, 4096] 23.3 -> 21.4 us, x[1, 8192] W[28672, 8192]^T 76.1 -> 73.3 us; with 16-row
  // strips, one per CU, the deep ring is faster: x[1, 14336] W[4096, 14336]^T 20.5 vs 26.0).
  switch (mb) {
    case 1:
      if constexpr (SW == 32)
        return launch_kernel((gemm_skinny_nk_kernel<T, 1, 32, 256, NT, 3>), grid, block, 0, s, p);
      else
        return launch_kernel((gemm_skinny_nk_kernel<T, 1, SW, SW == 64 ? 256 : 512, NT>), grid, block, 0, s, p);
    case 2: return launch_kernel((gemm_skinny_nk_kernel<T, 2, SW, 256, NT>), grid, block, 0, s, p);
    case 3: return launch_kernel((gemm_skinny_nk_kernel<T, 3, SW, SW == 64 ? 128 : 256, NT>), grid, block, 0, s, p);
    case 4: return launch_kernel((gemm_skinny_nk_kernel<T, 4, SW, SW == 64 ? 128 : 256, NT>), grid, block, 0, s, p);
    default: return hipErrorInvalidValue;
  }
}
template <typename T>
hipError_t launch_nk(int mb, int strip, const GemmParams& p, dim3 grid, hipStream_t s) {
  const bool nt = stream_once(p.N, p.K, p.stride_b, grid.z);
  if (strip == 16) return nt ? launch_nk<T, 16, true>(mb, p, grid, s) : launch_nk<T, 16, false>(mb, p, grid, s);
  if (strip == 64) return nt ? launch_nk<T, 64, true>(mb, p, grid, s) : launch_nk<T, 64, false>(mb, p, grid, s);
  return nt ? launch_nk<T, 32, true>(mb, p, grid, s) : launch_nk<T, 32, false>(mb, p, grid, s);
}
}  // namespace

hipError_t launch_skinny(DType dt, int mb, const GemmParams& p, dim3 grid, hipStream_t s) {
  if (dt == kF16) return launch<_Float16>(mb, p, grid, s);
  if (dt == kBF16) return launch<__bf16>(mb, p, grid, s);
  return hipErrorInvalidValue;
}

namespace {
template <typename T, bool NT>
hipError_t launch_wide(int mb, const GemmParams& p, float* ws, int splits, int ksplit, dim3 grid, hipStream_t s,
                       unsigned int* sem) {
  const dim3 block(256);
  switch (mb) {
    case 1: return launch_kernel((gemm_skinny_wide_kernel<T, 1, NT>), grid, block, 0, s, p, ws, splits, ksplit, sem);
    case 2: return launch_kernel((gemm_skinny_wide_kernel<T, 2, NT>), grid, block, 0, s, p, ws, splits, ksplit, sem);
    case 3: return launch_kernel((gemm_skinny_wide_kernel<T, 3, NT>), grid, block, 0, s, p, ws, splits, ksplit, sem);
    case 4: return launch_kernel((gemm_skinny_wide_kernel<T, 4, NT>), grid, block, 0, s, p, ws, splits, ksplit, sem);
    default: return hipErrorInvalidValue;
  }
}
template <typename T>
hipError_t launch_wide(int mb, const GemmParams& p, float* ws, int splits, int ksplit, dim3 grid, hipStream_t s,
                       unsigned int* sem) {
  return stream_once(p.K, p.N, p.stride_b, grid.z) ? launch_wide<T, true>(mb, p, ws, splits, ksplit, grid, s, sem)
                                                   : launch_wide<T, false>(mb, p, ws, splits, ksplit, grid, s, sem);
}
}  // namespace

hipError_t launch_skinny_wide(DType dt, int mb, const GemmParams& p, float* ws, int splits, int ksplit, dim3 grid,
                              hipStream_t s, unsigned int* sem) {
  if (splits <= 1) sem = nullptr;
  if (dt == kF16) return launch_wide<_Float16>(mb, p, ws, splits, ksplit, grid, s, sem);
  if (dt == kBF16) return launch_wide<__bf16>(mb, p, ws, splits, ksplit, grid, s, sem);
  return hipErrorInvalidValue;
}

namespace {
template <typename T, int V>
hipError_t launch_reduce(const GemmParams& p, const float* ws, int splits, int batch, int vec, dim3 grid,
                         hipStream_t s) {
  return launch_kernel((skinny_reduce_kernel<T, V>), grid, dim3(256), 0, s, p, ws, splits, batch, vec);
}
template <typename T>
hipError_t launch_reduce(int V, const GemmParams& p, const float* ws, int splits, int batch, int vec, dim3 grid,
                         hipStream_t s) {
  if (V == 8) return launch_reduce<T, 8>(p, ws, splits, batch, vec, grid, s);
  return launch_reduce<T, 4>(p, ws, splits, batch, vec, grid, s);
}
}  // namespace

hipError_t launch_skinny_reduce(DType dt, const GemmParams& p, const float* ws, int splits, int batch,
                                hipStream_t s) {
  // The split-K kernels write partial rows of N floats with 16-byte stores, so N % 4 == 0 here.
  if (p.N % 4 != 0 || splits < 1) return hipErrorInvalidValue;
  const int64_t rows = (int64_t)batch * p.M;
  if (rows <= 0 || p.N <= 0) return hipSuccess;
  // 8 columns per thread when that still gives >= 16 waves per CU, else 4 (twice the waves:
  // the sums are latency-bound when few)
  const int V = p.N % 8 == 0 && rows * (p.N / 8) >= 256ll * 16 * 64 ? 8 : 4;
  const int64_t esz = dt == kF32 ? 4 : 2;
  // C stores of V elements go out in pieces of at most 16 bytes; they need the
  // piece size as alignment of C, of its row pitch and of its batch stride.
  const int64_t align = std::min<int64_t>(16, V * esz);
  const int vec = (uintptr_t)p.C % align == 0 && (p.ldc * esz) % align == 0 &&
                  (batch == 1 || (p.stride_c * esz) % align == 0);
  // one V-column chunk per thread; past 65536 workgroups the threads loop (grid stride)
  const int64_t chunks = rows * (p.N / V);
  const dim3 grid((unsigned)std::min<int64_t>((chunks + 255) / 256, 65536));
  if (dt == kF16) return launch_reduce<_Float16>(V, p, ws, splits, batch, vec, grid, s);
  if (dt == kBF16) return launch_reduce<__bf16>(V, p, ws, splits, batch, vec, grid, s);
  return launch_reduce<float>(V, p, ws, splits, batch, vec, grid, s);
}
hipError_t launch_skinny_nk(DType dt, int mb, int strip, const GemmParams& p, dim3 grid, hipStream_t s) {
  if (dt == kF16) return launch_nk<_Float16>(mb, strip, p, grid, s);
  if (dt == kBF16) return launch_nk<__bf16>(mb, strip, p, grid, s);
  return hipErrorInvalidValue;
}
}  // namespace cmpext3
