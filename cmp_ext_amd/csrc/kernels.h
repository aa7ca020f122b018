// Launchers of the gfx950 GEMM kernels (one translation unit per family so
// they build in parallel).  Each returns the hipError_t of its launch.
#pragma once

#include <hip/hip_runtime_api.h>

#include "gemm_params.h"

namespace cmpext3 {

// f16/bf16 tile kernels, one entry per (type, B layout, K check): "whole" when K
// (every split's range) is a multiple of 64, "ragged" otherwise.
hipError_t launch_tile_f16_kn_whole(KernelId id, const GemmParams& p, dim3 grid, hipStream_t s);
hipError_t launch_tile_f16_kn_ragged(KernelId id, const GemmParams& p, dim3 grid, hipStream_t s);
hipError_t launch_tile_f16_nk_whole(KernelId id, const GemmParams& p, dim3 grid, hipStream_t s);
hipError_t launch_tile_f16_nk_ragged(KernelId id, const GemmParams& p, dim3 grid, hipStream_t s);
hipError_t launch_tile_bf16_kn_whole(KernelId id, const GemmParams& p, dim3 grid, hipStream_t s);
hipError_t launch_tile_bf16_kn_ragged(KernelId id, const GemmParams& p, dim3 grid, hipStream_t s);
hipError_t launch_tile_bf16_nk_whole(KernelId id, const GemmParams& p, dim3 grid, hipStream_t s);
hipError_t launch_tile_bf16_nk_ragged(KernelId id, const GemmParams& p, dim3 grid, hipStream_t s);
hipError_t launch_skinny(DType dt, int mb, const GemmParams& p, dim3 grid, hipStream_t s);
hipError_t launch_skinny_nk(DType dt, int mb, int strip, const GemmParams& p, dim3 grid, hipStream_t s);
// N <= 16 * mb: strips of `strip` rows of A over all of K, B as [N, K] or [K, N] (layout)
hipError_t launch_tall(DType dt, BLayout lay, int mb, int strip, const GemmParams& p, dim3 grid, hipStream_t s);
// sem: counters of the in-kernel split reduction (split_counters), or nullptr when the
// partials are left for launch_skinny_reduce.
hipError_t launch_skinny_wide(DType dt, int mb, const GemmParams& p, float* ws, int splits, int ksplit, dim3 grid,
                              hipStream_t s, unsigned int* sem);
// Counters for the split-K reductions done inside the splitting kernel (sem.hip): slots of
// kSemCounters per stream of a GPU, zero between kernels.  Returns the slot of stream s
// when `count` counters fit and s is neither capturing a graph nor beyond the first
// kSemSlots streams of its GPU, else nullptr (the caller then reduces in a second launch).
constexpr int kSemSlots = 64;
constexpr int kSemCounters = 4096;
unsigned int* split_counters(hipStream_t s, int64_t count);
hipError_t launch_skinny_reduce(DType dt, const GemmParams& p, const float* ws, int splits, int batch,
                                hipStream_t s);
// grid.x = 128-column tiles, grid.z = batch entries (one A shared by all, M <= 128); bias none or per row.
hipError_t launch_stream(DType dt, BLayout lay, const GemmParams& p, dim3 grid, hipStream_t s);
hipError_t launch_f32(KernelId id, BLayout lay, bool dma16, const GemmParams& p, dim3 grid, hipStream_t s);
hipError_t launch_generic(DType dt, BLayout lay, const GemmParams& p, dim3 grid, hipStream_t s);
// dst[b][r][c] = src[b][r][c] (elements of esz = 2 or 4 bytes) for r < rows, c < cols,
// zero elsewhere in dst_rows x dst_cols; dst_ld == dst_cols, rows of a multiple of 16
// bytes, dst 16-byte aligned.
hipError_t launch_pad_copy(const void* src, int64_t src_ld, int64_t src_stride, int rows, int cols, void* dst,
                           int64_t dst_ld, int64_t dst_stride, int dst_rows, int dst_cols, int64_t batch, int esz,
                           hipStream_t s);

}  // namespace cmpext3
