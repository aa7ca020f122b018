// Zero-padded copies of operands whose rows are not 16-byte aligned (odd K,
// odd N, offset views), so that the 16-byte LDS-DMA kernels can run on them:
// dst[b][r][c] = src[b][r][c] for r < rows, c < cols, and 0 elsewhere in the
// dst_rows x dst_cols block.  Elements of 2 bytes (f16/bf16) or 4 (fp32).  dst
// is dense (dst_ld == dst_cols, a multiple of 16 bytes) and 16-byte aligned;
// src may have any pitch and offset.  No counterpart in the reference, whose kernels read
// misaligned rows element by element (bf16_matmul.cu:31-38).
#include "device_common.h"
#include "kernels.h"

namespace cmpext3 {
namespace {
// 256 threads copy kChunk consecutive elements of the (dense) dst block: element
// loads with consecutive lanes on consecutive elements (32 per thread in flight),
// regrouped through LDS so that each thread then writes 16 bytes of them per store.
constexpr int kPer = 32, kChunk = 256 * kPer;
template <typename E>
__global__ void __launch_bounds__(256) pad_copy_kernel(const E* __restrict__ src, int64_t src_ld,
                                                       int64_t src_stride, int rows, int cols,
                                                       E* __restrict__ dst, int64_t dst_stride,
                                                       int dst_rows, int dst_cols) {
  constexpr int V = 16 / sizeof(E);  // elements per 16-byte store
  __shared__ __attribute__((aligned(16))) E buf[kChunk];
  const int64_t total = (int64_t)dst_rows * dst_cols;
  const int64_t e0 = (int64_t)blockIdx.x * kChunk;
  const int64_t b = blockIdx.z;
  const E* s = src + b * src_stride;
  const int tid = threadIdx.x;
  int r = (int)((e0 + tid) / dst_cols);
  int c = (int)((e0 + tid) - (int64_t)r * dst_cols);
  E v[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) {  // element e0 + tid + 256 i: advance (r, c) by 256
    const bool in = e0 + tid + 256 * i < total && r < rows && c < cols;
    v[i] = in ? s[(int64_t)r * src_ld + c] : (E)0;
    c += 256;
    while (c >= dst_cols) {
      c -= dst_cols;
      ++r;
    }
  }
#pragma unroll
  for (int i = 0; i < kPer; ++i) buf[tid + 256 * i] = v[i];
  __syncthreads();
#pragma unroll
  for (int j = 0; j < kPer / V; ++j) {
    const int q = tid + 256 * j;  // V-element piece of the chunk
    const int64_t e = e0 + V * q;
    if (e < total) *(u32x4*)(dst + b * dst_stride + e) = *(const u32x4*)(buf + V * q);
  }
}
}  // namespace

hipError_t launch_pad_copy(const void* src, int64_t src_ld, int64_t src_stride, int rows, int cols, void* dst,
                           int64_t dst_ld, int64_t dst_stride, int dst_rows, int dst_cols, int64_t batch,
                           int esz, hipStream_t s) {
  if (esz != 2 && esz != 4) return hipErrorInvalidValue;
  if (dst_ld != dst_cols || dst_cols % (16 / esz) != 0) return hipErrorInvalidValue;  // dst is a dense block
  constexpr int64_t kMaxZ = 65535;
  const dim3 block(256);
  const int64_t total = (int64_t)dst_rows * dst_cols;
  for (int64_t b0 = 0; b0 < batch; b0 += kMaxZ) {
    const int64_t nb = batch - b0 < kMaxZ ? batch - b0 : kMaxZ;
    const dim3 grid((unsigned)((total + kChunk - 1) / kChunk), 1, (unsigned)nb);
    hipError_t e;
    if (esz == 2)
      e = launch_kernel(pad_copy_kernel<uint16_t>, grid, block, 0, s, (const uint16_t*)src + b0 * src_stride,
                         src_ld, src_stride, rows, cols, (uint16_t*)dst + b0 * dst_stride, dst_stride, dst_rows,
                         dst_cols);
    else
      e = launch_kernel(pad_copy_kernel<uint32_t>, grid, block, 0, s, (const uint32_t*)src + b0 * src_stride,
                         src_ld, src_stride, rows, cols, (uint32_t*)dst + b0 * dst_stride, dst_stride, dst_rows,
                         dst_cols);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace cmpext3
