// Kernel argument block and kernel ids shared by the host selector, the
// launchers and the device code.  Plain C++ (no HIP types) so the selector can
// be compiled and tested on a machine without a GPU.
#pragma once

#include <stdint.h>

namespace cmpext3 {

enum DType : int { kF16 = 0, kBF16 = 1, kF32 = 2 };
enum BLayout : int { kKN = 0, kNK = 1 };

// Passed by value to every GEMM kernel.  Strides are in elements.
struct GemmParams {
  const void* A;
  const void* B;
  void* C;
  const void* bias;  // nullptr, or a vector of the input dtype added before rounding:
  int bias_row;      //   0: N elements, one per column of C (Linear); 1: M elements, one per row (conv 1x1)
  int bias_vec;      // the bias address is 8-byte aligned (per-column bias read four elements at a time)
  int64_t lda, ldb, ldc;
  int64_t stride_a, stride_b, stride_c;  // batch strides (grid.z)
  int M, N, K;
  int tiles_m, tiles_n;  // grid of output tiles (tiled kernels)
  int group_m;           // rows of tiles per ordering group
  // split-K tiled products: grid.z = batch * splits, split s sums k in [s*ksplit, (s+1)*ksplit)
  // and writes fp32 partials[s][batch][M][N] (summed, biased and rounded by a second launch)
  int splits, ksplit;
  float* partials;
};

// Every kernel the library can launch.  The selector returns one of these.
enum KernelId : int {
  kTile256x256 = 0,   // f16/bf16 MFMA 16x16x32, 8 waves of 64x128, LDS-DMA ring
  kTile256x224 = 1,   // same, 8 waves of 64x112 (N tiles of 224)
  kTile128x128 = 2,   // same, 4 waves of 64x64, two workgroups per CU
  kSkinny = 3,        // f16/bf16, M <= 64: 32-column strips through an LDS-DMA ring
  kF32Tile128 = 4,    // fp32 MFMA 16x16x4, 128x128 tile, 4- or 16-byte LDS-DMA ring
  kF32Tile64 = 5,     // same, 64x64 tile
  kGeneric16 = 6,     // f16/bf16 any shape and alignment (element loads)
  kSkinnyWide = 7,    // f16/bf16, M <= 64: 128-column strips, K split over workgroups
  kF32Tile96x64 = 8,  // fp32, 96x64 tile
  kTile64x256 = 9,    // f16/bf16 MFMA 16x16x32, 4 waves of 64x64, two workgroups per CU (M <= 64, short K)
  kSkinnyNK = 10,     // f16/bf16, M <= 64, B is [N,K]: 16- or 32-row strips of W, all of K per workgroup
  kF32Tile64K4 = 11,  // fp32, 64x64 tile, K split over the workgroup's four waves (few tiles per CU)
  kF32Tile16K4 = 12,  // same with 16x64 tiles (M <= 16)
  kStream64x128 = 13, // f16/bf16, M <= 64, K <= 256, B is [K,N]: persistent workgroups stream 128-column tiles
  kStream128x128 = 14,  // same with 128-row tiles (64 < M <= 128)
  kTall = 15,         // f16/bf16, N <= 128: strips of A's rows over all of K, B small ([N,K] or [K,N])
  kNumKernels = 16
};

}  // namespace cmpext3
