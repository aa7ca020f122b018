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
  const void* bias;  // nullptr or N elements of the input dtype
  int64_t lda, ldb, ldc;
  int64_t stride_a, stride_b, stride_c;  // batch strides (grid.z)
  int M, N, K;
  int tiles_m, tiles_n;  // grid of output tiles (tiled kernels)
  int group_m;           // rows of tiles per ordering group
  int k_per_wave;        // skinny kernel: K range of one wave (multiple of 32)
};

// Every kernel the library can launch.  The selector returns one of these.
enum KernelId : int {
  kTile256x256 = 0,   // f16/bf16 MFMA 16x16x32, 4 waves, 128x128 per wave
  kTile256x224 = 1,   // same, 128x112 per wave (N tiles of 224)
  kTile128x128 = 2,   // same, 64x64 per wave
  kSkinny = 3,        // f16/bf16, M <= 64, B streamed once, K split over waves
  kF32Tile128 = 4,    // fp32 MFMA 16x16x4, 128x128 tile
  kF32Tile64 = 5,     // fp32 MFMA 16x16x4, 64x64 tile
  kGeneric16 = 6,     // f16/bf16 any shape and alignment (element loads)
  kNumKernels = 7
};

}  // namespace cmpext3
