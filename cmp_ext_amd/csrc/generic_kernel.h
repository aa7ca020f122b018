// f16/bf16 GEMM for any shape, stride and alignment: C = A * op(B) (+ bias).
//
// The fast kernels need 16-byte aligned rows (K and N multiples of 8).  The
// reference's kernels silently read past row ends when that does not hold
// (src/cuda/fp16_matmul.cu:133-140, src/cuda/bf16_matmul.cu:106-119) and its
// Linear refuses odd N for fp16 (src/main.cpp:196-200).  This kernel has no
// such restriction: it loads one 16-bit element per buffer load (out-of-range
// elements read as zero), packs eight of them into a K-contiguous 16-byte LDS
// row, and runs the same v_mfma_f32_16x16x32 products as the tiled kernel on
// a 64x64 tile (2 x 2 waves of 32x32, BK = 32, single LDS stage).
#pragma once

#include "device_common.h"

namespace cmpext3 {

constexpr int kGenBM = 64, kGenBN = 64, kGenBK = 32, kGenLDR = 40;  // LDR in 16-bit elements

template <typename T, bool KN>
__global__ void __launch_bounds__(256) gemm_generic_kernel(const GemmParams p) {
  __shared__ __attribute__((aligned(16))) uint16_t sA[kGenBM * kGenLDR];
  __shared__ __attribute__((aligned(16))) uint16_t sB[kGenBN * kGenLDR];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  int tm, tn;
  int bzi;
  tile_coords(blockIdx.x, blockIdx.z, gridDim.z, p.tiles_m, p.tiles_n, p.group_m, tm, tn, bzi);
  const int m0 = tm * kGenBM, n0 = tn * kGenBN;
  const int M = p.M, N = p.N, K = p.K;
  const int64_t lda = p.lda, ldb = p.ldb;
  const int64_t bz = bzi;
  const T* Abase = (const T*)p.A + bz * p.stride_a + (int64_t)m0 * lda;
  const T* Bbase = KN ? (const T*)p.B + bz * p.stride_b + n0
                      : (const T*)p.B + bz * p.stride_b + (int64_t)n0 * ldb;

  // A (and NK-layout B): thread -> row tid/4, k run 8*(tid%4) .. +7.
  const int ar = tid >> 2, ak = 8 * (tid & 3);
  // KN-layout B: thread -> column tid%64, k run 8*(tid/64) .. +7.
  const int bn = KN ? (tid & 63) : ar;
  const int bk = KN ? 8 * (tid >> 6) : ak;

  const int r16 = lane & 15, g = lane >> 4;
  f32x4 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int k0 = 0; k0 < K; k0 += kGenBK) {
    const __amdgpu_buffer_rsrc_t a_rsrc = make_rsrc(Abase + k0);
    const __amdgpu_buffer_rsrc_t b_rsrc = make_rsrc(KN ? Bbase + (int64_t)k0 * ldb : Bbase + k0);
    uint16_t av[8], bv[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const bool aok = (m0 + ar < M) && (k0 + ak + e < K);
      av[e] = buf_load2(a_rsrc, aok ? (uint32_t)(ar * lda + ak + e) * 2u : kBufOOB);
      const bool bok = (n0 + bn < N) && (k0 + bk + e < K);
      const uint32_t boff = KN ? (uint32_t)((bk + e) * ldb + bn) * 2u : (uint32_t)(bn * ldb + bk + e) * 2u;
      bv[e] = buf_load2(b_rsrc, bok ? boff : kBufOOB);
    }
    u32x4 pa, pb;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      pa[d] = (uint32_t)av[2 * d] | ((uint32_t)av[2 * d + 1] << 16);
      pb[d] = (uint32_t)bv[2 * d] | ((uint32_t)bv[2 * d + 1] << 16);
    }
    __syncthreads();  // previous step's fragment reads are done
    *(u32x4*)(sA + ar * kGenLDR + ak) = pa;
    *(u32x4*)(sB + bn * kGenLDR + bk) = pb;
    __syncthreads();
    u32x4 af[2], bf[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) af[i] = *(const u32x4*)(sA + (wm * 32 + i * 16 + r16) * kGenLDR + 8 * g);
#pragma unroll
    for (int j = 0; j < 2; ++j) bf[j] = *(const u32x4*)(sB + (wn * 32 + j * 16 + r16) * kGenLDR + 8 * g);
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[i][j] = Mfma<T>::mma(bf[j], af[i], acc[i][j]);
  }

  T* Cb = (T*)p.C + bz * p.stride_c;
  const uint16_t* bias = (const uint16_t*)p.bias;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int m = m0 + wm * 32 + i * 16 + r16;
    if (m >= M) continue;
    uint16_t* crow = (uint16_t*)(Cb + (int64_t)m * p.ldc);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int n = n0 + wn * 32 + j * 16 + 4 * g;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (n + e < N) {
          float x = acc[i][j][e];
          if (bias) x += from_bits<T>(bias[p.bias_row ? m : n + e]);
          crow[n + e] = to_bits<T>(x);
        }
      }
    }
  }
}

}  // namespace cmpext3
