// Skinny-M f16/bf16 GEMM (M <= 64, B is [K,N]): C = A * B (+ bias).
//
// Decode-like shapes (e.g. 16 x 8192 x 8192) read B once and do ~16 flops per
// B byte, so they are bound by HBM bandwidth, not by the matrix cores.  The
// reference has no special path for them: its 128x128 tile kernel runs with
// 112 of 128 rows zero-filled and only ceil(N/128) workgroups
// (src/cuda/fp16_matmul.cu:318-321).  This kernel instead:
//   * gives each workgroup a 32-column strip of B and all of K, so the number
//     of workgroups is N/32 (256 for N = 8192: one per CU) and B is read
//     exactly once, in full 64-byte row segments; strips are ordered so that
//     neighbouring strips run on the same XCD;
//   * splits K over the 8 waves of the workgroup and keeps PF steps of loads in
//     flight per wave (each step: 32 k x 32 columns of B, 2 KB per wave);
//   * feeds v_mfma_f32_16x16x32 directly from registers: lane (c, g) loads the
//     32-bit pair B[k0+8g+i][2c..2c+1] for i = 0..7 and repacks it (v_perm)
//     into the K-contiguous operands for columns 2c and 2c+1;
//   * reduces the 8 per-wave partial sums in LDS and writes C once.
#pragma once

#include "device_common.h"

namespace cmpext3 {

constexpr int kSkinnyWaves = 8;
constexpr int kSkinnyStrip = 32;

__device__ __forceinline__ int strip_order(int wg, int total) {
  const int xcd = wg & 7, local = wg >> 3;
  const int base = total >> 3, rem = total & 7;
  return xcd * base + (xcd < rem ? xcd : rem) + local;
}

template <typename T, int MB, int PF>
__global__ void __launch_bounds__(kSkinnyWaves * 64) gemm_skinny_kernel(const GemmParams p) {
  __shared__ float red[kSkinnyWaves][MB * 16][kSkinnyStrip + 1];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int c = lane & 15, g = lane >> 4;
  const int strip = strip_order(blockIdx.x, gridDim.x);
  const int n0 = strip * kSkinnyStrip;
  const int M = p.M, N = p.N, K = p.K;
  const int64_t bz = blockIdx.z;
  const int64_t ldb = p.ldb;

  const T* Ab = (const T*)p.A + bz * p.stride_a;
  const T* Bb = (const T*)p.B + bz * p.stride_b + n0;
  const __amdgpu_buffer_rsrc_t a_rsrc = make_rsrc(Ab);

  const int kbeg = wave * p.k_per_wave;
  const int kend = min(K, kbeg + p.k_per_wave);
  const bool col_ok = n0 + 2 * c < N;  // N is even: the pair is in or out as a whole
  const uint32_t ldb_bytes = (uint32_t)(ldb * (int64_t)sizeof(T));
  const uint32_t b_lane = (uint32_t)(8 * g * ldb + 2 * c) * (uint32_t)sizeof(T);
  uint32_t a_lane[MB];
  bool a_row_ok[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int row = mb * 16 + c;
    a_row_ok[mb] = row < M;
    a_lane[mb] = (uint32_t)(row * p.lda + 8 * g) * (uint32_t)sizeof(T);
  }

  uint32_t bq[PF][8];
  u32x4 aq[PF][MB];

  auto load_step = [&](int s, int k) {
    const __amdgpu_buffer_rsrc_t b_rsrc = make_rsrc(Bb + (int64_t)k * ldb);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const bool ok = col_ok && (k + 8 * g + i < kend);
      bq[s][i] = buf_load4(b_rsrc, ok ? b_lane + i * ldb_bytes : kBufOOB);
    }
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const bool ok = a_row_ok[mb] && (k + 8 * g < kend);
      aq[s][mb] = buf_load16(a_rsrc, ok ? a_lane[mb] + (uint32_t)k * (uint32_t)sizeof(T) : kBufOOB);
    }
  };

  f32x4 acc[MB][2];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    acc[mb][0] = f32x4{0.f, 0.f, 0.f, 0.f};
    acc[mb][1] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  auto compute_step = [&](int s) {
    u32x4 b0, b1;  // K-contiguous operands of columns 2c and 2c+1
    b0.x = pack_lo16(bq[s][0], bq[s][1]);
    b0.y = pack_lo16(bq[s][2], bq[s][3]);
    b0.z = pack_lo16(bq[s][4], bq[s][5]);
    b0.w = pack_lo16(bq[s][6], bq[s][7]);
    b1.x = pack_hi16(bq[s][0], bq[s][1]);
    b1.y = pack_hi16(bq[s][2], bq[s][3]);
    b1.z = pack_hi16(bq[s][4], bq[s][5]);
    b1.w = pack_hi16(bq[s][6], bq[s][7]);
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      acc[mb][0] = Mfma<T>::mma(b0, aq[s][mb], acc[mb][0]);
      acc[mb][1] = Mfma<T>::mma(b1, aq[s][mb], acc[mb][1]);
    }
  };

  if (kbeg < kend) {
#pragma unroll
    for (int s = 0; s < PF; ++s) load_step(s, kbeg + 32 * s);
    for (int k = kbeg; k < kend; k += 32 * PF) {
#pragma unroll
      for (int s = 0; s < PF; ++s) {
        compute_step(s);
        load_step(s, k + 32 * (s + PF));
      }
    }
  }

  // acc[mb][jj][r] = C[mb*16 + c][n0 + 2*(4g + r) + jj]
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      red[wave][mb * 16 + c][2 * (4 * g + r)] = acc[mb][0][r];
      red[wave][mb * 16 + c][2 * (4 * g + r) + 1] = acc[mb][1][r];
    }
  __syncthreads();

  T* Cb = (T*)p.C + bz * p.stride_c;
  const uint16_t* bias = (const uint16_t*)p.bias;
  for (int o = tid; o < MB * 16 * kSkinnyStrip; o += kSkinnyWaves * 64) {
    const int row = o / kSkinnyStrip, col = o % kSkinnyStrip;
    const int n = n0 + col;
    if (row >= M || n >= N) continue;
    float s = 0.f;
#pragma unroll
    for (int w = 0; w < kSkinnyWaves; ++w) s += red[w][row][col];
    if (bias) s += from_bits<T>(bias[n]);
    ((uint16_t*)(Cb + (int64_t)row * p.ldc))[n] = to_bits<T>(s);
  }
}

}  // namespace cmpext3
