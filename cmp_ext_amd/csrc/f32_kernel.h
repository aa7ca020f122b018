// fp32 GEMM on the CDNA4 fp32 matrix cores: C = A * op(B) (+ bias).
//
// Counterpart of gemm_fp32_ga100_kernel (src/cuda/fp32_matmul.cu:31-184):
// same contract (row-major, any M/N/K, fully bounds-checked loads and stores),
// but the products run on v_mfma_f32_16x16x4_f32 (fused multiply-add with fp32
// accumulation) instead of the reference's separate __fmul_rn/__fadd_rn SIMT
// loop, which exists only to dodge a GA100 FMA limit (fp32_matmul.cu:20-26).
//
// Any alignment is accepted: every global access is a 32-bit buffer load of
// one element, predicated by an out-of-range offset (hardware zero-fill), so
// ragged shapes such as 4097 x 3001 x 2049 need no special casing.  Per BK=16
// step a thread issues BM/16 + BN/16 such loads; the matrix-core time of the
// step (BM*BN*16*2 flop at 256 flop/clk/CU) is far longer than their issue
// time, so narrow loads cost nothing here.
//
// LDS holds A as [m][k] and B as [n][k] (transposed on store for the KN
// layout), rows of 16 floats padded to 20 (80 bytes: 16-byte aligned, and 16
// consecutive rows start in 16 distinct 16-byte bank groups).  MFMA k-step s
// of lane group g uses k = 4g + s, so one ds_read_b128 per fragment feeds four
// MFMAs.
#pragma once

#include "device_common.h"

namespace cmpext3 {

template <int BM, int BN>
struct F32Shape {
  static constexpr int BK = 16;
  static constexpr int LDR = 20;  // floats per LDS row
  static constexpr int NT = 256;  // 2 x 2 waves
  static constexpr int WTM = BM / 2, WTN = BN / 2;
  static constexpr int FM = WTM / 16, FN = WTN / 16;
  static constexpr int A_LD = BM * BK / NT;
  static constexpr int B_LD = BN * BK / NT;
  static constexpr int STAGE = (BM + BN) * LDR;  // floats
  static_assert(BM * BK % NT == 0 && BN * BK % NT == 0, "tile");
};

template <bool KN, int BM, int BN>
__global__ void __launch_bounds__(256) gemm_f32_kernel(const GemmParams p) {
  using S = F32Shape<BM, BN>;
  constexpr int FM = S::FM, FN = S::FN;
  __shared__ __attribute__((aligned(16))) float smem[2 * S::STAGE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  int tm, tn;
  tile_coords(blockIdx.x, p.tiles_m, p.tiles_n, p.group_m, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int M = p.M, N = p.N, K = p.K;
  const int64_t lda = p.lda, ldb = p.ldb;
  const int64_t bz = blockIdx.z;
  const float* Abase = (const float*)p.A + bz * p.stride_a + (int64_t)m0 * lda;
  const float* Bbase = KN ? (const float*)p.B + bz * p.stride_b + n0
                          : (const float*)p.B + bz * p.stride_b + (int64_t)n0 * ldb;

  // A element e = tid + i*256: row e/16, k e%16 (16 consecutive k per row).
  uint32_t a_goff[S::A_LD], a_soff[S::A_LD];
  int a_k[S::A_LD];
  bool a_ok[S::A_LD];
#pragma unroll
  for (int i = 0; i < S::A_LD; ++i) {
    const int e = tid + i * S::NT;
    const int row = e >> 4, kk = e & 15;
    a_ok[i] = m0 + row < M;
    a_goff[i] = (uint32_t)(row * lda + kk) * 4u;
    a_soff[i] = (uint32_t)(row * S::LDR + kk);
    a_k[i] = kk;
  }
  // B: KN element e: k e/BN, n e%BN (coalesced along n); NK like A.
  uint32_t b_goff[S::B_LD], b_soff[S::B_LD];
  int b_k[S::B_LD];
  bool b_ok[S::B_LD];
#pragma unroll
  for (int i = 0; i < S::B_LD; ++i) {
    const int e = tid + i * S::NT;
    int n, kk;
    if (KN) {
      kk = e / BN;
      n = e % BN;
      b_goff[i] = (uint32_t)(kk * ldb + n) * 4u;
    } else {
      n = e >> 4;
      kk = e & 15;
      b_goff[i] = (uint32_t)(n * ldb + kk) * 4u;
    }
    b_ok[i] = n0 + n < N;
    b_soff[i] = (uint32_t)(n * S::LDR + kk);
    b_k[i] = kk;
  }

  float ra[S::A_LD], rb[S::B_LD];
  auto load_tile = [&](int k0) {
    const __amdgpu_buffer_rsrc_t a_rsrc = make_rsrc(Abase + k0);
    const __amdgpu_buffer_rsrc_t b_rsrc = make_rsrc(KN ? Bbase + (int64_t)k0 * ldb : Bbase + k0);
#pragma unroll
    for (int i = 0; i < S::A_LD; ++i)
      ra[i] = __uint_as_float(buf_load4(a_rsrc, (a_ok[i] && k0 + a_k[i] < K) ? a_goff[i] : kBufOOB));
#pragma unroll
    for (int i = 0; i < S::B_LD; ++i)
      rb[i] = __uint_as_float(buf_load4(b_rsrc, (b_ok[i] && k0 + b_k[i] < K) ? b_goff[i] : kBufOOB));
  };
  auto store_tile = [&](int stage) {
    float* sA = smem + stage * S::STAGE;
    float* sB = sA + BM * S::LDR;
#pragma unroll
    for (int i = 0; i < S::A_LD; ++i) sA[a_soff[i]] = ra[i];
#pragma unroll
    for (int i = 0; i < S::B_LD; ++i) sB[b_soff[i]] = rb[i];
  };

  const int r16 = lane & 15, g = lane >> 4;
  const int fa = (wm * S::WTM + r16) * S::LDR + 4 * g;
  const int fb = (wn * S::WTN + r16) * S::LDR + 4 * g;

  f32x4 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](int stage) {
    const float* sA = smem + stage * S::STAGE;
    const float* sB = sA + BM * S::LDR;
    f32x4 af[FM], bf[FN];
#pragma unroll
    for (int i = 0; i < FM; ++i) af[i] = *(const f32x4*)(sA + fa + i * 16 * S::LDR);
#pragma unroll
    for (int j = 0; j < FN; ++j) bf[j] = *(const f32x4*)(sB + fb + j * 16 * S::LDR);
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = mma_f32(bf[j][s], af[i][s], acc[i][j]);
  };

  const int nk = (K + S::BK - 1) / S::BK;
  if (nk > 0) {
    load_tile(0);
    store_tile(0);
  }
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int stage = kt & 1;
    const bool more = kt + 1 < nk;
    if (more) load_tile((kt + 1) * S::BK);
    compute(stage);
    if (more) store_tile(stage ^ 1);
    __syncthreads();
  }

  float* Cb = (float*)p.C + bz * p.stride_c;
  const float* bias = (const float*)p.bias;
#pragma unroll
  for (int i = 0; i < FM; ++i) {
    const int m = m0 + wm * S::WTM + i * 16 + r16;
    if (m >= M) continue;
    float* crow = Cb + (int64_t)m * p.ldc;
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int n = n0 + wn * S::WTN + j * 16 + 4 * g;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (n + e < N) {
          float x = acc[i][j][e];
          if (bias) x += bias[n + e];
          crow[n + e] = x;
        }
      }
    }
  }
}

}  // namespace cmpext3
