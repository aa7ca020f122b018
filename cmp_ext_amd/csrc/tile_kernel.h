// Large-shape f16/bf16 GEMM for gfx950: C = A * op(B) (+ bias), fp32 accumulate.
//
// Counterpart of gemm_fp16_ampere_optimized_v3 (src/cuda/fp16_matmul.cu:63-283)
// and gemm_bf16_kernel (src/cuda/bf16_matmul.cu:51-226): same contract (row-major
// A[M,K], B[K,N], C[M,N]; zero-filled out-of-range loads, per-element masked
// stores), but built around the CDNA4 matrix cores instead of SIMT half2 FMAs,
// and accumulating in fp32.
//
// Structure (one workgroup = one BM x BN output tile, WM x WN waves):
//   * BK = 64.  A and B tiles are staged in LDS, two stages (double buffer),
//     one barrier per K step.  Global loads for step k+1 are issued before the
//     MFMAs of step k and written to LDS after them.
//   * Global loads are 128-bit buffer loads; out-of-range chunks (rows >= M,
//     columns >= N, k >= K) use an offset beyond the descriptor's range, so
//     the hardware returns zeros without touching memory.
//   * A [M,K] is K-contiguous and lands in LDS as is.  B [K,N] (matmul) is
//     N-contiguous: each thread loads an 8(k) x 8(n) block, transposes it in
//     registers (v_perm) and stores eight K-contiguous 16-byte rows, so both
//     operands are read back with one ds_read_b128 per MFMA fragment.
//     B [N,K] (a Linear weight) is already K-contiguous and is staged like A.
//   * LDS rows are 128 bytes with the pair-swizzle of lds_off128(): fragment
//     reads and all tile stores are free of bank conflicts.
//   * Each wave owns a (BM/WM) x (BN/WN) block of 32x32 fp32 accumulators fed
//     by v_mfma_f32_32x32x16_{f16,bf16}: per 16-deep k step a 128x128 wave
//     tile reads 8 fragments (32 VGPRs) for 16 MFMAs.
#pragma once

#include "device_common.h"

namespace cmpext3 {

template <int BM, int BN, int WM, int WN>
struct TileShape {
  static constexpr int BK = 64;
  static constexpr int NT = WM * WN * 64;
  static constexpr int WTM = BM / WM;
  static constexpr int WTN = BN / WN;
  static constexpr int FM = WTM / 32;  // 32x32 accumulator blocks per wave
  static constexpr int FN = WTN / 32;
  static constexpr int A_BYTES = BM * 128;
  static constexpr int B_BYTES = BN * 128;
  static constexpr int STAGE = A_BYTES + B_BYTES;
  static constexpr int LDS = 2 * STAGE;
  static constexpr int A_LD = BM * 8 / NT;  // 16-byte A chunks per thread
  static constexpr int B_LD = BN * 8 / NT;  // NK layout: 16-byte B chunks per thread
  static constexpr int B_BLK = BN;  // KN layout: 8x8 blocks in a B stage (8 k-blocks x BN/8)
  static constexpr int B_BLD = (B_BLK + NT - 1) / NT;
  static_assert(WTM % 32 == 0 && WTN % 32 == 0, "wave tile must be a multiple of 32");
  static_assert(LDS <= 160 * 1024, "LDS budget");
  static_assert(BM * 8 % NT == 0 && BN * 8 % NT == 0, "whole chunk rows per pass");
};

template <typename T, bool KN, int BM, int BN, int WM, int WN>
__global__ void __launch_bounds__(WM * WN * 64, 1) gemm_tile_kernel(const GemmParams p) {
  using S = TileShape<BM, BN, WM, WN>;
  constexpr int NT = S::NT, FM = S::FM, FN = S::FN;
  __shared__ __attribute__((aligned(1024))) unsigned char smem[S::LDS];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WN;
  const int wn = wave - wm * WN;

  int tm, tn;
  tile_coords(blockIdx.x, p.tiles_m, p.tiles_n, p.group_m, tm, tn);
  const int m0 = tm * BM;
  const int n0 = tn * BN;
  const int M = p.M, N = p.N, K = p.K;
  const int64_t lda = p.lda, ldb = p.ldb;
  const int64_t bz = blockIdx.z;
  const T* Abase = (const T*)p.A + bz * p.stride_a + (int64_t)m0 * lda;
  const T* Bbase = KN ? (const T*)p.B + bz * p.stride_b + n0
                      : (const T*)p.B + bz * p.stride_b + (int64_t)n0 * ldb;

  // ---- per-thread load descriptors, fixed for the whole K loop ----
  // A (and NK-layout B) chunk loads: thread -> chunk c = tid%8 of rows
  // tid/8 + (NT/8)*i.  Row r+NT/8 is (NT/16)*256 bytes further on in LDS.
  constexpr int RSTEP = NT / 8;
  static_assert(RSTEP % 16 == 0, "row step must keep the LDS swizzle phase");
  const int ch = tid & 7;
  const int crow = tid >> 3;
  const uint32_t a_goff = (uint32_t)(crow * lda + 8 * ch) * (uint32_t)sizeof(T);
  const uint32_t a_rstep = (uint32_t)(RSTEP * lda) * (uint32_t)sizeof(T);
  const uint32_t c_soff = lds_off128(crow, ch);
  const int a_rows = M - m0 - crow;  // row i is valid when RSTEP*i < a_rows
  // KN-layout B: thread -> 8x8 block (k-block kc = tid%8, n-block nc = tid/8).
  const int kc = tid & 7, nc = tid >> 3;
  const bool b_blk = (S::B_BLK % NT == 0) || tid < S::B_BLK;
  const bool b_col_ok = b_blk && (n0 + 8 * nc < N);
  const uint32_t b_goff = KN ? (uint32_t)((8 * kc) * ldb + 8 * nc) * (uint32_t)sizeof(T)
                             : (uint32_t)(crow * ldb + 8 * ch) * (uint32_t)sizeof(T);
  const uint32_t b_rstep = (uint32_t)(RSTEP * ldb) * (uint32_t)sizeof(T);
  const int b_rows = N - n0 - crow;
  const uint32_t ldb_bytes = (uint32_t)(ldb * (int64_t)sizeof(T));
  static_assert(!KN || S::B_BLD == 1, "KN layout: one 8x8 block per thread");

  u32x4 ra[S::A_LD];
  u32x4 rb[KN ? 8 : S::B_LD];

  auto load_tile = [&](int k0) {
    const __amdgpu_buffer_rsrc_t ra_rsrc = make_rsrc(Abase + k0);
    const bool a_kok = k0 + 8 * ch < K;
#pragma unroll
    for (int i = 0; i < S::A_LD; ++i) {
      const bool ok = a_kok && (RSTEP * i < a_rows);
      ra[i] = buf_load16(ra_rsrc, ok ? a_goff + i * a_rstep : kBufOOB);
    }
    if (KN) {
      const __amdgpu_buffer_rsrc_t rb_rsrc = make_rsrc(Bbase + (int64_t)k0 * ldb);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const bool ok = b_col_ok && (k0 + 8 * kc + j < K);
        rb[j] = buf_load16(rb_rsrc, ok ? b_goff + j * ldb_bytes : kBufOOB);
      }
    } else {
      const __amdgpu_buffer_rsrc_t rb_rsrc = make_rsrc(Bbase + k0);
#pragma unroll
      for (int i = 0; i < S::B_LD; ++i) {
        const bool ok = a_kok && (RSTEP * i < b_rows);
        rb[i] = buf_load16(rb_rsrc, ok ? b_goff + i * b_rstep : kBufOOB);
      }
    }
  };

  auto store_tile = [&](int stage) {
    unsigned char* sA = smem + stage * S::STAGE;
    unsigned char* sB = sA + S::A_BYTES;
#pragma unroll
    for (int i = 0; i < S::A_LD; ++i) *(u32x4*)(sA + c_soff + i * (RSTEP / 2) * 256) = ra[i];
    if (KN) {
      if (b_blk) {
        u32x4 cols[8];
        transpose8x8_b16(rb, cols);
#pragma unroll
        for (int j = 0; j < 8; ++j) *(u32x4*)(sB + lds_off128(8 * nc + j, kc)) = cols[j];
      }
    } else {
#pragma unroll
      for (int i = 0; i < S::B_LD; ++i) *(u32x4*)(sB + c_soff + i * (RSTEP / 2) * 256) = rb[i];
    }
  };

  // Fragment read offsets: row r32 of the wave's first 32-row block at chunk
  // 2*ks + h (k16 step ks, lane half h); each further 32-row block is 4096
  // bytes further on (the swizzle repeats every 16 rows).
  const int r32 = lane & 31, h = lane >> 5;
  uint32_t fa_off[4], fb_off[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    fa_off[ks] = lds_off128(wm * S::WTM + r32, 2 * ks + h);
    fb_off[ks] = lds_off128(wn * S::WTN + r32, 2 * ks + h);
  }

  f32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  auto compute = [&](int stage) {
    const unsigned char* sA = smem + stage * S::STAGE;
    const unsigned char* sB = sA + S::A_BYTES;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      u32x4 af[FM], bf[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i) af[i] = *(const u32x4*)(sA + fa_off[ks] + i * 4096);
#pragma unroll
      for (int j = 0; j < FN; ++j) bf[j] = *(const u32x4*)(sB + fb_off[ks] + j * 4096);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = Mfma32<T>::mma(bf[j], af[i], acc[i][j]);
    }
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

  // ---- epilogue: register 4q..4q+3 of block (i, j) is C[m][n..n+3] with
  // m = 32i + lane%32 and n = 32j + 8q + 4*(lane/32) ----
  T* Cb = (T*)p.C + bz * p.stride_c;
  const T* bias = (const T*)p.bias;
#pragma unroll
  for (int i = 0; i < FM; ++i) {
    const int m = m0 + wm * S::WTM + i * 32 + r32;
    if (m >= M) continue;
    T* crow = Cb + (int64_t)m * p.ldc;
#pragma unroll
    for (int j = 0; j < FN; ++j) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int n = n0 + wn * S::WTN + j * 32 + 8 * q + 4 * h;
        if (n >= N) continue;
        float v[4] = {acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
        if (n + 4 <= N) {
          if (bias) {
            const u32x2 bb = *(const u32x2*)(bias + n);
            v[0] += from_bits<T>((uint16_t)(bb.x & 0xFFFF));
            v[1] += from_bits<T>((uint16_t)(bb.x >> 16));
            v[2] += from_bits<T>((uint16_t)(bb.y & 0xFFFF));
            v[3] += from_bits<T>((uint16_t)(bb.y >> 16));
          }
          *(u32x2*)(crow + n) = u32x2{pack2<T>(v[0], v[1]), pack2<T>(v[2], v[3])};
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            if (n + e < N) {
              float x = v[e];
              if (bias) x += from_bits<T>(((const uint16_t*)bias)[n + e]);
              ((uint16_t*)crow)[n + e] = to_bits<T>(x);
            }
          }
        }
      }
    }
  }
}

}  // namespace cmpext3
