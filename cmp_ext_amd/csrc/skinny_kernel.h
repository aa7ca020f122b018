// Skinny-M f16/bf16 GEMM (M <= 64, B is [K,N]): C = A * B (+ bias).
//
// Decode-like shapes (e.g. 16 x 8192 x 8192) read B once and do ~16 flops per
// B byte, so they are bound by HBM bandwidth, not by the matrix cores.  The
// reference has no special path for them: its 128x128 tile kernel runs with
// 112 of 128 rows zero-filled and only ceil(N/128) workgroups
// (src/cuda/fp16_matmul.cu:318-321).  This kernel instead:
//   * gives each workgroup (4 waves) a 32-column strip of B and all of K, so
//     there are N/32 workgroups (256 for N = 8192: one per CU) and B is read
//     exactly once; strips are ordered so that neighbouring strips (the two
//     halves of each 128-byte line) run on the same XCD and share its L2;
//   * streams the strip, and the matching A columns, global -> LDS with
//     LDS-DMA (buffer_load_dwordx4 ... lds) through a ring of NS stages of KS
//     k-rows, keeping NS-2 stages (tens of KB per CU) in flight to cover HBM
//     latency without registers;
//   * reads B fragments with ds_read_b64_tr_b16 (LDS keeps B as [k][n]) and A
//     fragments with ds_read_b128 (A rows XOR-swizzled by row%16);
//   * splits every stage's 32-deep k-blocks over the 4 waves
//     (v_mfma_f32_16x16x32 with the M rows in the MFMA's 16-wide dimension)
//     and reduces the 4 partial sums in LDS at the end.
#pragma once

#include "device_common.h"

namespace cmpext3 {

constexpr int kSkinnyStrip = 32;  // columns per workgroup

template <int MB>
struct SkinnyShape {
  static constexpr int KS = MB <= 2 ? 256 : 128;  // k rows per stage
  static constexpr int B_BYTES = KS * kSkinnyStrip * 2;
  static constexpr int A_PITCH = KS * 2;           // bytes per A row in LDS
  static constexpr int A_BYTES = MB * 16 * A_PITCH;
  static constexpr int STAGE = A_BYTES + B_BYTES;
  static constexpr int NS = (160 * 1024) / STAGE > 8 ? 8 : (160 * 1024) / STAGE;
  static constexpr int A_DMA = A_BYTES / 4096;  // 1 KB LDS-DMA loads per wave per stage
  static constexpr int B_DMA = B_BYTES / 4096;
  static constexpr int DMA = A_DMA + B_DMA;
  static constexpr int KB = KS / 32 / 4;  // 32-deep k-blocks per wave per stage
  static_assert(A_BYTES % 4096 == 0 && B_BYTES % 4096 == 0, "whole DMA loads per wave");
  static_assert(NS >= 3 && (NS - 2) * DMA <= 63, "ring depth / vmcnt range");
  static_assert(4 * MB * 16 * kSkinnyStrip * 4 <= NS * STAGE, "reduction fits the ring");
};

// The streamed operand (B, W, or A for the swapped kernel) of one launch is read with the non-temporal policy when it
// is at least kStreamOnceBytes: a smaller one may still sit in the 256 MB Infinity Cache at
// the next call, which the policy would give up (MI355X, fp16, operands rotating over four
// buffers: 16 x 8192 x 8192 27.6 -> 26.1 us, W of 8192 x 8192 for one row 28.3 -> 25.0 us,
// 14336 x 4096 for 16 rows 25.9 -> 23.3 us; 4096 x 4096, whose four copies fit the cache,
// 7.9 -> 8.8 us).
constexpr int64_t kStreamOnceBytes = 64ll << 20;
inline bool stream_once(int64_t rows, int64_t cols, int64_t stride, unsigned batch) {
  return rows * cols * 2 * (stride != 0 ? (int64_t)batch : 1) >= kStreamOnceBytes;
}

__device__ __forceinline__ int strip_order(int wg, int total) {
  const int xcd = wg & 7, local = wg >> 3;
  const int base = total >> 3, rem = total & 7;
  return xcd * base + (xcd < rem ? xcd : rem) + local;
}

// Byte offset in the B part of a stage of row k, 16-column half h (0/1):
// rows are 64 bytes; the halves of rows with bit 3 of k set are swapped so
// that a transposing read (rows k..k+3 and k+8..k+11 of one half) is
// conflict free.
__device__ __forceinline__ uint32_t skinny_off(int k, int h) {
  return (uint32_t)(k * 64 + ((h ^ ((k >> 3) & 1)) << 5));
}

template <typename T, int MB>
__global__ void __launch_bounds__(256) gemm_skinny_narrow_kernel(const GemmParams p) {
  using S = SkinnyShape<MB>;
  constexpr int NS = S::NS;
  __shared__ __attribute__((aligned(1024))) unsigned char smem[NS * S::STAGE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int strip = strip_order(blockIdx.x, gridDim.x);
  const int n0 = strip * kSkinnyStrip;
  const int M = p.M, N = p.N, K = p.K;
  const int64_t bz = blockIdx.z;
  const int64_t lda = p.lda, ldb = p.ldb;
  const T* Ab = (const T*)p.A + bz * p.stride_a;
  const T* Bb = (const T*)p.B + bz * p.stride_b + n0;

  // ---- DMA sources (inverse of the LDS layouts), relative to the stage's k0 ----
  uint32_t b_off[S::B_DMA];
  int b_k[S::B_DMA];
#pragma unroll
  for (int i = 0; i < S::B_DMA; ++i) {
    const int row = 16 * (wave * S::B_DMA + i) + (lane >> 2);  // 16 rows of 64 bytes per load
    const int pos = 16 * (lane & 3);
    const int h = (pos >> 5) ^ ((row >> 3) & 1);
    const int col = h * 16 + ((pos & 31) >> 1);
    b_off[i] = (n0 + col < N) ? (uint32_t)(row * ldb + col) * (uint32_t)sizeof(T) : kBufOOB;
    b_k[i] = row;
  }
  uint32_t a_off[S::A_DMA];
  int a_k[S::A_DMA];
#pragma unroll
  for (int i = 0; i < S::A_DMA; ++i) {
    const int pos = (wave * S::A_DMA + i) * 1024 + 16 * lane;
    const int row = pos / S::A_PITCH;
    const int chunk = ((pos % S::A_PITCH) >> 4) ^ (row & 15);
    a_off[i] = (row < M) ? (uint32_t)(row * lda + 8 * chunk) * (uint32_t)sizeof(T) : kBufOOB;
    a_k[i] = 8 * chunk;
  }
  auto load_stage = [&](int st) {
    const int k0 = st * S::KS;
    const uint32_t dst = lds_addr(smem) + (uint32_t)((st % NS) * S::STAGE);
    const int krem = K - k0;
    const i32x4 rb = make_rsrc_sgpr(Bb + (int64_t)k0 * ldb);
    const i32x4 ra = make_rsrc_sgpr(Ab + k0);
#pragma unroll
    for (int i = 0; i < S::B_DMA; ++i)
      dma_load16(rb, b_k[i] < krem ? b_off[i] : kBufOOB, dst + (wave * S::B_DMA + i) * 1024);
#pragma unroll
    for (int i = 0; i < S::A_DMA; ++i)
      dma_load16(ra, a_k[i] < krem ? a_off[i] : kBufOOB, dst + S::B_BYTES + (wave * S::A_DMA + i) * 1024);
  };

  // ---- fragments: lane (c = l%16, g = l/16) ----
  // B (first MFMA operand): column nb + c at k = kb + 8g .. +7, two
  //   transposing reads of source rows kb + 8g + 4r + c/4, columns 4*(c%4)..
  // A (second operand): A[16*mb + c][kb + 8g .. +7]
  const int c = lane & 15, g = lane >> 4;
  typedef short s16x4 __attribute__((ext_vector_type(4)));
  f32x4 acc[2][MB];
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[h][mb] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto compute_stage = [&](int st) {
    const unsigned char* stage = smem + (st % NS) * S::STAGE;
#pragma unroll
    for (int b = 0; b < S::KB; ++b) {
      const int kb = (wave * S::KB + b) * 32;
      u32x4 af[MB];
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
        af[mb] = *(const u32x4*)(stage + S::B_BYTES + (16 * mb + c) * S::A_PITCH + 16 * ((kb / 8 + g) ^ c));
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        u32x4 bf;
#pragma unroll
        for (int r = 0; r < 2; ++r) {
          const int k = kb + 8 * g + 4 * r + (c >> 2);
          const unsigned char* q = stage + skinny_off(k, h) + 8 * (c & 3);
          const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)q);
          const u32x2 v2 = __builtin_bit_cast(u32x2, v);
          bf[2 * r] = v2.x;
          bf[2 * r + 1] = v2.y;
        }
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) acc[h][mb] = Mfma<T>::mma(bf, af[mb], acc[h][mb]);
      }
    }
  };

  const int nst = (K + S::KS - 1) / S::KS;
  // Step st: DMA stage st+NS-1 (zeros past K), compute st, then wait until at
  // most NS-2 stages' DMA are in flight and barrier: stage st+1 is complete
  // in LDS and stage st's slot may be refilled.
#pragma unroll
  for (int t = 0; t < NS - 1; ++t) load_stage(t);
  asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" : : "n"((NS - 2) * S::DMA) : "memory");
  for (int st = 0; st < nst; ++st) {
    load_stage(st + NS - 1);
    compute_stage(st);
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" : : "n"((NS - 2) * S::DMA) : "memory");
  }
  asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" : : : "memory");

  // ---- reduce the 4 waves' partial sums through LDS (the ring is free) ----
  // acc[h][mb][r] = C[16*mb + c][n0 + 16*h + 4*g + r]
  float* red = (float*)smem;  // [wave][MB*16][32]
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        red[(wave * MB * 16 + 16 * mb + c) * kSkinnyStrip + 16 * h + 4 * g + r] = acc[h][mb][r];
  __syncthreads();
  T* Cb = (T*)p.C + bz * p.stride_c;
  const uint16_t* bias = (const uint16_t*)p.bias;
  for (int o = tid; o < MB * 16 * kSkinnyStrip; o += 256) {
    const int row = o / kSkinnyStrip, col = o % kSkinnyStrip;
    const int n = n0 + col;
    if (row >= M || n >= N) continue;
    float s = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) s += red[(w * MB * 16 + row) * kSkinnyStrip + col];
    if (bias) s += from_bits<T>(bias[p.bias_row ? row : n]);
    ((uint16_t*)(Cb + (int64_t)row * p.ldc))[n] = to_bits<T>(s);
  }
}

// Skinny-M product with B given as [N, K] (a Linear weight used as W^T, decode
// shapes such as x[16, 4096] * W[14336, 4096]^T): each workgroup owns SW rows of W
// (SW output columns) and all of K.  W rows are K-contiguous, so a stage holds KS k
// of each row -- 2*KS contiguous bytes per row per load, which keeps HBM reads in
// long runs -- stored like A (rows of 2*KS bytes, 16-byte chunks XORed with row%16)
// and read with ds_read_b128 straight into the MFMA's first operand.  As above,
// the stage's 32-deep k-blocks are split over the 4 waves and the partial sums
// reduced in LDS at the end; no workspace, no second launch.
// NSMAX caps the ring depth (otherwise as many stages as fit, up to 8), e.g. so that two
// workgroups share a CU.
//
// SWAP: the same kernel for the mirror case, N <= 16*MB and M large (C = A B with a
// narrow B, e.g. attention's P V, or x W^T with few rows of W, e.g. a router): the
// streamed rows are A's (strips of SW rows of C), the small operand is B -- as [N, K]
// (XKN false: read like A above) or as [K, N] (XKN true: stored [k][n] in rows of 32*MB
// bytes, kn128_off / kn_off, and read with the transposing ds_read_b64_tr_b16) -- and C
// is written transposed from the reduction.
template <int MB, int SW, int KS_, int NSMAX = 8, bool SWAP = false>
struct SkinnyNKShape {
  static constexpr int KS = KS_;
  static constexpr int PITCH = KS * 2;             // bytes per LDS row (W and A alike)
  static constexpr int W_BYTES = SW * PITCH;
  static constexpr int A_BYTES = MB * 16 * PITCH;  // = KS rows of 32*MB bytes ([k][n] form)
  static constexpr int STAGE = W_BYTES + A_BYTES;
  static constexpr int NS = (160 * 1024) / STAGE > NSMAX ? NSMAX : (160 * 1024) / STAGE;
  static constexpr int W_DMA = W_BYTES / 4096;  // 1 KB LDS-DMA loads per wave per stage
  static constexpr int A_DMA = A_BYTES / 4096;
  static constexpr int DMA = W_DMA + A_DMA;
  static constexpr int KB = KS / 32 / 4;        // 32-deep k-blocks per wave per stage
  // reduction rows (floats): MB*16 x rows of SW, or (SWAP) SW rows of MB*16 + 4 (the pad
  // spreads the four lane groups' writes over the banks)
  static constexpr int RED = SWAP ? SW * (MB * 16 + 4) : MB * 16 * SW;
  static_assert(W_BYTES % 4096 == 0 && A_BYTES % 4096 == 0 && KB >= 1, "whole DMA loads per wave");
  static_assert(NS >= 3 && (NS - 2) * DMA <= 63, "ring depth / vmcnt range");
  static_assert(4 * RED * 4 <= NS * STAGE, "reduction fits the ring");
};

// NT: stream W with the non-temporal policy (W larger than the Infinity Cache would keep
// for the next call).
template <typename T, int MB, int SW, int KS, bool NT = false, int NSMAX = 8, bool SWAP = false, bool XKN = false>
__global__ void __launch_bounds__(256) gemm_skinny_nk_kernel(const GemmParams p) {
  using S = SkinnyNKShape<MB, SW, KS, NSMAX, SWAP>;
  constexpr int NS = S::NS;
  constexpr int NB = SW / 16;  // 16-column blocks per strip
  constexpr int XP = 32 * MB;  // bytes per k row of a [K, N] small operand in LDS
  static_assert(!XKN || (SWAP && (XP == 128 || XP == 256)), "[K, N] small operand: swapped roles, 64 or 128 columns");
  __shared__ __attribute__((aligned(1024))) unsigned char smem[NS * S::STAGE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // Workgroup w (x fastest, then z) runs on XCD w % 8: each XCD takes a contiguous range of
  // (z, strip) in z-major order, so its L2 holds the small operand of one or two batch
  // entries (or K ranges) rather than of all of them.
  // (32-bit arithmetic where the grid allows: a 64-bit division costs every wave ~0.5 us)
  int zz, strip;
  const int64_t total = (int64_t)gridDim.x * gridDim.z;
  if (gridDim.z == 1) {
    zz = 0;
    strip = strip_order(blockIdx.x, gridDim.x);
  } else if (total <= 0x7FFFFFFF) {
    const uint32_t order = (uint32_t)strip_order(blockIdx.x + gridDim.x * blockIdx.z, (int)total);
    zz = (int)(order / gridDim.x);
    strip = (int)(order - (uint32_t)zz * gridDim.x);
  } else {
    const int64_t wg = blockIdx.x + (int64_t)gridDim.x * blockIdx.z;
    const int64_t xcd = wg & 7, base = total >> 3, rem = total & 7;
    const int64_t order = xcd * base + (xcd < rem ? xcd : rem) + (wg >> 3);
    zz = (int)(order / gridDim.x);
    strip = (int)(order - (int64_t)zz * gridDim.x);
  }
  const int n0 = strip * SW;
  // split K (p.splits > 1): grid.z = batch * splits, split ks sums k in [ks*ksplit, +ksplit)
  // and writes fp32 partials[ks][batch][M][N] (summed, biased and rounded by a second launch)
  const int splits = p.splits > 1 ? p.splits : 1;
  const int ks = zz % splits;
  const int64_t bz = zz / splits;
  const int kbeg = ks * p.ksplit;
  const int K = splits > 1 ? min(p.K - kbeg, p.ksplit) : p.K;
  // W: the streamed operand (B's rows, or A's when SWAP); X: the small one (A, or B)
  const int w_rows = SWAP ? p.M : p.N, x_rows = SWAP ? p.N : p.M;
  const int64_t ldw = SWAP ? p.lda : p.ldb, ldx = SWAP ? p.ldb : p.lda;
  const T* Wb = (SWAP ? (const T*)p.A + bz * p.stride_a : (const T*)p.B + bz * p.stride_b) + (int64_t)n0 * ldw + kbeg;
  const T* Xb = (SWAP ? (const T*)p.B + bz * p.stride_b : (const T*)p.A + bz * p.stride_a) +
                (XKN ? (int64_t)kbeg * ldx : (int64_t)kbeg);

  // ---- DMA sources: rows of PITCH bytes, chunk c of row r stored at chunk c ^ (r % 16) ----
  auto geom = [&](int piece, int& row, int& chunk) {
    const int pos = piece * 1024 + 16 * lane;
    row = pos / S::PITCH;
    chunk = ((pos % S::PITCH) >> 4) ^ (row & 15);
  };
  uint32_t w_off[S::W_DMA];
  int w_k[S::W_DMA];
#pragma unroll
  for (int i = 0; i < S::W_DMA; ++i) {
    int row, chunk;
    geom(wave * S::W_DMA + i, row, chunk);
    w_off[i] = (n0 + row < w_rows) ? (uint32_t)(row * ldw + 8 * chunk) * (uint32_t)sizeof(T) : kBufOOB;
    w_k[i] = 8 * chunk;
  }
  uint32_t a_off[S::A_DMA];
  int a_k[S::A_DMA];
#pragma unroll
  for (int i = 0; i < S::A_DMA; ++i) {
    if constexpr (XKN) {  // row k of the stage, columns n .. n+7
      int k, n;
      if constexpr (XP == 128)
        dma_kn128_geom(wave * S::A_DMA + i, lane, k, n);
      else
        dma_kn_geom(wave * S::A_DMA + i, lane, XP, k, n);
      a_off[i] = (n < x_rows) ? (uint32_t)(k * ldx + n) * (uint32_t)sizeof(T) : kBufOOB;
      a_k[i] = k;
    } else {
      int row, chunk;
      geom(wave * S::A_DMA + i, row, chunk);
      a_off[i] = (row < x_rows) ? (uint32_t)(row * ldx + 8 * chunk) * (uint32_t)sizeof(T) : kBufOOB;
      a_k[i] = 8 * chunk;
    }
  }
  auto load_stage = [&](int st) {
    const int k0 = st * S::KS;
    const uint32_t dst = lds_addr(smem) + (uint32_t)((st % NS) * S::STAGE);
    const int krem = K - k0;
    const i32x4 rw = make_rsrc_sgpr(Wb + k0);
    const i32x4 ra = make_rsrc_sgpr(XKN ? Xb + (int64_t)k0 * ldx : Xb + k0);
#pragma unroll
    for (int i = 0; i < S::W_DMA; ++i)
      if constexpr (NT)
        dma_load16_stream(rw, w_k[i] < krem ? w_off[i] : kBufOOB, dst + (wave * S::W_DMA + i) * 1024);
      else
        dma_load16(rw, w_k[i] < krem ? w_off[i] : kBufOOB, dst + (wave * S::W_DMA + i) * 1024);
#pragma unroll
    for (int i = 0; i < S::A_DMA; ++i)
      dma_load16(ra, a_k[i] < krem ? a_off[i] : kBufOOB, dst + S::W_BYTES + (wave * S::A_DMA + i) * 1024);
  };

  // ---- fragments: lane (c = l%16, g = l/16) ----
  // first MFMA operand: W row 16h + c at k = kb + 8g .. +7
  // second operand:     X row 16mb + c at the same k
  const int c = lane & 15, g = lane >> 4;
  typedef short s16x4 __attribute__((ext_vector_type(4)));
  f32x4 acc[NB][MB];
#pragma unroll
  for (int h = 0; h < NB; ++h)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[h][mb] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto compute_stage = [&](int st) {
    const unsigned char* stage = smem + (st % NS) * S::STAGE;
#pragma unroll
    for (int b = 0; b < S::KB; ++b) {
      const int kc = (wave * S::KB + b) * 4 + g;  // 16-byte chunk of the lane's 8 k
      u32x4 af[MB];
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        if constexpr (XKN) {
          // rows 8kc + 4r + c/4, columns 16mb + 4(c%4) .. +3: the transposing read hands
          // lane c column 16mb + c at the four k
#pragma unroll
          for (int r = 0; r < 2; ++r) {
            const int k = 8 * kc + 4 * r + (c >> 2), bc = 32 * mb + 8 * (c & 3);
            const unsigned char* q = stage + S::W_BYTES + (XP == 128 ? kn128_off(k, bc) : kn_off(k, XP, bc));
            const u32x2 v = __builtin_bit_cast(
                u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)q));
            af[mb][2 * r] = v.x;
            af[mb][2 * r + 1] = v.y;
          }
        } else {
          af[mb] = *(const u32x4*)(stage + S::W_BYTES + (16 * mb + c) * S::PITCH + 16 * (kc ^ c));
        }
      }
#pragma unroll
      for (int h = 0; h < NB; ++h) {
        const u32x4 wf = *(const u32x4*)(stage + (16 * h + c) * S::PITCH + 16 * (kc ^ c));
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) acc[h][mb] = Mfma<T>::mma(wf, af[mb], acc[h][mb]);
      }
    }
  };

  const int nst = (K + S::KS - 1) / S::KS;
#pragma unroll
  for (int t = 0; t < NS - 1; ++t) load_stage(t);
  asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" : : "n"((NS - 2) * S::DMA) : "memory");
  for (int st = 0; st < nst; ++st) {
    load_stage(st + NS - 1);
    compute_stage(st);
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" : : "n"((NS - 2) * S::DMA) : "memory");
  }
  asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" : : : "memory");

  // ---- reduce the 4 waves' partial sums through LDS (the ring is free) ----
  // acc[h][mb][r] = (X row 16*mb + c) . (W row n0 + 16*h + 4*g + r)
  float* red = (float*)smem;
  T* Cb = (T*)p.C + bz * p.stride_c;
  float* part = splits > 1 ? p.partials + ((int64_t)ks * (gridDim.z / splits) + bz) * p.M * p.N : nullptr;
  const uint16_t* bias = (const uint16_t*)p.bias;
  if constexpr (SWAP) {
    // red[wave][W row][X row], rows of RP floats; C[n0 + W row][X row]
    constexpr int XR = MB * 16, RP = MB * 16 + 4;
#pragma unroll
    for (int h = 0; h < NB; ++h)
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int r = 0; r < 4; ++r) red[(wave * SW + 16 * h + 4 * g + r) * RP + 16 * mb + c] = acc[h][mb][r];
    __syncthreads();
    for (int o = tid; o < SW * XR; o += 256) {
      const int wr = o / XR, xr = o % XR;
      const int m = n0 + wr;
      if (m >= w_rows || xr >= x_rows) continue;
      float s = 0.f;
#pragma unroll
      for (int w = 0; w < 4; ++w) s += red[(w * SW + wr) * RP + xr];
      if (part) {
        part[(int64_t)m * p.N + xr] = s;
        continue;
      }
      if (bias) s += from_bits<T>(bias[p.bias_row ? m : xr]);
      ((uint16_t*)(Cb + (int64_t)m * p.ldc))[xr] = to_bits<T>(s);
    }
  } else {
    // red[wave][X row][SW]; C[X row][n0 + column]
#pragma unroll
    for (int h = 0; h < NB; ++h)
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int r = 0; r < 4; ++r) red[(wave * MB * 16 + 16 * mb + c) * SW + 16 * h + 4 * g + r] = acc[h][mb][r];
    __syncthreads();
    for (int o = tid; o < MB * 16 * SW; o += 256) {
      const int row = o / SW, col = o % SW;
      const int n = n0 + col;
      if (row >= x_rows || n >= w_rows) continue;
      float s = 0.f;
#pragma unroll
      for (int w = 0; w < 4; ++w) s += red[(w * MB * 16 + row) * SW + col];
      if (part) {
        part[(int64_t)row * p.N + n] = s;
        continue;
      }
      if (bias) s += from_bits<T>(bias[p.bias_row ? row : n]);
      ((uint16_t*)(Cb + (int64_t)row * p.ldc))[n] = to_bits<T>(s);
    }
  }
}

}  // namespace cmpext3
