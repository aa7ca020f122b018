// Large-shape f16/bf16 GEMM for gfx950: C = A * op(B) (+ bias), fp32 accumulate.
//
// Counterpart of gemm_fp16_ampere_optimized_v3 (src/cuda/fp16_matmul.cu:63-283)
// and gemm_bf16_kernel (src/cuda/bf16_matmul.cu:51-226): same contract (row-major
// A[M,K], B[K,N], C[M,N]; zero-filled out-of-range loads, per-element masked
// stores), but built around the CDNA4 matrix cores instead of SIMT half2 FMAs,
// and accumulating in fp32.
//
// Structure (one workgroup of 4 waves = one BM x BN output tile):
//   * BK = 32.  Every operand tile goes global -> LDS by buffer_load_dwordx4
//     ... lds (LDS DMA: no registers, no ds_write), into a ring of NS LDS
//     stages.  The loads of K step t+NS-1 are issued while step t computes, so
//     about NS-2 steps of matrix-core time cover the global-memory latency
//     (a two-stage ring leaves the latency exposed on MI355X).
//   * Step t+1 is certified (its DMA complete in every wave) at the barrier
//     that ends step t-1, so the fragment reads for step t+1 are issued
//     during step t, before that step's barrier: the barrier never waits on
//     LDS latency.
//   * A [M,K] and B [N,K] (the Linear-weight layout) are K-contiguous: LDS
//     rows of 64 bytes (four 16-byte chunks), XOR-swizzled by row/4 so that a
//     32x32x16 fragment read (16 rows per phase, one chunk) is conflict free.
//     One ds_read_b128 per fragment.
//   * B [K,N] (matmul) is N-contiguous: it stays [k][n] in LDS (64-byte
//     segments XOR-swizzled by k%4) and each fragment is read with two
//     ds_read_b64_tr_b16, the CDNA4 transposing LDS read: a 16-lane group
//     pointing at a 4(k) x 16(n) block receives it transposed, lane i holding
//     column i at 4 consecutive k.
//   * Out-of-range chunks (rows >= M, columns >= N, k >= K) use an offset past
//     the buffer descriptor's range: the hardware writes zeros into LDS and
//     touches no memory.
//   * Each wave owns a (BM/WM) x (BN/WN) block of 32x32 fp32 accumulators
//     (AGPRs) fed by v_mfma_f32_32x32x16_{f16,bf16}.  The LDS reads of the
//     next sub-step's fragments and the DMA pieces of step t+NS-1 are spread
//     evenly between the MFMAs of both sub-steps (16 k each), so neither the
//     LDS queue nor the per-CU memory address FIFOs fill and hold up the
//     matrix-core issue.
#pragma once

#include "device_common.h"

namespace cmpext3 {

template <int BM, int BN, int WM, int WN, bool KN, int NS_, int BK_>
struct TileShape {
  static constexpr int BK = BK_;
  static constexpr int NS = NS_;
  static constexpr int ROW = BK * 2;  // bytes per LDS row of a K-contiguous operand
  static constexpr int NT = WM * WN * 64;
  static constexpr int WTM = BM / WM;
  static constexpr int WTN = BN / WN;
  static constexpr int FM = WTM / 32;  // 32x32 accumulator blocks per wave
  static constexpr int FN = WTN / 32;
  static constexpr int A_BYTES = BM * ROW;
  static constexpr int B_PITCH = KN ? (BN * 2 + 255) / 256 * 256 : ROW;  // bytes per LDS row of B
  static constexpr int B_BYTES = KN ? BK * B_PITCH : (BN + 63) / 64 * 64 * ROW;  // rows >= BN are OOB
  static constexpr int STAGE = A_BYTES + B_BYTES;
  static constexpr int LDS = NS * STAGE;
  static constexpr int A_DMA = A_BYTES / 1024 / 4;  // 1 KB LDS-DMA loads per wave per stage
  static constexpr int B_DMA = B_BYTES / 1024 / 4;
  static constexpr int DMA = A_DMA + B_DMA;
  static_assert(NT == 256, "four waves");
  static_assert(WTM % 32 == 0 && WTN % 32 == 0, "wave tile must be a multiple of 32");
  static_assert(A_BYTES % 4096 == 0 && B_BYTES % 4096 == 0, "whole DMA loads per wave");
  static_assert(BK == 32 || BK == 64, "64- or 128-byte rows");
  static_assert(BK == 32 ? NS >= 3 : NS == 2, "BK 32: ring of >= 3 stages; BK 64: two stages");
  static_assert(LDS <= 160 * 1024, "LDS budget");
};

// LDS byte offset of 16-byte chunk `chunk` (0..3) of row `row` in a tile of
// 64-byte rows: groups of four rows fill one 256-byte bank line, chunks are
// XORed with (row/4)%4, so 16 consecutive rows at one chunk hit 16 distinct
// 4-bank groups.
__device__ __forceinline__ uint32_t lds_off64(int row, int chunk) {
  return (uint32_t)((row >> 2) * 256 + 16 * (4 * (row & 3) + (chunk ^ ((row >> 2) & 3))));
}

// Row and chunk that lane `lane` of 1 KB LDS-DMA load `slot` must fetch so
// that LDS holds the lds_off64() layout (inverse of lds_off64 at byte
// slot*1024 + 16*lane).
__device__ __forceinline__ void dma64_geom(int slot, int lane, int& row, int& chunk) {
  row = 16 * slot + 4 * (lane >> 4) + ((lane & 15) >> 2);
  chunk = (lane & 3) ^ (lane >> 4);
}

// K-contiguous tiles: 64-byte rows (BK = 32) use lds_off64, 128-byte rows
// (BK = 64) use lds_off128; both are conflict free for 16 consecutive rows
// at one chunk, and chunk 2*ks + h of either is chunk h XOR 32*ks in bytes.
template <int BK>
__device__ __forceinline__ uint32_t kc_off(int row, int chunk) {
  return BK == 32 ? lds_off64(row, chunk) : lds_off128(row, chunk);
}
template <int BK>
__device__ __forceinline__ void kc_geom(int slot, int lane, int& row, int& chunk) {
  if (BK == 32)
    dma64_geom(slot, lane, row, chunk);
  else
    dma128_geom(slot, lane, row, chunk);
}

// [k][n] layout of an N-contiguous B tile: rows of `pitch` bytes (a multiple
// of 256), 64-byte segments XORed with k%4.  Lane `lane` of DMA load `slot`
// fetches row k, columns n..n+7.
__device__ __forceinline__ void dma_kn_geom(int slot, int lane, int pitch, int& k, int& n) {
  const int pos = slot * 1024 + 16 * lane;
  k = pos / pitch;
  const int within = pos - k * pitch;
  const int seg = (within >> 6) ^ (k & 3);
  n = (seg * 64 + (within & 63)) >> 1;
}

template <typename T, bool KN, int BM, int BN, int WM, int WN, int NS, int BK = 32>
__global__ void __launch_bounds__(WM * WN * 64, 1) gemm_tile_kernel(const GemmParams p) {
  using S = TileShape<BM, BN, WM, WN, KN, NS, BK>;
  constexpr int FM = S::FM, FN = S::FN;
  __shared__ __attribute__((aligned(1024))) unsigned char smem[S::LDS];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
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

  // ---- per-lane DMA sources, fixed for the whole K loop ----
  // offsets are relative to the step's first k; rows past the matrix are OOB
  uint32_t a_off[S::A_DMA];
  int a_kx[S::A_DMA];  // k offset of the lane's chunk within the step
#pragma unroll
  for (int i = 0; i < S::A_DMA; ++i) {
    int row, chunk;
    kc_geom<BK>(wave * S::A_DMA + i, lane, row, chunk);
    a_off[i] = (m0 + row < M) ? (uint32_t)(row * lda + 8 * chunk) * (uint32_t)sizeof(T) : kBufOOB;
    a_kx[i] = 8 * chunk;
  }
  uint32_t b_off[S::B_DMA];
  int b_kx[S::B_DMA];
#pragma unroll
  for (int i = 0; i < S::B_DMA; ++i) {
    if (KN) {
      int k, n;
      dma_kn_geom(wave * S::B_DMA + i, lane, S::B_PITCH, k, n);
      const bool ok = n < BN && n0 + n < N;
      b_off[i] = ok ? (uint32_t)(k * ldb + n) * (uint32_t)sizeof(T) : kBufOOB;
      b_kx[i] = k;
    } else {
      int row, chunk;
      kc_geom<BK>(wave * S::B_DMA + i, lane, row, chunk);
      b_off[i] = (row < BN && n0 + row < N) ? (uint32_t)(row * ldb + 8 * chunk) * (uint32_t)sizeof(T) : kBufOOB;
      b_kx[i] = 8 * chunk;
    }
  }

  // LDS-DMA load `d` (0 .. DMA-1; A pieces first, then B) of K step `kt`, into
  // ring slot kt % NS.  Every k is checked against K, so steps at or past the
  // end load zeros.
  auto dma_piece = [&](int kt, int d) {
    const int k0 = kt * S::BK;
    const uint32_t sA = lds_addr(smem) + (uint32_t)((kt % NS) * S::STAGE);
    const int krem = K - k0;
    if (d < S::A_DMA) {
      const int i = d;
      dma_load16(make_rsrc_sgpr(Abase + k0), a_kx[i] < krem ? a_off[i] : kBufOOB,
                 sA + (wave * S::A_DMA + i) * 1024);
    } else {
      const int i = d - S::A_DMA;
      dma_load16(make_rsrc_sgpr(KN ? Bbase + (int64_t)k0 * ldb : Bbase + k0), b_kx[i] < krem ? b_off[i] : kBufOOB,
                 sA + S::A_BYTES + (wave * S::B_DMA + i) * 1024);
    }
  };
  auto load_step = [&](int kt) {
#pragma unroll
    for (int d = 0; d < S::DMA; ++d) dma_piece(kt, d);
  };
  // Wait until at most NS-3 steps' DMA are in flight (so every step up to
  // the one two ahead has landed in this wave's share of LDS), then barrier:
  // after it, that step is complete for the whole workgroup.
  auto certify = [&]() {
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" : : "n"(NS >= 3 ? (NS - 3) * S::DMA : 0) : "memory");
  };

  // ---- fragment read addresses ----
  const int r32 = lane & 31, h = lane >> 5;
  const uint32_t fa0 = kc_off<BK>(wm * S::WTM + r32, h);  // sub-step ks: ^ (ks << 5)
  uint32_t fb0[KN ? FN : 1];
  if (KN) {
    // transposing reads: lane (group G = lane/16, s = lane%16) points at row
    // 8*(G/2) + s/4 (+ 4 for the second read, + 16 for sub-step 1), columns
    // 32j + 16*(G%2) + 4*(s%4) of the wave's block.
    const int G = lane >> 4, s = lane & 15;
    const int k = 8 * (G >> 1) + (s >> 2);
    const int seg0 = (wn * S::WTN) >> 5;
#pragma unroll
    for (int j = 0; j < FN; ++j)
      fb0[j] = (uint32_t)(k * S::B_PITCH + (((seg0 + j) ^ (k & 3)) << 6) + 32 * (G & 1) + 8 * (s & 3));
  } else {
    fb0[0] = kc_off<BK>(wn * S::WTN + r32, h);
  }

  f32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  typedef short s16x4 __attribute__((ext_vector_type(4)));
  u32x4 fa[2][FM], fb[2][FN];
  // LDS read r (0 .. RD-1) of sub-step ks of step kt into fragment buffer buf:
  // r < FM reads A block r; then B (two transposing reads per block for
  // [K,N], one ds_read_b128 for [N,K]).
  constexpr int RD = FM + (KN ? 2 : 1) * FN;
  auto read_one = [&](int kt, int ks, int buf, int r) {
    const unsigned char* sA = smem + (kt % NS) * S::STAGE;
    const unsigned char* sB = sA + S::A_BYTES;
    if (r < FM) {
      fa[buf][r] = *(const u32x4*)(sA + (fa0 ^ (uint32_t)(ks << 5)) + r * 32 * S::ROW);
    } else if (KN) {
      const int j = (r - FM) >> 1, half = (r - FM) & 1;
      const unsigned char* q = sB + fb0[j] + ks * 16 * S::B_PITCH + half * 4 * S::B_PITCH;
      const u32x2 v = __builtin_bit_cast(
          u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)q));
      if (half == 0) {
        fb[buf][j].x = v.x;
        fb[buf][j].y = v.y;
      } else {
        fb[buf][j].z = v.x;
        fb[buf][j].w = v.y;
      }
    } else {
      const int j = r - FM;
      fb[buf][j] = *(const u32x4*)(sB + (fb0[0] ^ (uint32_t)(ks << 5)) + j * 32 * S::ROW);
    }
  };
  // One sub-step (16 k) of MFMAs on fragment buffer `buf`, with the reads of
  // the next sub-step's fragments (into the other buffer) spread over its
  // MFMA slots (all 16 of a 128x128 wave block; the first three quarters of
  // smaller blocks, whose last reads would otherwise land too late) and DMA
  // pieces [d0, d1) of step `dkt` spread evenly:
  // short bursts keep the per-CU address FIFOs and the LDS queue from
  // filling, which would stall the MFMA issue behind them.  A scheduling
  // barrier after every MFMA slot keeps the compiler from regrouping them.
  constexpr int X = FM * FN;
  constexpr int XR = X >= 16 ? X : (3 * X + 3) / 4;  // MFMA slots that carry reads
  auto substep = [&](int buf, int rkt, int rks, int d0, int d1, int dkt) {
#pragma unroll
    for (int x = 0; x < X; ++x) {
      const int i = x / FN, j = x % FN;
      acc[i][j] = Mfma32<T>::mma(fb[buf][j], fa[buf][i], acc[i][j]);
#pragma unroll
      for (int r = 0; r < RD; ++r)
        if (x < XR && r * XR / RD == x) read_one(rkt, rks, buf ^ 1, r);
#pragma unroll
      for (int d = 0; d < S::DMA; ++d)
        if (d >= d0 && d < d1 && (d - d0) * X / (d1 - d0) == x) dma_piece(dkt, d);
      __builtin_amdgcn_sched_barrier(0);  // keep the slots in this order
    }
  };

  const int nk = (K + S::BK - 1) / S::BK;
  if constexpr (NS >= 3) {
    if (nk > 0) {
    // BK = 32, ring of NS stages: step t+2 is certified at the barrier that
    // ends step t, so both sub-steps read ahead and no barrier waits on LDS.
#pragma unroll
    for (int t = 0; t < NS - 1; ++t) load_step(t);
    certify();
#pragma unroll
    for (int r = 0; r < RD; ++r) read_one(0, 0, 0, r);
    for (int kt = 0; kt < nk; ++kt) {
      // sub-step 0 reads sub-step 1's fragments; sub-step 1 reads step kt+1's
      // first fragments (certified at the last barrier; after the last step
      // this reads a stale slot, which is never used).  Step kt+NS-1's DMA is
      // split over both.
      substep(0, kt, 1, 0, S::DMA / 2, kt + NS - 1);
      substep(1, kt + 1, 0, S::DMA / 2, S::DMA, kt + NS - 1);
      certify();  // step kt+2
    }
    asm volatile("s_waitcnt vmcnt(0)" : : : "memory");  // no LDS DMA may outlive the workgroup
    }
  } else if (nk > 0) {
    // BK = 64, two stages of 64 KB (256 x 256): the barrier of step t sits
    // before its last sub-step, once every fragment of step t is in
    // registers and step t+1 has landed.  Right after it the freed slot
    // starts receiving step t+2 (first half of its DMA in the last sub-step,
    // second half in sub-step 0 of step t+1), and the last sub-step's MFMAs
    // cover the reads of step t+1's first fragments.
    constexpr int KS = S::BK / 16;  // sub-steps per step
    constexpr int H = S::DMA / 2;
    load_step(0);
#pragma unroll
    for (int d = 0; d < H; ++d) dma_piece(1, d);
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" : : "n"(H) : "memory");  // step 0 landed
#pragma unroll
    for (int r = 0; r < RD; ++r) read_one(0, 0, 0, r);
    for (int kt = 0; kt < nk; ++kt) {
      substep(0, kt, 1, H, S::DMA, kt + 1);
#pragma unroll
      for (int ks = 1; ks < KS - 1; ++ks) substep(ks & 1, kt, ks + 1, 0, 0, 0);
      // every fragment of step kt read, step kt+1 landed (this wave), then barrier
      asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" : : : "memory");
      substep((KS - 1) & 1, kt + 1, 0, 0, H, kt + 2);
    }
    asm volatile("s_waitcnt vmcnt(0)" : : : "memory");  // no LDS DMA may outlive the workgroup
  }

  // ---- epilogue.  Register 4q+e of block (i, j) is C[m][n] with m = 32i + lane%32 and
  // n = 32j + 8q + 4h + e (h = lane/32): four consecutive columns per lane.
  // After rounding to 16-bit pairs, one v_permlane32_swap per dword trades
  // q = 1 of the lower half-wave for q = 0 of the upper half (and q = 3 for
  // q = 2), so every lane holds 8 consecutive columns, n = 32j + 16pp + 8h + 0..7
  // (pp = 0, 1), and C is written with 16-byte stores: half as many store
  // instructions as 8-byte pieces, which is what bounds this tail. ----
  T* Cb = (T*)p.C + bz * p.stride_c;
  const uint16_t* cbias = p.bias_row ? nullptr : (const uint16_t*)p.bias;  // per column
  const uint16_t* rbias = p.bias_row ? (const uint16_t*)p.bias : nullptr;  // per row
  const bool st16 = (p.ldc & 7) == 0;
  const int mw = m0 + wm * S::WTM, nw = n0 + wn * S::WTN;
#pragma unroll
  for (int i = 0; i < FM; ++i) {
    const int m = mw + i * 32 + r32;
    const float bm = (rbias != nullptr && m < M) ? from_bits<T>(rbias[m]) : 0.f;
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      uint32_t P[4][2];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = acc[i][j][4 * q + e];
        if (rbias) {
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] += bm;
        }
        if (cbias) {
          const int n = nw + j * 32 + 8 * q + 4 * h;
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (n + e < N) v[e] += from_bits<T>(cbias[n + e]);
        }
        P[q][0] = pack2<T>(v[0], v[1]);
        P[q][1] = pack2<T>(v[2], v[3]);
      }
#pragma unroll
      for (int pp = 0; pp < 2; ++pp)
#pragma unroll
        for (int w = 0; w < 2; ++w) {
          const auto sw = __builtin_amdgcn_permlane32_swap(P[2 * pp][w], P[2 * pp + 1][w], false, false);
          P[2 * pp][w] = sw[0];
          P[2 * pp + 1][w] = sw[1];
        }
      if (m >= M) continue;
#pragma unroll
      for (int pp = 0; pp < 2; ++pp) {
        const int n = nw + j * 32 + 16 * pp + 8 * h;
        if (n >= N) continue;
        T* dst = Cb + (int64_t)m * p.ldc + n;
        const u32x4 v = {P[2 * pp][0], P[2 * pp][1], P[2 * pp + 1][0], P[2 * pp + 1][1]};
        if (n + 8 <= N) {
          if (st16) {
            *(u32x4*)dst = v;
          } else {  // ldc % 8 == 4: 8-byte aligned rows
            *(u32x2*)dst = u32x2{v.x, v.y};
            *(u32x2*)(dst + 4) = u32x2{v.z, v.w};
          }
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (n + e < N) ((uint16_t*)dst)[e] = (uint16_t)(v[e >> 1] >> (16 * (e & 1)));
        }
      }
    }
  }
}

}  // namespace cmpext3
