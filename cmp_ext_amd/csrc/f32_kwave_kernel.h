// fp32 GEMM, 64x64 (or 16x64) output tile with K split four ways across the
// workgroup's waves.
//
// For products that leave a CU only one or two workgroups (2048 x 1024 x 1024:
// 512 tiles of 64x64, 128 of 128x128), the tiles of gemm_f32_kernel run
// latency-bound: a 64x64 workgroup there gives each wave 16 MFMAs per 16-k
// step.  Here every wave owns the whole 64x64 tile over its own quarter of the K
// steps (steps wave, wave + 4, wave + 8, ...): 64 MFMAs per step, like one wave of
// the 128x128 tile, from LDS that only that wave writes (its own ring of NS
// stages, filled by its own LDS-DMA), so the main loop needs no barrier, only the
// wave's own "s_waitcnt vmcnt".  At the end the four partial tiles are summed
// through LDS in a fixed order (wave 0 + 1 + 2 + 3: deterministic), each wave
// adding and storing 16 of the 64 rows.
//
// BM = 16 (16x64 tiles, four workgroups per CU) serves products with M <= 16,
// which are bound by streaming B: the 64-row tile would compute 48 zero rows.
//
// Same contract, layouts and fragment order as gemm_f32_kernel (f32_kernel.h):
// A (and B given as [N,K]) as [row][16 floats] with chunks XORed by (row/4)%4, B
// given as [K,N] as [k][64 floats] with 16-float segments XORed by (k/4)%4; 4-byte
// LDS-DMA for any alignment, 16-byte (DMA16) when the selector has checked that
// rows are 16-byte aligned and K (and N for [K,N]) are multiples of 4; SPLITK
// stores fp32 partials for skinny_reduce_kernel<float>.  The products are summed
// in another order than gemm_f32_kernel's (per-wave partials), so results may
// differ from the other fp32 tiles in the last bits (within the fp32 bound).
#pragma once

#include "f32_kernel.h"

namespace cmpext3 {

template <int BM, bool KN, int NS, bool SPLITK = false, bool DMA16 = false>
__global__ void __launch_bounds__(256, BM == 16 ? 4 : 2) gemm_f32_kwave_kernel(const GemmParams p) {
  static_assert(BM == 16 || BM == 64, "tile rows");
  constexpr int BN = 64, BK = 16, FM = BM / 16;
  constexpr int A_BYTES = BM * BK * 4, B_BYTES = BN * BK * 4, SUB = A_BYTES + B_BYTES;  // bytes per step
  constexpr int NA = DMA16 ? A_BYTES / 1024 : A_BYTES / 256;  // DMA instructions per step, all by this wave
  constexpr int NB = DMA16 ? B_BYTES / 1024 : B_BYTES / 256;
  static_assert(NS >= 2 && (NS - 2) * (NA + NB) <= 63, "ring depth / vmcnt range");
  static_assert(4 * NS * SUB * (BM == 16 ? 4 : 2) <= 160 * 1024, "workgroups per CU");
  __shared__ __attribute__((aligned(1024))) unsigned char smem[4 * NS * SUB];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

  int tm, tn, bzi;
  tile_coords(blockIdx.x, blockIdx.z, gridDim.z, p.tiles_m, p.tiles_n, p.group_m, tm, tn, bzi);
  const int m0 = tm * BM, n0 = tn * BN;
  const int M = p.M, N = p.N;
  const int64_t lda = p.lda, ldb = p.ldb;
  const int ks = SPLITK ? bzi % p.splits : 0;
  const int64_t bz = SPLITK ? bzi / p.splits : bzi;
  const int kbeg = SPLITK ? ks * p.ksplit : 0;
  const int K = SPLITK ? min(p.K - kbeg, p.ksplit) : p.K;
  const float* Abase = (const float*)p.A + bz * p.stride_a + (int64_t)m0 * lda + kbeg;
  const float* Bbase = KN ? (const float*)p.B + bz * p.stride_b + (int64_t)kbeg * ldb + n0
                          : (const float*)p.B + bz * p.stride_b + (int64_t)n0 * ldb + kbeg;

  // ---- DMA sources of one step (the inverse of the LDS layouts), relative to its k0 ----
  // Row blocks (f32_off): 4-byte instruction t writes slots 16 (t % 4) .. +15 of group
  // t / 4, lane l element l % 4 of slot 16 (t % 4) + l / 4; 16-byte instruction t writes
  // group t, lane l slot l.  B as [K,N]: 4-byte instruction t writes row k = t, lane l in
  // segment slot l/16 holding data segment slot ^ ((k/4)%4); 16-byte: floats 256t + 4l .. +3.
  uint32_t a_off[NA], b_off[NB];
  int a_k[NA], b_k[NB];
  auto row_piece = [&](int t, int& row, int& k) {
    int r, c;
    f32_slot_src(DMA16 ? lane : 16 * (t & 3) + (lane >> 2), r, c);
    row = DMA16 ? 16 * t + r : 16 * (t >> 2) + r;
    k = DMA16 ? 4 * c : 4 * c + (lane & 3);
  };
#pragma unroll
  for (int t = 0; t < NA; ++t) {
    int row, k;
    row_piece(t, row, k);
    a_off[t] = (m0 + row < M) ? (uint32_t)(row * lda + k) * 4u : kBufOOB;
    a_k[t] = k;
  }
#pragma unroll
  for (int t = 0; t < NB; ++t) {
    if (KN) {
      int k, n;
      if (DMA16) {
        const int f = 256 * t + 4 * lane;
        k = f / BN;
        n = 16 * (((f % BN) >> 4) ^ ((k >> 2) & 3)) + (f & 15);
      } else {
        k = t;
        n = 16 * ((lane >> 4) ^ ((k >> 2) & 3)) + (lane & 15);
      }
      b_off[t] = (n0 + n < N) ? (uint32_t)(k * ldb + n) * 4u : kBufOOB;
      b_k[t] = k;
    } else {
      int row, k;
      row_piece(t, row, k);
      b_off[t] = (n0 + row < N) ? (uint32_t)(row * ldb + k) * 4u : kBufOOB;
      b_k[t] = k;
    }
  }
  unsigned char* ring = smem + wave * (NS * SUB);
  // this wave's j-th step covers k0 = 16 * (4j + wave); steps past K load zeros
  // (a step wholly inside K loads its pieces unchecked; only the one holding K's end and
  // those past it compare each piece's k with K)
  auto load_step = [&](int j) {
    const int k0 = BK * (4 * j + wave);
    const int krem = K - k0;
    const uint32_t dst = lds_addr(ring) + (uint32_t)((j % NS) * SUB);
    const i32x4 ra = make_rsrc_sgpr(Abase + k0);
    const i32x4 rb = make_rsrc_sgpr(KN ? Bbase + (int64_t)k0 * ldb : Bbase + k0);
    if (krem >= BK) {  // wave-uniform
#pragma unroll
      for (int t = 0; t < NA; ++t) {
        if (DMA16)
          dma_load16(ra, a_off[t], dst + t * 1024);
        else
          dma_load4(ra, a_off[t], dst + t * 256);
      }
#pragma unroll
      for (int t = 0; t < NB; ++t) {
        if (DMA16)
          dma_load16(rb, b_off[t], dst + A_BYTES + t * 1024);
        else
          dma_load4(rb, b_off[t], dst + A_BYTES + t * 256);
      }
      return;
    }
#pragma unroll
    for (int t = 0; t < NA; ++t) {
      if (DMA16)
        dma_load16(ra, a_k[t] < krem ? a_off[t] : kBufOOB, dst + t * 1024);
      else
        dma_load4(ra, a_k[t] < krem ? a_off[t] : kBufOOB, dst + t * 256);
    }
#pragma unroll
    for (int t = 0; t < NB; ++t) {
      if (DMA16)
        dma_load16(rb, b_k[t] < krem ? b_off[t] : kBufOOB, dst + A_BYTES + t * 1024);
      else
        dma_load4(rb, b_k[t] < krem ? b_off[t] : kBufOOB, dst + A_BYTES + t * 256);
    }
  };

  // ---- fragments (lane r16 = l%16, g = l/16), the whole BM x 64 tile ----
  const int r16 = lane & 15, g = lane >> 4;
  const uint32_t fa = f32_off(r16, g);                    // + 1024 per 16 rows
  const uint32_t fb_nk = A_BYTES + f32_off(r16, g);       // + 1024 per 16 columns
  const uint32_t fb_kn = A_BYTES + (uint32_t)(4 * g * BN * 4 + 4 * r16);
  f32x4 acc[FM][4];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto compute_step = [&](int jstep) {
    const unsigned char* stage = ring + (jstep % NS) * SUB;
    f32x4 af[FM];
#pragma unroll
    for (int i = 0; i < FM; ++i) af[i] = *(const f32x4*)(stage + fa + i * 1024);
    if (KN) {
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        float bf[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) bf[j] = *(const float*)(stage + fb_kn + s * BN * 4 + ((j ^ g) << 6));
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[i][j] = mma_f32(bf[j], af[i][s], acc[i][j]);
      }
    } else {
      f32x4 bf[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) bf[j] = *(const f32x4*)(stage + fb_nk + j * 1024);
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[i][j] = mma_f32(bf[j][s], af[i][s], acc[i][j]);
    }
  };

  const int steps = (K + BK - 1) / BK;                            // 16-k steps of the workgroup
  const int mine = steps > wave ? (steps - wave + 3) / 4 : 0;     // of this wave
  // Step j: DMA step j+NS-1 into the slot step j-1 was read from (this wave's own reads
  // of it completed: their results fed step j-1's MFMAs), compute j, wait for step j+1.
#pragma unroll
  for (int t = 0; t < NS - 1; ++t) load_step(t);
  asm volatile("s_waitcnt vmcnt(%0)" : : "n"((NS - 2) * (NA + NB)) : "memory");
  for (int j = 0; j < mine; ++j) {
    load_step(j + NS - 1);
    compute_step(j);
    asm volatile("s_waitcnt vmcnt(%0)" : : "n"((NS - 2) * (NA + NB)) : "memory");
  }
  asm volatile("s_waitcnt vmcnt(0)" : : : "memory");  // no LDS DMA may outlive the loop

  // ---- sum the four partial tiles: of the FM x 4 16x16 blocks (flattened b = 4i + j),
  // wave w adds and stores blocks FM*w .. FM*w + FM-1 (BM = 64: the 16 rows of block row
  // w; BM = 16: column block w) ----
  __syncthreads();  // every wave is done with its ring
  f32x4* red = (f32x4*)smem;  // [wave][i][j][lane], FM * 4 KiB per wave
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) red[((wave * FM + i) * 4 + j) * 64 + lane] = acc[i][j];
  __syncthreads();
  f32x4 sum[FM];
#pragma unroll
  for (int t = 0; t < FM; ++t) {
    const int b = FM * wave + t;
    sum[t] = red[b * 64 + lane];
#pragma unroll
    for (int q = 1; q < 4; ++q) sum[t] += red[(q * 4 * FM + b) * 64 + lane];
  }

  // sum[t][e] = C[m0 + 16i + r16][n0 + 16j + 4g + e] for block b = FM*wave + t = 4i + j
  const float* bias = p.bias_row ? nullptr : (const float*)p.bias;
  const float* rbias = p.bias_row ? (const float*)p.bias : nullptr;
  const bool vec = ((p.ldc | N) & 3) == 0 && ((uintptr_t)((const float*)p.C + bz * p.stride_c) & 15) == 0;
  const __amdgpu_buffer_rsrc_t crs = make_rsrc((float*)p.C + bz * p.stride_c + (int64_t)m0 * p.ldc + n0);
  // every block's bias values before any store (a load after a store waits for it)
  f32x4 bb[FM];
#pragma unroll
  for (int t = 0; t < FM; ++t) {
    const int b = FM * wave + t;
    const int row = 16 * (b >> 2) + r16, col = 16 * (b & 3) + 4 * g;
    const float bm = (rbias != nullptr && m0 + row < M) ? rbias[m0 + row] : 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      bb[t][e] = bm + ((bias != nullptr && n0 + col + e < N) ? bias[n0 + col + e] : 0.f);
  }
#pragma unroll
  for (int t = 0; t < FM; ++t) {
    const int b = FM * wave + t;
    const int row = 16 * (b >> 2) + r16;
    const bool row_ok = m0 + row < M;
    const int col = 16 * (b & 3) + 4 * g;
    if constexpr (SPLITK) {
      const int batch = (int)gridDim.z / p.splits;
      float* part = p.partials + ((int64_t)ks * batch + bz) * M * N;
      if (row_ok && n0 + col < N) *(f32x4*)(part + (int64_t)(m0 + row) * N + n0 + col) = sum[t];
      continue;
    }
    f32x4 v = sum[t];
    if (p.bias != nullptr) v += bb[t];  // a bias per column or per row (one is zero in bb)
    if (vec) {
      buf_store16(crs, row_ok && n0 + col < N ? (uint32_t)(row * p.ldc + col) * 4u : kBufOOB, v);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        buf_store4(crs, row_ok && n0 + col + e < N ? (uint32_t)(row * p.ldc + col + e) * 4u : kBufOOB, v[e]);
    }
  }
}

}  // namespace cmpext3
