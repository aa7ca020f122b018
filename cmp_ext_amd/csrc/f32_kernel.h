// fp32 GEMM on the CDNA4 fp32 matrix cores: C = A * op(B) (+ bias).
//
// Counterpart of gemm_fp32_ga100_kernel (src/cuda/fp32_matmul.cu:31-184):
// same contract (row-major, any M/N/K, fully bounds-checked loads and stores),
// but the products run on v_mfma_f32_16x16x4_f32 (fused multiply-add with fp32
// accumulation) instead of the reference's separate __fmul_rn/__fadd_rn SIMT
// loop, which exists only to dodge a GA100 FMA limit (fp32_matmul.cu:20-26).
//
// Any alignment is accepted: global memory is read by 4-byte LDS-DMA
// (buffer_load_dword ... lds, 256 contiguous LDS bytes per instruction), with
// an out-of-range offset (hardware zero-fill) for every element past M, N or
// K, so ragged shapes such as 4097 x 3001 x 2049 need no special casing.
// Operands whose rows are 16-byte aligned with K (and N for B given as [K,N])
// a multiple of 4 use 16-byte LDS-DMA instead (DMA16: buffer_load_dwordx4 ...
// lds, 1 KiB per instruction): a quarter of the load instructions and their
// address work, measured 132 -> 142 TFLOP/s at 4096^3 on 128 x 128 tiles.  The
// DMA fills a ring of NS stages of BK = 16 k; each wave counts its own DMA in
// vmcnt, and one "s_waitcnt vmcnt; s_barrier" per step certifies that the
// next stage is complete and that the slot about to be refilled is free, so
// NS-2 stages of loads are always in flight without staging registers.
//
// LDS layouts (per stage):
//   A, and B given as [N,K]: rows of 16 floats (64 bytes) in groups of 16 rows
//     (1 KiB); the 16-byte chunk c (k = 4c..4c+3) of row r sits at slot
//     f32_slot(r % 16, c) of its group, a layout measured free of LDS bank
//     conflicts for the fragment read (16 consecutive rows at one chunk per 16
//     lanes, ds_read_b128).  A DMA instruction writes a quarter of a group
//     (4-byte DMA) or a whole group (16-byte DMA), each lane fetching the
//     element f32_slot_src names for its slot.
//   B given as [K,N]: [k][n], rows of BN floats, 16-float segment s of row k
//     stored at segment s ^ ((k/4)%4): the fragment read of MFMA step s
//     (rows s, 4+s, 8+s, 12+s at 16 columns, ds_read_b32) hits 64 distinct
//     banks, and one DMA instruction writes 64 consecutive floats of a row.
// MFMA k-step s of lane group g uses k = 4g + s, so one ds_read_b128 per A
// fragment feeds four MFMAs.
#pragma once

#include "device_common.h"

namespace cmpext3 {

template <int BM, int BN, int NS_, bool DMA16 = false>
struct F32Shape {
  static constexpr int BK = 16;
  static constexpr int NS = NS_;
  static constexpr int NT = 256;  // 2 x 2 waves
  static constexpr int WTM = BM / 2, WTN = BN / 2;
  static constexpr int FM = WTM / 16, FN = WTN / 16;
  static constexpr int A_BYTES = BM * BK * 4;
  static constexpr int B_BYTES = BN * BK * 4;
  static constexpr int STAGE = A_BYTES + B_BYTES;
  static constexpr int A_DMA = A_BYTES / 256 / 4;  // 256-byte DMA instructions per wave per stage
  static constexpr int B_DMA = B_BYTES / 256 / 4;
  // DMA16: 1 KiB instructions t = 4i + wave, i < A16 (B16), skipping t >= A_BYTES / 1024
  static constexpr int A16 = (A_BYTES / 1024 + 3) / 4;
  static constexpr int B16 = (B_BYTES / 1024 + 3) / 4;
  static constexpr int DMA = DMA16 ? A16 + B16 : A_DMA + B_DMA;
  static_assert(BN % 64 == 0 && BM % 32 == 0, "whole DMA instructions per wave, 64-float B rows");
  static_assert(!DMA16 || NS == 2, "DMA16 waves may issue different counts: vmcnt(0) only");
  static_assert(NS >= 2 && (NS - 2) * DMA <= 63, "ring depth / vmcnt range");
  static_assert(NS * STAGE <= 160 * 1024, "LDS");
};

// 16-byte slot (0..63) of chunk c (0..3) of row r (0..15) in its 1 KiB group of 16 rows:
// with bits r0..r3 of r and c0, c1 of c, slot bits are r1^c0^c1, r0^r1^r3, r0^r3, r0,
// r2, r2^c1.  Found by sweeping GF(2)-linear layouts of the group on MI355X with the LDS
// bank-conflict counter (SQ_LDS_BANK_CONFLICT): for the fragment read (lane l reads chunk
// l / 16 of row l % 16, ds_read_b128) this one measured zero conflict cycles at every
// LDS base offset tried, where the earlier chunk ^ (r / 4) % 4 swizzle (four rows per 256
// bytes) took one extra cycle per read, as did a third of the layouts swept.
__device__ __forceinline__ int f32_slot(int r, int c) {
  const int r0 = r & 1, r1 = (r >> 1) & 1, r2 = (r >> 2) & 1, r3 = (r >> 3) & 1, c0 = c & 1, c1 = (c >> 1) & 1;
  return (r1 ^ c0 ^ c1) | ((r0 ^ r1 ^ r3) << 1) | ((r0 ^ r3) << 2) | (r0 << 3) | (r2 << 4) | ((r2 ^ c1) << 5);
}
// The row (0..15) and chunk whose data slot s of a group holds (the inverse of f32_slot).
__device__ __forceinline__ void f32_slot_src(int s, int& r, int& c) {
  const int s0 = s & 1, s1 = (s >> 1) & 1, s2 = (s >> 2) & 1, s3 = (s >> 3) & 1, s4 = (s >> 4) & 1, s5 = (s >> 5) & 1;
  const int r0 = s3, r1 = s1 ^ s2, r2 = s4, r3 = s2 ^ s3, c1 = s4 ^ s5, c0 = s0 ^ r1 ^ c1;
  r = r0 | (r1 << 1) | (r2 << 2) | (r3 << 3);
  c = c0 | (c1 << 1);
}
// Byte offset of 16-byte chunk `chunk` (0..3) of row `row` in a block of rows of 16 floats.
__device__ __forceinline__ uint32_t f32_off(int row, int chunk) {
  return (uint32_t)((row >> 4) * 1024 + 16 * f32_slot(row & 15, chunk));
}

// WAVES: waves per SIMD the kernel is compiled for (caps its registers at 512 / WAVES).
// Enough resident workgroups matter more than registers here: 96 x 64 tiles at 8
// waves per SIMD run all 2021 tiles of a 4097 x 3001 product in one round (measured
// 460 -> 421 us on MI355X against the compiler's choice of 7).
// SPLITK: grid.z = batch * p.splits; this workgroup sums its split's K range and
// stores the sums into p.partials (bias added by the reduction).
template <bool KN, int BM, int BN, int NS, int WAVES, bool SPLITK = false, bool DMA16 = false>
__global__ void __launch_bounds__(256, WAVES) gemm_f32_kernel(const GemmParams p) {
  using S = F32Shape<BM, BN, NS, DMA16>;
  constexpr int FM = S::FM, FN = S::FN;
  __shared__ __attribute__((aligned(1024))) unsigned char smem[NS * S::STAGE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;

  int tm, tn;
  int bzi;
  tile_coords(blockIdx.x, blockIdx.z, gridDim.z, p.tiles_m, p.tiles_n, p.group_m, tm, tn, bzi);
  const int m0 = tm * BM, n0 = tn * BN;
  const int M = p.M, N = p.N;
  const int64_t lda = p.lda, ldb = p.ldb;
  // split-K: entry bzi of the grid's z range is split bzi % splits of batch entry bzi / splits
  const int ks = SPLITK ? bzi % p.splits : 0;
  const int64_t bz = SPLITK ? bzi / p.splits : bzi;
  const int kbeg = SPLITK ? ks * p.ksplit : 0;
  const int K = SPLITK ? min(p.K - kbeg, p.ksplit) : p.K;  // this workgroup's K range
  const float* Abase = (const float*)p.A + bz * p.stride_a + (int64_t)m0 * lda + kbeg;
  const float* Bbase = KN ? (const float*)p.B + bz * p.stride_b + (int64_t)kbeg * ldb + n0
                          : (const float*)p.B + bz * p.stride_b + (int64_t)n0 * ldb + kbeg;

  // ---- DMA sources: the inverse of the LDS layouts, relative to the stage's k0 ----
  // Row blocks: 4-byte instruction t writes slots 16 (t % 4) .. +15 of group t / 4, lane l
  // element l % 4 of slot 16 (t % 4) + l / 4.
  uint32_t a_off[S::A_DMA];
  int a_k[S::A_DMA];
#pragma unroll
  for (int i = 0; i < S::A_DMA; ++i) {
    const int t = wave * S::A_DMA + i;
    int r, c;
    f32_slot_src(16 * (t & 3) + (lane >> 2), r, c);
    const int row = 16 * (t >> 2) + r;
    const int k = 4 * c + (lane & 3);
    a_off[i] = (m0 + row < M) ? (uint32_t)(row * lda + k) * 4u : kBufOOB;
    a_k[i] = k;
  }
  // B: [K,N] -> instruction t writes row k = t / (BN/64), floats 64*(t%(BN/64)) ..
  //    +63; lane l lands in segment slot 4*(t%(BN/64)) + l/16, which holds data
  //    segment slot ^ ((k/4)%4).  [N,K] -> as A.
  uint32_t b_off[S::B_DMA];
  int b_k[S::B_DMA];
#pragma unroll
  for (int i = 0; i < S::B_DMA; ++i) {
    const int t = wave * S::B_DMA + i;
    if (KN) {
      constexpr int PER_ROW = BN / 64;
      const int k = t / PER_ROW;
      const int seg = (4 * (t % PER_ROW) + (lane >> 4)) ^ ((k >> 2) & 3);
      const int n = 16 * seg + (lane & 15);
      b_off[i] = (n0 + n < N) ? (uint32_t)(k * ldb + n) * 4u : kBufOOB;
      b_k[i] = k;
    } else {
      int r, c;
      f32_slot_src(16 * (t & 3) + (lane >> 2), r, c);
      const int row = 16 * (t >> 2) + r;
      const int k = 4 * c + (lane & 3);
      b_off[i] = (n0 + row < N) ? (uint32_t)(row * ldb + k) * 4u : kBufOOB;
      b_k[i] = k;
    }
  }
  // DMA16 sources: A (and B as [N,K]) instruction t writes group t (rows 16t .. 16t+15),
  // lane l slot l; B as [K,N]: instruction t writes floats 256t + 4l .. +3 of the stage's
  // [16][BN] block.
  uint32_t va_off[S::A16], vb_off[S::B16];
  int va_k[S::A16], vb_k[S::B16];
  if constexpr (DMA16) {
#pragma unroll
    for (int i = 0; i < S::A16; ++i) {
      int r, c;
      f32_slot_src(lane, r, c);
      const int row = 16 * (4 * i + wave) + r;
      const int k = 4 * c;
      va_off[i] = (m0 + row < M) ? (uint32_t)(row * lda + k) * 4u : kBufOOB;
      va_k[i] = k;
    }
#pragma unroll
    for (int i = 0; i < S::B16; ++i) {
      if (KN) {
        const int f = 256 * (4 * i + wave) + 4 * lane;
        const int k = f / BN;
        const int n = 16 * (((f % BN) >> 4) ^ ((k >> 2) & 3)) + (f & 15);
        vb_off[i] = (n0 + n < N) ? (uint32_t)(k * ldb + n) * 4u : kBufOOB;
        vb_k[i] = k;
      } else {
        int r, c;
        f32_slot_src(lane, r, c);
        const int row = 16 * (4 * i + wave) + r;
        const int k = 4 * c;
        vb_off[i] = (n0 + row < N) ? (uint32_t)(row * ldb + k) * 4u : kBufOOB;
        vb_k[i] = k;
      }
    }
  }
  // Stage st's loads.  A stage wholly inside K loads every piece unchecked; only the stage
  // that holds K's end (and those past it, all zeros) compares each piece's k with K (the
  // per-piece compare and select on every stage cost 7 %: cfg5 419.5 -> 391.7 us).
  auto load_stage = [&](int st) {
    const int k0 = st * S::BK;
    const int krem = K - k0;
    const uint32_t dst = lds_addr(smem) + (uint32_t)((st % NS) * S::STAGE);
    const i32x4 ra = make_rsrc_sgpr(Abase + k0);
    const i32x4 rb = make_rsrc_sgpr(KN ? Bbase + (int64_t)k0 * ldb : Bbase + k0);
    const bool whole = krem >= S::BK;  // wave-uniform
    if constexpr (DMA16) {
      if (whole) {
#pragma unroll
        for (int i = 0; i < S::A16; ++i)
          if (4 * i + wave < S::A_BYTES / 1024) dma_load16(ra, va_off[i], dst + (4 * i + wave) * 1024);
#pragma unroll
        for (int i = 0; i < S::B16; ++i)
          if (4 * i + wave < S::B_BYTES / 1024) dma_load16(rb, vb_off[i], dst + S::A_BYTES + (4 * i + wave) * 1024);
        return;
      }
#pragma unroll
      for (int i = 0; i < S::A16; ++i)
        if (4 * i + wave < S::A_BYTES / 1024)
          dma_load16(ra, va_k[i] < krem ? va_off[i] : kBufOOB, dst + (4 * i + wave) * 1024);
#pragma unroll
      for (int i = 0; i < S::B16; ++i)
        if (4 * i + wave < S::B_BYTES / 1024)
          dma_load16(rb, vb_k[i] < krem ? vb_off[i] : kBufOOB, dst + S::A_BYTES + (4 * i + wave) * 1024);
    } else {
      if (whole) {
#pragma unroll
        for (int i = 0; i < S::A_DMA; ++i) dma_load4(ra, a_off[i], dst + (wave * S::A_DMA + i) * 256);
#pragma unroll
        for (int i = 0; i < S::B_DMA; ++i) dma_load4(rb, b_off[i], dst + S::A_BYTES + (wave * S::B_DMA + i) * 256);
        return;
      }
#pragma unroll
      for (int i = 0; i < S::A_DMA; ++i)
        dma_load4(ra, a_k[i] < krem ? a_off[i] : kBufOOB, dst + (wave * S::A_DMA + i) * 256);
#pragma unroll
      for (int i = 0; i < S::B_DMA; ++i)
        dma_load4(rb, b_k[i] < krem ? b_off[i] : kBufOOB, dst + S::A_BYTES + (wave * S::B_DMA + i) * 256);
    }
  };

  // ---- fragments: lane (r16 = l%16, g = l/16) ----
  const int r16 = lane & 15, g = lane >> 4;
  const uint32_t fa = f32_off(wm * S::WTM + r16, g);  // + 1024 per 16 rows
  const uint32_t fb_nk = S::A_BYTES + f32_off(wn * S::WTN + r16, g);
  // [K,N] B, MFMA step s, fragment j: row 4g + s, segment (wn*FN + j) ^ g, column r16.
  const uint32_t fb_kn = S::A_BYTES + (uint32_t)(4 * g * BN * 4 + 4 * r16);

  f32x4 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto compute_stage = [&](int st) {
    const unsigned char* stage = smem + (st % NS) * S::STAGE;
    f32x4 af[FM];
#pragma unroll
    for (int i = 0; i < FM; ++i) af[i] = *(const f32x4*)(stage + fa + i * 1024);
    if (KN) {
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        float bf[FN];
#pragma unroll
        for (int j = 0; j < FN; ++j)
          bf[j] = *(const float*)(stage + fb_kn + s * BN * 4 + (((wn * FN + j) ^ g) << 6));
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j) acc[i][j] = mma_f32(bf[j], af[i][s], acc[i][j]);
      }
    } else {
      f32x4 bf[FN];
#pragma unroll
      for (int j = 0; j < FN; ++j) bf[j] = *(const f32x4*)(stage + fb_nk + j * 1024);
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j) acc[i][j] = mma_f32(bf[j][s], af[i][s], acc[i][j]);
    }
  };
  auto certify = [&]() {
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" : : "n"((NS - 2) * S::DMA) : "memory");
  };

  const int nst = (K + S::BK - 1) / S::BK;
  // Step st: DMA stage st+NS-1 (zeros past K), compute st, certify st+1.
#pragma unroll
  for (int t = 0; t < NS - 1; ++t) load_stage(t);
  certify();
  for (int st = 0; st < nst; ++st) {
    load_stage(st + NS - 1);
    compute_stage(st);
    certify();
  }
  asm volatile("s_waitcnt vmcnt(0)" : : : "memory");  // no LDS DMA may outlive the workgroup

  if constexpr (SPLITK) {  // fp32 partial sums, four consecutive columns per store (N % 4 == 0)
    const int batch = (int)gridDim.z / p.splits;
    float* part = p.partials + ((int64_t)ks * batch + bz) * M * N;
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const int m = m0 + wm * S::WTM + i * 16 + r16;
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int n = n0 + wn * S::WTN + j * 16 + 4 * g;
        if (m < M && n < N) *(f32x4*)(part + (int64_t)m * N + n) = acc[i][j];
      }
    }
    return;
  }
  // acc[i][j][e] = C[m0 + wm*WTM + 16i + r16][n0 + wn*WTN + 16j + 4g + e]; elements
  // outside C get an out-of-range offset and are dropped by the store.
  const __amdgpu_buffer_rsrc_t crs = make_rsrc((float*)p.C + bz * p.stride_c + (int64_t)m0 * p.ldc + n0);
  const float* bias = p.bias_row ? nullptr : (const float*)p.bias;    // per column
  const float* rbias = p.bias_row ? (const float*)p.bias : nullptr;   // per row
  float bv[FN][4];
#pragma unroll
  for (int j = 0; j < FN; ++j)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int n = n0 + wn * S::WTN + j * 16 + 4 * g + e;
      bv[j][e] = (bias != nullptr && n < N) ? bias[n] : 0.f;
    }
  // C rows 16-byte aligned and N % 4 == 0: one 16-byte store per lane and block (the four
  // columns are all inside C or all outside), measured 8.3 -> 1.9 us per workgroup epilogue
  // on MI355X with every workgroup of a 256-CU launch storing at once.
  if (((p.ldc | N) & 3) == 0 && ((uintptr_t)((const float*)p.C + bz * p.stride_c) & 15) == 0) {
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const int row = wm * S::WTM + i * 16 + r16;
      const bool row_ok = m0 + row < M;
      const float bm = (rbias != nullptr && row_ok) ? rbias[m0 + row] : 0.f;
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int col = wn * S::WTN + j * 16 + 4 * g;
        f32x4 v = acc[i][j];
        if (bias != nullptr) v += f32x4{bv[j][0], bv[j][1], bv[j][2], bv[j][3]};
        if (rbias != nullptr) v += bm;
        buf_store16(crs, row_ok && n0 + col < N ? (uint32_t)(row * p.ldc + col) * 4u : kBufOOB, v);
      }
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < FM; ++i) {
    const int row = wm * S::WTM + i * 16 + r16;
    const bool row_ok = m0 + row < M;
    const float bm = (rbias != nullptr && row_ok) ? rbias[m0 + row] : 0.f;
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int col = wn * S::WTN + j * 16 + 4 * g;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const bool ok = row_ok && n0 + col + e < N;
        const float x = bias != nullptr ? acc[i][j][e] + bv[j][e]
                        : rbias != nullptr ? acc[i][j][e] + bm : acc[i][j][e];
        buf_store4(crs, ok ? (uint32_t)(row * p.ldc + col + e) * 4u : kBufOOB, x);
      }
    }
  }
}

}  // namespace cmpext3
