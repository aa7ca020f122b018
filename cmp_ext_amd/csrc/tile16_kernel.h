// Large-shape f16/bf16 GEMM for gfx950 on 16x16x32 matrix-core products:
// C = A * op(B) (+ bias), fp32 accumulate.
//
// Counterpart of gemm_fp16_ampere_optimized_v3 (src/cuda/fp16_matmul.cu:63-283)
// and gemm_bf16_kernel (src/cuda/bf16_matmul.cu:51-226): same contract (row-major
// A[M,K], B[K,N], C[M,N]; zero-filled out-of-range loads, per-element masked
// stores), built around the CDNA4 matrix cores and accumulating in fp32.
//
// Structure (one workgroup of WM x WN waves = one BM x BN tile):
//   * Each wave owns a (BM/WM) x (BN/WN) block of C as 16 x 16 blocks of fp32
//     accumulators, fed by v_mfma_f32_16x16x32_{f16,bf16}.  The 16-wide block
//     grain lets a 256 x 224 tile (the MLP shape) use the same grid as 256 x 256.
//   * Two waves per SIMD: the 256-row tiles run 8 waves (4 x 2, at most 256
//     VGPRs each) in one workgroup per CU, the 128 x 128 tile 4 waves (2 x 2) in
//     two workgroups per CU.  One wave's matrix products then run while the other
//     waits on LDS reads or on the issue of its LDS-DMA loads; measured on
//     MI355X, 8 waves beat 4 waves of twice the block (fewer fragment bytes per
//     MFMA, one wave per SIMD) by ~9 % in loop cycles and halve the epilogue.
//   * K steps of BK = 64 go global -> LDS by buffer_load_dwordx4 ... lds (LDS
//     DMA: no registers, no ds_write) into a two-stage ring.  A step is two
//     sub-steps of 32 k.  All reads of a step's slot are issued by the end of its
//     first sub-step (they fetch the second sub-step's fragments), so one barrier
//     between the two sub-steps both frees slot t and certifies step t+1; the
//     second sub-step then reads step t+1's first fragments and issues all of
//     step t+2's DMA into slot t, which has a sub-step and a half to land before
//     the next barrier.
//   * A (and B given as [N,K]) are K-contiguous: LDS rows of 128 bytes in the
//     lds_off128 layout, one ds_read_b128 per 16 x 32 fragment, conflict free.
//   * B given as [K,N] stays [k][n] in LDS (rows padded to a multiple of 256
//     bytes, swizzled by kn_off) and is read with
//     ds_read_b64_tr_b16, the CDNA4 transposing LDS read: two per fragment.
//   * Out-of-range pieces (rows >= M, columns >= N, k >= K) use an offset past
//     the buffer descriptor's range: the hardware writes zeros into LDS.
//   * The reads of the next sub-step's fragments and the DMA pieces are spread
//     one per MFMA slot, with a scheduling barrier after every slot.
//   * Epilogue: fp32 -> T, bias added in fp32 first (per column, or per row;
//     staged in LDS);
//     one v_permlane16_swap per dword pairs accumulator blocks j and j+1 so
//     that every lane holds 8 consecutive columns, and C is written with
//     16-byte stores covering 64 contiguous bytes of each of 16 rows.
#pragma once

#include <type_traits>
#include <utility>

#include "device_common.h"

namespace cmpext3 {

// f(std::integral_constant<int, I>) for I = 0 .. N-1, fully unrolled (register
// arrays indexed by I stay in registers).
template <typename F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

template <int BM, int BN, bool KN, int WM, int WN>
struct Tile16Shape {
  static constexpr int BK = 64;
  static constexpr int ROW = BK * 2;  // bytes per LDS row of a K-contiguous operand
  static constexpr int NW = WM * WN;
  static constexpr int WTM = BM / WM, WTN = BN / WN;
  static constexpr int FM = WTM / 16, FN = WTN / 16;
  static constexpr int A_BYTES = BM * ROW;
  static constexpr int B_PITCH = KN ? (BN * 2 + 255) / 256 * 256 : ROW;  // bytes per LDS row of B
  static constexpr int B_BYTES = KN ? BK * B_PITCH : (BN + 63) / 64 * 64 * ROW;  // rows >= BN are OOB
  // LDS: the two ring slots of A, then the two of B, so that a fragment read of either
  // slot is a fixed base register plus an immediate offset below 64 KiB
  static constexpr int B_REGION = 2 * A_BYTES;
  static constexpr int LDS = 2 * (A_BYTES + B_BYTES);
  static constexpr int A_DMA = A_BYTES / 1024 / NW;  // 1 KB LDS-DMA loads per wave per step
  static constexpr int B_DMA = B_BYTES / 1024 / NW;
  static constexpr int DMA = A_DMA + B_DMA;
  static_assert(WTM % 16 == 0 && WTN % 16 == 0, "16-row/column blocks");
  static_assert(A_BYTES % (1024 * NW) == 0 && B_BYTES % (1024 * NW) == 0, "whole DMA loads per wave");
  static_assert(LDS <= 160 * 1024, "LDS budget");
  static_assert(DMA <= 63, "vmcnt range");
  static_assert(A_BYTES + 14 * 2048 <= 65535 && B_BYTES + 36 * B_PITCH <= 65535, "immediate LDS offsets");
};

// BIAS: 0 none, 1 per column of C (Linear), 2 per row (conv 1x1).  A kernel per
// mode keeps the bias-free epilogue lean: the register allocator then keeps the
// accumulators in AGPRs through the main loop.
// SPLITK: grid.z = batch * p.splits; this workgroup sums its split's K range and
// stores the fp32 sums (no bias, no rounding) into p.partials.
// KCHECK: K (every split's K range) is not a multiple of 64, so the loads compare
// each piece's k with K; otherwise they load whole steps unchecked.
template <typename T, bool KN, int BM, int BN, int WM, int WN, int BIAS, int MINB, bool SPLITK = false,
          bool KCHECK = false>
__global__ void __launch_bounds__(64 * WM * WN, MINB) gemm_tile16_kernel(const GemmParams p) {
  using S = Tile16Shape<BM, BN, KN, WM, WN>;
  constexpr int FM = S::FM, FN = S::FN;
  __shared__ __attribute__((aligned(1024))) unsigned char smem[S::LDS];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
  const int wm = wave / WN, wn = wave % WN;

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
  const T* Abase = (const T*)p.A + bz * p.stride_a + (int64_t)m0 * lda + kbeg;
  const T* Bbase = KN ? (const T*)p.B + bz * p.stride_b + (int64_t)kbeg * ldb + n0
                      : (const T*)p.B + bz * p.stride_b + (int64_t)n0 * ldb + kbeg;

  // ---- per-lane DMA sources, relative to the step's first k; rows past the matrix are OOB ----
  uint32_t a_off[S::A_DMA];
  int a_kx[S::A_DMA];  // k offset of the lane's 16-byte piece within the step
#pragma unroll
  for (int i = 0; i < S::A_DMA; ++i) {
    int row, chunk;
    dma128_geom(wave * S::A_DMA + i, lane, row, chunk);
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
      b_off[i] = (n < BN && n0 + n < N) ? (uint32_t)(k * ldb + n) * (uint32_t)sizeof(T) : kBufOOB;
      b_kx[i] = k;
    } else {
      int row, chunk;
      dma128_geom(wave * S::B_DMA + i, lane, row, chunk);
      b_off[i] = (row < BN && n0 + row < N) ? (uint32_t)(row * ldb + 8 * chunk) * (uint32_t)sizeof(T) : kBufOOB;
      b_kx[i] = 8 * chunk;
    }
  }
  // LDS-DMA load d (A pieces first, then B) of K step kt into ring slot kt % 2.  A (and B
  // as [N,K]) keep one descriptor at the tile base and advance along K through the SGPR
  // offset; B as [K,N] gets a descriptor per step.  The destination goes through M0
  // (one s_add per piece from a per-wave base).  With CHECK each piece's k is compared
  // with K; a step at or past the end loads through an empty descriptor (num_records 0:
  // the hardware writes zeros and reads no memory), so the loop needs no branch for it.
  const i32x4 rsrc_a = make_rsrc_sgpr(Abase);
  const i32x4 rsrc_b_nk = make_rsrc_sgpr(Bbase);
  const uint32_t lds_a = lds_addr(smem) + (uint32_t)(wave * S::A_DMA * 1024);
  const uint32_t lds_b = lds_addr(smem) + (uint32_t)(S::B_REGION + wave * S::B_DMA * 1024);
  const int nk_all = (K + S::BK - 1) / S::BK;
  auto dma_piece = [&](int kt, auto slotc, auto dc, auto checkc) {
    constexpr int slot = decltype(slotc)::value, d = decltype(dc)::value;
    constexpr bool check = decltype(checkc)::value;
    const int k0 = kt * S::BK;
    const bool live = kt < nk_all;  // wave-uniform
    if constexpr (d < S::A_DMA) {
      constexpr uint32_t dst = (uint32_t)(slot * S::A_BYTES + d * 1024);
      const uint32_t voff = !check || a_kx[d] < K - k0 ? a_off[d] : kBufOOB;
      i32x4 r = rsrc_a;
      r[2] = live ? (int)kBufRecords : 0;
      dma_load16_m0(r, voff, (uint32_t)k0 * (uint32_t)sizeof(T), lds_a, std::integral_constant<uint32_t, dst>{});
    } else {
      constexpr int i = d - S::A_DMA;
      constexpr uint32_t dst = (uint32_t)(slot * S::B_BYTES + i * 1024);
      const uint32_t voff = !check || b_kx[i] < K - k0 ? b_off[i] : kBufOOB;
      i32x4 r = KN ? make_rsrc_sgpr(Bbase + (int64_t)(live ? k0 : 0) * ldb) : rsrc_b_nk;
      r[2] = live ? (int)kBufRecords : 0;
      dma_load16_m0(r, voff, KN ? 0u : (uint32_t)k0 * (uint32_t)sizeof(T), lds_b, std::integral_constant<uint32_t, dst>{});
    }
  };

  // ---- fragment addresses: lane (r16 = lane%16, G = lane/16) supplies row/column r16
  // and k = 8G .. 8G+7 of a 32-k sub-step ----
  const int r16 = lane & 15, G = lane >> 4;
  uint32_t fa_off[2];  // A block 0 of sub-step s (block i: + 16 rows = 2048 bytes)
#pragma unroll
  for (int s = 0; s < 2; ++s) fa_off[s] = lds_off128(wm * S::WTM + r16, 4 * s + G);
  uint32_t fb_off[KN ? FN : 2];
  if (KN) {
    // lanes of group G point at k row 8G + r16/4 (+4 for the second read, +32 for sub-step
    // 1), columns 16j + 4(r16%4) of the wave's block: a transposing read hands lane r16 of
    // the group column 16j + r16 at four consecutive k
    const int kr = 8 * G + (r16 >> 2);
#pragma unroll
    for (int j = 0; j < (KN ? FN : 2); ++j) {
      const int cb = (wn * S::WTN + 16 * j + 4 * (r16 & 3)) * 2;  // byte column
      // + (32s + 4 half) rows keeps both swizzle terms; the B region's start is folded in so
      // that the remaining offsets fit a read's immediate
      fb_off[j] = S::B_REGION + kn_off(kr, S::B_PITCH, cb);
    }
  } else {
#pragma unroll
    for (int s = 0; s < 2; ++s) fb_off[s] = S::B_REGION + lds_off128(wn * S::WTN + r16, 4 * s + G);
  }

  f32x4 acc[FM][FN];
  static_for<FM * FN>([&](auto xc) {
    constexpr int x = decltype(xc)::value;
    acc[x / FN][x % FN] = f32x4{0.f, 0.f, 0.f, 0.f};
  });

  typedef short s16x4 __attribute__((ext_vector_type(4)));
  u32x4 fa[2][FM], fb[2][FN];
  // LDS read r of sub-step s of step kt into fragment buffer buf: r < FM reads A block r;
  // then B (two transposing reads per block for [K,N], one ds_read_b128 for [N,K]).
  constexpr int RD = FM + (KN ? 2 : 1) * FN;
  auto read_one = [&](auto slotc, int s, int buf, auto rc) {
    constexpr int r = decltype(rc)::value, slot = decltype(slotc)::value;
    const unsigned char* sa = smem + slot * S::A_BYTES;
    const unsigned char* sb = smem + slot * S::B_BYTES;  // fb_off includes the B region's start
    if constexpr (r < FM) {
      fa[buf][r] = *(const u32x4*)(sa + fa_off[s] + r * 16 * S::ROW);
    } else if constexpr (KN) {
      constexpr int j = (r - FM) >> 1, half = (r - FM) & 1;
      const unsigned char* q = sb + fb_off[j] + (32 * s + 4 * half) * S::B_PITCH;
      const u32x2 v = __builtin_bit_cast(
          u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)q));
      if constexpr (half == 0) {
        fb[buf][j].x = v.x;
        fb[buf][j].y = v.y;
      } else {
        fb[buf][j].z = v.x;
        fb[buf][j].w = v.y;
      }
    } else {
      constexpr int j = r - FM;
      fb[buf][j] = *(const u32x4*)(sb + fb_off[s] + j * 16 * S::ROW);
    }
  };
  // One 32-k sub-step of MFMAs on fragment buffer BUF; MFMA slot x also issues read
  // r * X / RD == x of sub-step RS of ring slot RSLOT into the other buffer and, for
  // DMA mode 1 (full step) or 2 (the step holding K's end), DMA piece d * X / DMA == x of
  // step dkt into ring slot DSLOT.
  constexpr int X = FM * FN;
  auto substep = [&](auto bufc, auto rslotc, int rs, auto dmac, int dkt, auto dslotc) {
    constexpr int buf = decltype(bufc)::value;
    constexpr int dma = decltype(dmac)::value;
    static_for<X>([&](auto xc) {
      constexpr int x = decltype(xc)::value;
      constexpr int i = x / FN, j = x % FN;
      acc[i][j] = Mfma<T>::mma(fb[buf][j], fa[buf][i], acc[i][j]);
      static_for<RD>([&](auto rc) {
        if constexpr (decltype(rc)::value * X / RD == x) read_one(rslotc, rs, buf ^ 1, rc);
      });
      if constexpr (dma != 0) {
        static_for<S::DMA>([&](auto dc) {
          if constexpr (decltype(dc)::value * X / S::DMA == x)
            dma_piece(dkt, dslotc, dc, std::integral_constant<bool, dma == 2>{});
        });
      }
      __builtin_amdgcn_sched_barrier(0);  // keep the slots in this order
    });
  };
  using B0 = std::integral_constant<int, 0>;
  using B1 = std::integral_constant<int, 1>;
  // K step kt from ring slot SLOT: the second half's fragments are read during the
  // first sub-step; one barrier certifies that every read of the slot is done and
  // that step kt+1 (the other slot) has landed; the second sub-step reads step
  // kt+1's first fragments and loads step kt+2 into this slot (DMA mode as above).
  auto step = [&](int kt, auto slotc, auto dmac) {
    using Other = std::integral_constant<int, 1 - decltype(slotc)::value>;
    substep(B0{}, slotc, 1, B0{}, 0, slotc);
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" : : : "memory");
    substep(B1{}, Other{}, 0, dmac, kt + 2, slotc);
  };

  const int nk = (K + S::BK - 1) / S::BK;
  if (nk > 0) {
    using Mode = std::integral_constant<int, KCHECK ? 2 : 1>;  // checked or whole-step loads
    using Check = std::integral_constant<bool, KCHECK>;
    static_for<S::DMA>([&](auto dc) { dma_piece(0, B0{}, dc, Check{}); });
    static_for<S::DMA>([&](auto dc) { dma_piece(1, B1{}, dc, Check{}); });  // zeros if nk == 1
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" : : "n"(S::DMA) : "memory");  // step 0 landed
    static_for<RD>([&](auto rc) { read_one(B0{}, 0, 0, rc); });
    // pairs of steps, ring slots 0 and 1 (two copies of the step's code: the slot offsets
    // are immediates)
    for (int kt = 0; kt < nk; kt += 2) {
      step(kt, B0{}, Mode{});
      if (kt + 1 < nk) step(kt + 1, B1{}, Mode{});
    }
    asm volatile("s_waitcnt vmcnt(0)" : : : "memory");  // no LDS DMA may outlive the workgroup
  }

  // ---- epilogue: acc[i][j][e] = C[m = 16i + r16][n = 16j + 4G + e] of the wave's block.
  // For a pair of blocks (j, j+1), one v_permlane16_swap per dword trades G = 1's columns
  // of block j for G = 0's of block j+1 (and G = 3's of j for G = 2's of j+1): lane (r16, G)
  // then holds columns 16j' + 8(G/2) .. +7 of block j' = j + G%2. ----
  if constexpr (SPLITK) {
    // fp32 partial sums: acc[i][j] holds C[16i + r16][16j + 4G .. +3] of the wave's block
    // (N % 4 == 0, so the four columns are all in or all out)
    const int batch = (int)gridDim.z / p.splits;
    float* part = p.partials + ((int64_t)ks * batch + bz) * M * N;
    const int mw = m0 + wm * S::WTM, nw = n0 + wn * S::WTN;
    static_for<FM * FN>([&](auto xc) {
      constexpr int x = decltype(xc)::value;
      const int m = mw + 16 * (x / FN) + r16, n = nw + 16 * (x % FN) + 4 * G;
      if (m < M && n < N) *(f32x4*)(part + (int64_t)m * N + n) = acc[x / FN][x % FN];
    });
    return;
  }
  T* Cb = (T*)p.C + bz * p.stride_c;
  const uint16_t* bias = (const uint16_t*)p.bias;
  // store width C's rows allow (every batch entry's): 16 bytes, 8 bytes, or one element
  const int64_t cpitch = p.ldc | (gridDim.z > 1 ? p.stride_c : 0);
  const bool st16 = (cpitch & 7) == 0, st8 = (cpitch & 3) == 0;
  const int mw = m0 + wm * S::WTM, nw = n0 + wn * S::WTN;
  // The tile's bias values (BN per column, or BM per row) go to LDS first -- one load per
  // thread, after every wave's last fragment reads -- so that the epilogue's adds wait on
  // no global load queued behind its own stores.  Per column: four values per thread, one
  // 8-byte load when all four exist and the bias is 8-byte aligned, else one 2-byte load
  // each (a descriptor of 2N bytes returns zeros past N); per row: one value per thread.
  uint16_t* sbias = (uint16_t*)smem;
  if constexpr (BIAS != 0) {
    __syncthreads();
    const int tid = threadIdx.x;
    if constexpr (BIAS == 1) {
      if (tid < BN / 4) {
        const int n = n0 + 4 * tid;
        const __amdgpu_buffer_rsrc_t br = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(bias), 0, 2 * N, kBufWord3);
        u32x2 bb;
        if (n + 4 <= N && p.bias_vec) {
          bb = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(br, (uint32_t)(2 * n), 0, 0));
        } else {
          uint32_t h[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) h[e] = buf_load2(br, (uint32_t)(2 * (n + e)));
          bb = u32x2{h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
        }
        *(u32x2*)(sbias + 4 * tid) = bb;
      }
    } else {
      if (tid < BM) sbias[tid] = m0 + tid < M ? bias[m0 + tid] : (uint16_t)0;
    }
    __syncthreads();
  }
  auto bias_add = [&](int i, int j, f32x4 v) {
    if constexpr (BIAS == 2) {
      const float b = from_bits<T>(sbias[wm * S::WTM + 16 * i + r16]);
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] += b;
    } else if constexpr (BIAS == 1) {
      const u32x2 bb = *(const u32x2*)(sbias + wn * S::WTN + 16 * j + 4 * G);
      v[0] += from_bits<T>((uint16_t)(bb.x & 0xFFFF));
      v[1] += from_bits<T>((uint16_t)(bb.x >> 16));
      v[2] += from_bits<T>((uint16_t)(bb.y & 0xFFFF));
      v[3] += from_bits<T>((uint16_t)(bb.y >> 16));
    }
    return v;
  };
  static_for<FM>([&](auto ic) {
    constexpr int i = decltype(ic)::value;
    const int m = mw + 16 * i + r16;
    static_for<(FN + 1) / 2>([&](auto qc) {
      constexpr int j = 2 * decltype(qc)::value;
      const f32x4 v0 = bias_add(i, j, acc[i][j]);
      uint32_t P0[2] = {pack2<T>(v0[0], v0[1]), pack2<T>(v0[2], v0[3])};
      if constexpr (j + 1 < FN) {
        const f32x4 v1 = bias_add(i, j + 1, acc[i][j + 1]);
        uint32_t P1[2] = {pack2<T>(v1[0], v1[1]), pack2<T>(v1[2], v1[3])};
#pragma unroll
        for (int w = 0; w < 2; ++w) {
          const auto sw = __builtin_amdgcn_permlane16_swap(P0[w], P1[w], false, false);
          P0[w] = sw[0];
          P1[w] = sw[1];
        }
        const int n = nw + 16 * (j + (G & 1)) + 8 * (G >> 1);
        if (m < M && n < N) {
          T* dst = Cb + (int64_t)m * p.ldc + n;
          const u32x4 v = {P0[0], P0[1], P1[0], P1[1]};
          if (n + 8 <= N && st16) {
            *(u32x4*)dst = v;
          } else if (n + 8 <= N && st8) {  // 8-byte aligned rows
            *(u32x2*)dst = u32x2{v.x, v.y};
            *(u32x2*)(dst + 4) = u32x2{v.z, v.w};
          } else {
#pragma unroll
            for (int e = 0; e < 8; ++e)
              if (n + e < N) ((uint16_t*)dst)[e] = (uint16_t)(v[e >> 1] >> (16 * (e & 1)));
          }
        }
      } else {  // odd last block: four columns per lane
        const int n = nw + 16 * j + 4 * G;
        if (m < M && n < N) {
          T* dst = Cb + (int64_t)m * p.ldc + n;
          const u32x2 v = {P0[0], P0[1]};
          if (n + 4 <= N && st8) {
            *(u32x2*)dst = v;
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (n + e < N) ((uint16_t*)dst)[e] = (uint16_t)(v[e >> 1] >> (16 * (e & 1)));
          }
        }
      }
    });
  });
}

// Launches gemm_tile16_kernel (WM x WN waves, MINB workgroups per CU) with the
// bias mode and the K split the arguments ask for.
template <typename T, bool KN, int BM, int BN, int WM, int WN, int MINB, bool KCHECK>
hipError_t launch_tile16_k(const GemmParams& p, dim3 grid, hipStream_t s) {
  const dim3 block(64 * WM * WN);
  if constexpr (BM >= 128) {
    if (p.splits > 1)  // fp32 partials; the bias comes with the reduction
      return launch_kernel((gemm_tile16_kernel<T, KN, BM, BN, WM, WN, 0, MINB, true, KCHECK>), grid, block, 0, s, p);
  }
  if (p.bias == nullptr)
    return launch_kernel((gemm_tile16_kernel<T, KN, BM, BN, WM, WN, 0, MINB, false, KCHECK>), grid, block, 0, s, p);
  if (p.bias_row)
    return launch_kernel((gemm_tile16_kernel<T, KN, BM, BN, WM, WN, 2, MINB, false, KCHECK>), grid, block, 0, s, p);
  return launch_kernel((gemm_tile16_kernel<T, KN, BM, BN, WM, WN, 1, MINB, false, KCHECK>), grid, block, 0, s, p);
}

}  // namespace cmpext3
