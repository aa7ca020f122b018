// Skinny-M f16/bf16 GEMM with split K (M <= 64, B is [K,N]), for callers that
// provide a workspace: C = A * B (+ bias).
//
// HBM reads of 64-byte row segments (the 32-column strips of the narrow
// skinny kernel) top out near 4 TB/s on MI355X; 256-byte segments reach
// ~5.6 TB/s.  So here a workgroup owns a 128-column strip, and the K range is
// split S ways across workgroups so that there are still ~256 of them
// (16 x 8192 x 8192: 64 strips x 4 splits).  Each workgroup
//   * streams its B block (k-rows of 256 bytes) and the matching A columns
//     global -> LDS with LDS-DMA through a ring of NS stages of 64 k-rows;
//   * gives each of its 4 waves 32 of the 128 columns, so waves never need
//     to combine results; B fragments come from ds_read_b64_tr_b16 on the
//     [k][n] tile, A fragments from ds_read_b128 (v_mfma_f32_16x16x32, the M
//     rows in the MFMA's 16-wide dimension);
//   * with S == 1 writes C directly; otherwise writes its fp32 partial block
//     to the workspace and counts itself in on its strip's counter (`sem`);
//     the last of the strip's S workgroups to arrive sums the S partials in
//     split order, adds the bias, rounds to the output type, writes C and
//     resets the counter.  Without counters (sem == nullptr)
//     skinny_reduce_kernel does that sum in a second launch, with the same
//     arithmetic (bit-identical results).
#pragma once

#include <type_traits>

#include "device_common.h"

namespace cmpext3 {

constexpr int kWideStrip = 128;  // columns per workgroup
constexpr int kWideKS = 64;      // k rows per ring stage

template <int MB>
struct WideShape {
  static constexpr int B_BYTES = kWideKS * kWideStrip * 2;  // 16 KB, rows of 256 bytes
  static constexpr int A_BYTES = MB * 16 * 128;             // rows of 64 k = 128 bytes
  static constexpr int STAGE = B_BYTES + A_BYTES;
  // Four stages (64-96 KiB): measured on MI355X against the deepest ring that fits
  // (8, 8, 7, 6 stages for MB = 1..4), 16/32/48/64 x 8192 x 8192 with 4 splits ran
  // 27.5/28.8/30.1/31.5 us against 28.2/29.6/30.9/31.9.
  static constexpr int NS = 4;
  static constexpr int B_DMA = B_BYTES / 4096;  // per wave
  static constexpr int A_DMA_WG = A_BYTES / 1024;  // per workgroup, dealt round-robin to waves
  static constexpr int A_HI = (A_DMA_WG + 3) / 4;  // A loads of waves < A_DMA_WG % 4 (or all)
  static constexpr int A_LO = A_DMA_WG / 4;
  static_assert(NS >= 4 && (NS - 2) * (B_DMA + A_HI) <= 63, "ring depth / vmcnt range");
};

// Byte offset in a B stage of row k, 16-column segment seg (0..7): the
// segments are XORed with (k%4) + 4*((k/8)%2), so a transposing read (rows
// k..k+3 and k+8..k+11 of one segment, 32 lanes) hits 8 distinct 32-byte
// bank slots.
__device__ __forceinline__ int wide_swz(int k) { return (k & 3) | (((k >> 3) & 1) << 2); }
__device__ __forceinline__ uint32_t wide_off(int k, int seg) {
  return (uint32_t)(k * 256 + ((seg ^ wide_swz(k)) << 5));
}

// NT: stream B with the non-temporal policy (B larger than the Infinity Cache would keep
// for the next call).
template <typename T, int MB, bool NT = false>
__global__ void __launch_bounds__(256) gemm_skinny_wide_kernel(const GemmParams p, float* ws, int splits,
                                                               int ksplit, unsigned int* sem) {
  using S = WideShape<MB>;
  constexpr int NS = S::NS;
  __shared__ __attribute__((aligned(1024))) unsigned char smem[NS * S::STAGE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int strip = blockIdx.x / splits;
  const int split = blockIdx.x - strip * splits;
  const int n0 = strip * kWideStrip;
  const int M = p.M, N = p.N;
  const int kbeg = split * ksplit;
  const int kend = min(p.K, kbeg + ksplit);
  const int64_t bz = blockIdx.z;
  const int64_t lda = p.lda, ldb = p.ldb;
  const T* Ab = (const T*)p.A + bz * p.stride_a + kbeg;
  const T* Bb = (const T*)p.B + bz * p.stride_b + (int64_t)kbeg * ldb + n0;
  const int klen = kend - kbeg;

  // ---- DMA sources (inverse of the LDS layouts), relative to the stage's k0 ----
  uint32_t b_off[S::B_DMA];
  int b_k[S::B_DMA];
#pragma unroll
  for (int i = 0; i < S::B_DMA; ++i) {
    const int row = 4 * (wave * S::B_DMA + i) + (lane >> 4);  // 4 rows of 256 bytes per load
    const int seg = ((lane & 15) >> 1) ^ wide_swz(row);
    const int col = seg * 16 + (lane & 1) * 8;
    b_off[i] = (n0 + col < N) ? (uint32_t)(row * ldb + col) * (uint32_t)sizeof(T) : kBufOOB;
    b_k[i] = row;
  }
  const int a_cnt = wave < (S::A_DMA_WG & 3) || (S::A_DMA_WG & 3) == 0 ? S::A_HI : S::A_LO;
  uint32_t a_off[S::A_HI];
  int a_k[S::A_HI];
#pragma unroll
  for (int j = 0; j < S::A_HI; ++j) {
    int row, chunk;
    dma128_geom(4 * j + wave, lane, row, chunk);
    a_off[j] = (row < M) ? (uint32_t)(row * lda + 8 * chunk) * (uint32_t)sizeof(T) : kBufOOB;
    a_k[j] = 8 * chunk;
  }
  auto load_stage = [&](int st) {
    const int k0 = st * kWideKS;
    const uint32_t dst = lds_addr(smem) + (uint32_t)((st % NS) * S::STAGE);
    const int krem = klen - k0;
    const i32x4 rb = make_rsrc_sgpr(Bb + (int64_t)k0 * ldb);
    const i32x4 ra = make_rsrc_sgpr(Ab + k0);
#pragma unroll
    for (int i = 0; i < S::B_DMA; ++i)
      if constexpr (NT)
        dma_load16_stream(rb, b_k[i] < krem ? b_off[i] : kBufOOB, dst + (wave * S::B_DMA + i) * 1024);
      else
        dma_load16(rb, b_k[i] < krem ? b_off[i] : kBufOOB, dst + (wave * S::B_DMA + i) * 1024);
#pragma unroll
    for (int j = 0; j < S::A_HI; ++j)
      if (j < a_cnt)
        dma_load16(ra, a_k[j] < krem ? a_off[j] : kBufOOB, dst + S::B_BYTES + (4 * j + wave) * 1024);
  };
  // Wait until at most NS-2 younger stages' DMA are in flight, then barrier.
  auto certify = [&]() {
    if (a_cnt == S::A_HI)
      asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" : : "n"((NS - 2) * (S::B_DMA + S::A_HI)) : "memory");
    else
      asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" : : "n"((NS - 2) * (S::B_DMA + S::A_LO)) : "memory");
  };

  // ---- fragments: lane (c = l%16, g = l/16); wave owns columns 32w .. 32w+31 ----
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
    for (int kb = 0; kb < kWideKS; kb += 32) {
      u32x4 af[MB];
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
        af[mb] = *(const u32x4*)(stage + S::B_BYTES + lds_off128(16 * mb + c, kb / 8 + g));
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int seg = 2 * wave + h;
        u32x4 bf;
#pragma unroll
        for (int r = 0; r < 2; ++r) {
          const int k = kb + 8 * g + 4 * r + (c >> 2);
          const unsigned char* q = stage + wide_off(k, seg) + 8 * (c & 3);
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

  const int nst = (klen + kWideKS - 1) / kWideKS;
#pragma unroll
  for (int t = 0; t < NS - 1; ++t) load_stage(t);
  certify();  // stage 0
  for (int st = 0; st < nst; ++st) {
    load_stage(st + NS - 1);
    compute_stage(st);
    certify();  // stage st+1
  }
  asm volatile("s_waitcnt vmcnt(0)" : : : "memory");  // no LDS DMA may outlive the workgroup

  // acc[h][mb][r] = C[16*mb + c][n0 + 32*wave + 16*h + 4*g + r]
  const uint16_t* bias = (const uint16_t*)p.bias;
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int m = 16 * mb + c;
    if (m >= M) continue;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int n = n0 + 32 * wave + 16 * h + 4 * g;
      if (n >= N) continue;  // N % 8 == 0: the four columns are all in or all out
      if (splits == 1) {
        uint16_t* crow = (uint16_t*)((T*)p.C + bz * p.stride_c + (int64_t)m * p.ldc);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float x = acc[h][mb][r];
          if (bias) x += from_bits<T>(bias[p.bias_row ? m : n + r]);
          crow[n + r] = to_bits<T>(x);
        }
      } else {
        float* blk = ws + ((int64_t)split * gridDim.z + bz) * M * N;  // this (split, batch entry) block
        if (sem != nullptr)
          store16_coherent(blk, (uint32_t)(m * N + n) * 4u, acc[h][mb]);
        else
          *(f32x4*)(blk + m * N + n) = acc[h][mb];
      }
    }
  }
  if (splits == 1 || sem == nullptr) return;

  // ---- the strip's split reduction, by the last of its workgroups to arrive ----
  // The partials went out as GPU-coherent stores (store16_coherent); every wave waits
  // for them to complete, then one thread counts the workgroup in with an agent-scope
  // atomic.  The last to arrive reads the others' partials with GPU-coherent loads.
  // (Agent-scope release/acquire fences would instead write back and invalidate the
  // XCD's whole L2 per workgroup: measured on MI355X, 16 x 8192 x 8192 took 34.7 us
  // with one such fence pair per workgroup against ~28 us for two launches.)
  __shared__ int last;
  unsigned int* count = sem + bz * (gridDim.x / splits) + strip;
  asm volatile("s_waitcnt vmcnt(0)" : : : "memory");
  __syncthreads();
  if (tid == 0)
    last = __hip_atomic_fetch_add(count, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
           (unsigned int)(splits - 1);
  __syncthreads();
  if (!last) return;
  const int cols = min(kWideStrip, N - n0);  // a multiple of 8
  for (int idx = tid; idx < M * (kWideStrip / 4); idx += 256) {
    const int m = idx / (kWideStrip / 4), n = n0 + 4 * (idx % (kWideStrip / 4));
    if (n - n0 >= cols) continue;
    // sum in split order from zero, then the bias, then one rounding: the arithmetic of
    // skinny_reduce_kernel
    f32x4 acc4 = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int s0 = 0; s0 < splits; s0 += 8) {  // up to 8 loads in flight, then the adds in order
      f32x4 part[8];
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (s0 + j < splits)
          part[j] = load16_coherent(ws + ((s0 + j) * gridDim.z + bz) * M * N, (uint32_t)(m * N + n) * 4u);
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (s0 + j < splits) acc4 += part[j];
    }
    uint16_t* crow = (uint16_t*)((T*)p.C + bz * p.stride_c + (int64_t)m * p.ldc) + n;
    uint16_t h[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float x = acc4[r];
      if (bias) x += from_bits<T>(bias[p.bias_row ? m : n + r]);
      h[r] = to_bits<T>(x);
    }
    if (((uintptr_t)crow & 7) == 0) {
      *(u32x2*)crow = u32x2{(uint32_t)h[0] | ((uint32_t)h[1] << 16), (uint32_t)h[2] | ((uint32_t)h[3] << 16)};
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r) crow[r] = h[r];
    }
  }
  if (tid == 0) __hip_atomic_store(count, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // for the next kernel
}

// C = sum over the S partial blocks in the workspace (+ bias), rounded to T.
// Thread t of the grid-stride loop sums V consecutive columns (N % V == 0) of one row of
// the batch * M rows: chunk idx = row * (N / V) + column / V, so that a workgroup covers
// several rows when N is small (one row per workgroup left 240 of 256 threads idle at N =
// 128).  V / 4 16-byte loads per split, several splits in flight at once; the V results go
// out as V * sizeof(T)-byte stores (16-byte pieces) when `vec` says C's rows and batch
// entries keep those stores aligned, else element by element.  The splits are summed in
// order 0, 1, ..: the result does not depend on the launch geometry.
template <typename T, int V>
__global__ void __launch_bounds__(256) skinny_reduce_kernel(const GemmParams p, const float* ws, int splits,
                                                            int batch, int vec) {
  static_assert(V == 4 || V == 8, "4 or 8 columns per thread");
  const int M = p.M, N = p.N;
  const int64_t nv = N / V, total = (int64_t)batch * M * nv;
  const int64_t split_stride = (int64_t)batch * M * N;  // floats between one split's block and the next
  for (int64_t idx = blockIdx.x * 256ll + threadIdx.x; idx < total; idx += (int64_t)gridDim.x * 256) {
    const int64_t row = idx / nv;
    const int n = (int)(idx - row * nv) * V;
    const int64_t bz = row / M;
    const int m = (int)(row - bz * M);
    const float* w = ws + row * N + n;
    f32x4 s[V / 4];
#pragma unroll
    for (int v = 0; v < V / 4; ++v) s[v] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
    for (int sp = 0; sp < splits; ++sp) {
#pragma unroll
      for (int v = 0; v < V / 4; ++v) s[v] += *(const f32x4*)(w + sp * split_stride + 4 * v);
    }
    float x[V];
#pragma unroll
    for (int r = 0; r < V; ++r) x[r] = s[r / 4][r % 4];
    if constexpr (std::is_same<T, float>::value) {  // fp32 products (split-K fp32 tiles)
      const float* bias = (const float*)p.bias;
      if (bias) {
#pragma unroll
        for (int r = 0; r < V; ++r) x[r] += bias[p.bias_row ? m : n + r];
      }
      float* crow = (float*)p.C + bz * p.stride_c + (int64_t)m * p.ldc + n;
      if (vec) {
#pragma unroll
        for (int v = 0; v < V / 4; ++v)
          *(f32x4*)(crow + 4 * v) = f32x4{x[4 * v], x[4 * v + 1], x[4 * v + 2], x[4 * v + 3]};
      } else {
#pragma unroll
        for (int r = 0; r < V; ++r) crow[r] = x[r];
      }
    } else {
      const uint16_t* bias = (const uint16_t*)p.bias;
      if (bias) {
#pragma unroll
        for (int r = 0; r < V; ++r) x[r] += from_bits<T>(bias[p.bias_row ? m : n + r]);
      }
      uint16_t* crow = (uint16_t*)((T*)p.C + bz * p.stride_c + (int64_t)m * p.ldc + n);
      if (vec) {
        uint32_t q[V / 2];
#pragma unroll
        for (int v = 0; v < V / 2; ++v) q[v] = (uint32_t)to_bits<T>(x[2 * v]) | ((uint32_t)to_bits<T>(x[2 * v + 1]) << 16);
        if constexpr (V == 8)
          *(u32x4*)crow = u32x4{q[0], q[1], q[2], q[3]};
        else
          *(u32x2*)crow = u32x2{q[0], q[1]};
      } else {
#pragma unroll
        for (int r = 0; r < V; ++r) crow[r] = to_bits<T>(x[r]);
      }
    }
  }
}

}  // namespace cmpext3
