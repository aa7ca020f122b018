// Device helpers shared by the gfx950 GEMM kernels: operand vector types,
// MFMA wrappers, buffer-resource loads with hardware zero-fill, the LDS
// swizzle, the 8x8 16-bit register transpose and the XCD-aware tile order.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "gemm_params.h"

namespace cmpext3 {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

// Offset that is always outside a buffer resource whose num_records is
// kBufRecords: a buffer load with it returns zeros and touches no memory.
constexpr uint32_t kBufRecords = 0x7FFFFFFFu;
constexpr uint32_t kBufOOB = 0x80000000u;

// gfx9 buffer descriptor word 3 (32-bit untyped access).
constexpr int kBufWord3 = 0x00020000;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)kBufRecords, kBufWord3);
}

// LDS DMA of 16 bytes per lane: global (rsrc + voff) -> LDS (lds_addr +
// 16 * lane), where lds_addr is wave-uniform and goes through M0.  Issued as
// inline asm so that the compiler does not guard every later LDS read with a
// wait for it: the kernels place their own "s_waitcnt vmcnt" fences (the
// "memory" clobber keeps LDS accesses from moving across the issue point).
typedef int i32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ i32x4 make_rsrc_sgpr(const void* base) {
  const uint64_t a = (uint64_t)base;
  i32x4 r;
  r[0] = (int)(uint32_t)a;
  r[1] = (int)((a >> 32) & 0xFFFF);
  r[2] = (int)kBufRecords;
  r[3] = kBufWord3;
  return r;
}
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma_load16(i32x4 rsrc, uint32_t voff, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %2\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
               :
               : "v"(voff), "s"(rsrc), "s"(lds_addr)
               : "memory", "m0");
}
// LDS DMA of 16 bytes per lane from global (rsrc + soff + voff) to LDS
// (lds_base + DST + 16 * lane): M0 = lds_base + DST (the addition is left to
// the compiler, which knows it sets SCC; then the one wait state an M0 write
// needs before an LDS DMA reads it); soff is an SGPR byte offset that advances
// along K without rebuilding the descriptor (it is part of the range check,
// like voff).
template <uint32_t DST>
__device__ __forceinline__ void dma_load16_m0(i32x4 rsrc, uint32_t voff, uint32_t soff, uint32_t lds_base,
                                              std::integral_constant<uint32_t, DST> = {}) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, %3 offen lds"
               :
               : "v"(voff), "s"(rsrc), "s"(lds_base + DST), "s"(soff)
               : "memory", "m0");
}
// Same with the non-temporal cache policy (nt): for operands that are read exactly
// once, so that their lines do not displace reusable data in L2 (the skinny kernels'
// B or W stream; 16 x 8192 x 8192 fp16 on MI355X: 27.4 -> 26.1 us per call).
__device__ __forceinline__ void dma_load16_stream(i32x4 rsrc, uint32_t voff, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %2\n\tbuffer_load_dwordx4 %0, %1, 0 offen nt lds"
               :
               : "v"(voff), "s"(rsrc), "s"(lds_addr)
               : "memory", "m0");
}
// Same with 4 bytes per lane (LDS destination lds_addr + 4 * lane): any
// 4-byte-aligned source, e.g. fp32 rows of odd length.
__device__ __forceinline__ void dma_load4(i32x4 rsrc, uint32_t voff, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %2\n\tbuffer_load_dword %0, %1, 0 offen lds"
               :
               : "v"(voff), "s"(rsrc), "s"(lds_addr)
               : "memory", "m0");
}
#pragma clang diagnostic pop
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(size_t)(__attribute__((address_space(3))) const void*)p;
}

__device__ __forceinline__ u32x4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
__device__ __forceinline__ uint32_t buf_load4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}
__device__ __forceinline__ uint16_t buf_load2(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(uint16_t, __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0));
}
// Cache policy of buffer loads and stores that are coherent across the whole
// device (sc1, the policy the compiler gives relaxed agent-scope atomic loads and
// stores on gfx950): a store reaches the memory side instead of staying in the
// issuing XCD's L2, and a load does not hit a stale line there, so no L2
// write-back or invalidate is needed.  Workgroups that hand partial results to one
// another use them: the writer waits for its stores to complete (s_waitcnt
// vmcnt(0)) before it bumps an agent-scope counter, and the reader loads only
// after that counter has told it the others are done.  `off` is a byte offset
// from `base` (below 2^31).
constexpr int kCoherent = 16;
__device__ __forceinline__ void store16_coherent(float* base, uint32_t off, f32x4 v) {
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(base, 0, (int)kBufRecords, kBufWord3);
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, off, 0, kCoherent);
}
__device__ __forceinline__ f32x4 load16_coherent(const float* base, uint32_t off) {
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), 0, (int)kBufRecords, kBufWord3);
  return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kCoherent));
}

// Vector store of 4 bytes; an offset past num_records (kBufOOB) is dropped by
// the hardware, which is how edge elements are masked without branches.
__device__ __forceinline__ void buf_store4(__amdgpu_buffer_rsrc_t r, uint32_t off, float v) {
  __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), r, off, 0, 0);
}
// Same with 16 bytes (off a multiple of 16).
__device__ __forceinline__ void buf_store16(__amdgpu_buffer_rsrc_t r, uint32_t off, f32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, off, 0, 0);
}

// ---------------------------------------------------------------------------
// MFMA wrappers.  The products are issued "swapped": the first MFMA operand
// carries B (its rows are output columns n), the second carries A (its
// columns are output rows m).  The 16x16 result block D[n][m] = C[m][n] then
// lands with lane l holding C[m = l%16][n = 4*(l/16) + i], i = 0..3: four
// consecutive columns of one row, which is the layout the epilogue stores.
// ---------------------------------------------------------------------------
template <typename T> struct Mfma;

template <> struct Mfma<_Float16> {
  static __device__ __forceinline__ f32x4 mma(u32x4 b, u32x4 a, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, b),
                                                  __builtin_bit_cast(f16x8, a), c, 0, 0, 0);
  }
};
template <> struct Mfma<__bf16> {
  static __device__ __forceinline__ f32x4 mma(u32x4 b, u32x4 a, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, b),
                                                   __builtin_bit_cast(bf16x8, a), c, 0, 0, 0);
  }
};

// 32x32x16 products, same operand convention: lane l supplies row (first
// operand) or column (second operand) l%32 and eight k values of group l/32;
// result register r of lane l is C[m = l%32][n = 8*(r/4) + 4*(l/32) + r%4].
template <typename T> struct Mfma32;
template <> struct Mfma32<_Float16> {
  static __device__ __forceinline__ f32x16 mma(u32x4 b, u32x4 a, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, b),
                                                  __builtin_bit_cast(f16x8, a), c, 0, 0, 0);
  }
};
template <> struct Mfma32<__bf16> {
  static __device__ __forceinline__ f32x16 mma(u32x4 b, u32x4 a, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, b),
                                                   __builtin_bit_cast(bf16x8, a), c, 0, 0, 0);
  }
};

__device__ __forceinline__ f32x4 mma_f32(float b, float a, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(b, a, c, 0, 0, 0);
}

// fp32 -> storage type, round to nearest even (hardware conversions).
template <typename T> __device__ __forceinline__ uint16_t to_bits(float x);
template <> __device__ __forceinline__ uint16_t to_bits<_Float16>(float x) {
  return __builtin_bit_cast(uint16_t, (_Float16)x);
}
template <> __device__ __forceinline__ uint16_t to_bits<__bf16>(float x) {
  return __builtin_bit_cast(uint16_t, (__bf16)x);
}
template <typename T> __device__ __forceinline__ float from_bits(uint16_t b);
template <> __device__ __forceinline__ float from_bits<_Float16>(uint16_t b) {
  return (float)__builtin_bit_cast(_Float16, b);
}
template <> __device__ __forceinline__ float from_bits<__bf16>(uint16_t b) {
  return __uint_as_float(((uint32_t)b) << 16);
}
template <typename T> __device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  return (uint32_t)to_bits<T>(lo) | ((uint32_t)to_bits<T>(hi) << 16);
}

// ---------------------------------------------------------------------------
// 16-bit lane packing.  perm(hi_src, lo_src, sel): byte i of the result is
// byte sel[i] of the 8-byte value {hi_src:lo_src}.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t pack_lo16(uint32_t x, uint32_t y) {  // {x.lo, y.lo}
  return __builtin_amdgcn_perm(y, x, 0x05040100u);
}
__device__ __forceinline__ uint32_t pack_hi16(uint32_t x, uint32_t y) {  // {x.hi, y.hi}
  return __builtin_amdgcn_perm(y, x, 0x07060302u);
}

// Transpose an 8x8 block of 16-bit values held as r[row] = 8 elements of one
// row (element 2j in the low half of dword j).  On return c[col] holds the 8
// elements of column `col`, row 0 in the low half of dword 0.
__device__ __forceinline__ void transpose8x8_b16(const u32x4 r[8], u32x4 c[8]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    // columns 2j (low halves) and 2j+1 (high halves) of dword j of each row
    u32x4 lo, hi;
    lo.x = pack_lo16(r[0][j], r[1][j]);
    lo.y = pack_lo16(r[2][j], r[3][j]);
    lo.z = pack_lo16(r[4][j], r[5][j]);
    lo.w = pack_lo16(r[6][j], r[7][j]);
    hi.x = pack_hi16(r[0][j], r[1][j]);
    hi.y = pack_hi16(r[2][j], r[3][j]);
    hi.z = pack_hi16(r[4][j], r[5][j]);
    hi.w = pack_hi16(r[6][j], r[7][j]);
    c[2 * j] = lo;
    c[2 * j + 1] = hi;
  }
}

// ---------------------------------------------------------------------------
// LDS tile layout for 16-bit operands: rows of 64 k-values (128 bytes, eight
// 16-byte chunks).  Rows are stored in pairs of 256 bytes (all 64 banks); the
// 16 chunks of a pair are permuted so that
//   * a 16-lane phase reading 16 consecutive rows at one chunk (an MFMA
//     fragment read) hits 16 distinct 4-bank groups, and
//   * a 16-lane phase writing chunks 0..7 of two rows, or chunk c of rows
//     {n, n+8} for eight (c, n) pairs (the transposed B store), does too.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t lds_off128(int row, int chunk) {
  const int p = row >> 1;
  const int bg = ((((row & 1) ^ ((p >> 2) & 1))) << 3) | ((chunk ^ p) & 7);
  return (uint32_t)(p * 256 + bg * 16);
}

// Row and chunk (relative to the tile's first row) of the 16-byte piece that
// lane `lane` of 1 KB LDS-DMA load `slot` must fetch so that LDS ends up in
// the lds_off128() layout (the inverse of lds_off128 at slot*1024 + 16*lane).
__device__ __forceinline__ void dma128_geom(int slot, int lane, int& row, int& chunk) {
  const int pp = 4 * slot + (lane >> 4);
  const int bg = lane & 15;
  row = 2 * pp + (((bg >> 3) ^ (pp >> 2)) & 1);
  chunk = (bg & 7) ^ (pp & 7);
}

// [k][n] layout of an N-contiguous B tile: rows of `pitch` bytes (a multiple
// of 256), 64-byte segments XORed with k%4 and their 32-byte halves with
// (k/8)%2.  A transposing fragment read (lanes of group G at rows 8G + 0..3,
// 8 bytes each) then covers all 64 banks once per 32 lanes; without the half
// swap, groups G and G+1 hit the same 32 banks (measured: 8.5M bank-conflict
// cycles per 4096^3 launch, now 0).
__device__ __forceinline__ uint32_t kn_off(int k, int pitch, int byte_col) {
  return (uint32_t)(k * pitch + (((byte_col >> 6) ^ (k & 3)) << 6) + ((byte_col & 63) ^ (((k >> 3) & 1) << 5)));
}
// Lane `lane` of 1 KB LDS-DMA load `slot` fetches row k, columns n..n+7 (the
// inverse of kn_off at byte slot*1024 + 16*lane).
__device__ __forceinline__ void dma_kn_geom(int slot, int lane, int pitch, int& k, int& n) {
  const int pos = slot * 1024 + 16 * lane;
  k = pos / pitch;
  const int within = pos - k * pitch;
  const int seg = (within >> 6) ^ (k & 3);
  n = (seg * 64 + ((within & 63) ^ (((k >> 3) & 1) << 5))) >> 1;
}

// The same for rows of 128 bytes (64 columns): 32-byte slots XORed with (k/2)%2 +
// 2((k/8)%2), so that the rows k..k+3 (4 | k) of a transposing read by 16 lanes and the
// rows k+8..k+11 of the next 16 lanes fill the 64 banks once.
__device__ __forceinline__ int kn128_swz(int k) { return ((k >> 1) & 1) | (((k >> 3) & 1) << 1); }
__device__ __forceinline__ uint32_t kn128_off(int k, int byte_col) {
  return (uint32_t)(k * 128 + (((byte_col >> 5) ^ kn128_swz(k)) << 5) + (byte_col & 31));
}
__device__ __forceinline__ void dma_kn128_geom(int slot, int lane, int& k, int& n) {
  const int pos = slot * 1024 + 16 * lane;
  k = pos >> 7;
  const int within = pos & 127;
  n = ((((within >> 5) ^ kn128_swz(k)) << 5) + (within & 31)) >> 1;
}

// ---------------------------------------------------------------------------
// Tile order.  The dispatcher hands workgroup w (x fastest, then z) to XCD
// w % 8; consecutive logical tiles -- batch entry by batch entry -- are given to
// the same XCD so that its L2 sees a compact block of A rows and B columns (and
// whole batch entries of a batched product), and inside an entry tiles are
// grouped `group_m` rows at a time (column-major within the group).
// ---------------------------------------------------------------------------
__device__ __forceinline__ void tile_coords(int x, int z, int nz, int tiles_m, int tiles_n, int group_m,
                                            int& tm, int& tn, int& bz) {
  const int tiles = tiles_m * tiles_n;
  const int64_t total = (int64_t)tiles * nz;
  const int64_t wg = x + (int64_t)tiles * z;
  const int xcd = (int)(wg & 7);
  const int64_t base = total >> 3, rem = total & 7;
  const int64_t s = xcd * base + (xcd < rem ? xcd : rem) + (wg >> 3);
  bz = (int)(s / tiles);
  const int t = (int)(s - (int64_t)bz * tiles);
  const int per_group = group_m * tiles_n;
  const int g = t / per_group;
  const int first_m = g * group_m;
  const int gsz = (tiles_m - first_m) < group_m ? (tiles_m - first_m) : group_m;
  const int r = t - g * per_group;
  tm = first_m + r % gsz;
  tn = r / gsz;
}

// ---------------------------------------------------------------------------
// Host side: launches `kernel` on `s` and returns the status of this launch
// alone.  (hipGetLastError after a launch would also report, and clear, an
// earlier failure of unrelated work on the calling thread.)
// ---------------------------------------------------------------------------
template <typename T>
struct Same {
  using type = T;
};
template <typename... P>
inline hipError_t launch_kernel(void (*kernel)(P...), dim3 grid, dim3 block, size_t shmem, hipStream_t s,
                                typename Same<P>::type... args) {
  void* argv[] = {(void*)&args..., nullptr};
  return hipLaunchKernel((const void*)kernel, grid, block, argv, shmem, s);
}

}  // namespace cmpext3
