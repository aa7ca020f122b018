// Short-K f16/bf16 GEMM over many columns: C[b] = A * B[b] (+ bias per row),
// M <= 2048 and K <= 256, B as [K,N] -- the shape of a 1x1 convolution over NCHW
// activations (A = the weight, shared by every batch entry; B[b] = one image's
// [C_in][H*W]; C[b] = its [C_out][H*W]); counterpart of the reference's conv2d
// routed through its GEMM (csrc/main.cpp:402-424).
//
// Such a product moves ~3 bytes per 64 flops: it is bound by streaming B in and
// C out, and a tile kernel that holds one 64 x 256 tile per workgroup leaves
// each CU idle between its tiles' loads (measured 3.9 TB/s).  Here a persistent
// workgroup per CU walks the 128-column tiles t = blockIdx.x, + gridDim.x, ...
// (batch entry t / tiles_n) of its row block with
//   * tiles of MT = 64 WG rows by 128 columns (M > 128: up to 16 row blocks of 128 rows,
//     each with its own set of workgroups, the sets in step so that a B chunk comes from
//     HBM once and from L2 for the other blocks), WG = 1 or 2 groups of 4 waves,
//     group g computing rows 64 g .. 64 g + 63; each tile read as KC = 1 or 2 chunks of
//     128 k-rows (K <= 128 KC);
//   * A held in registers for the whole kernel (each wave its 64 rows x 128 KC as MFMA
//     fragments);
//   * B chunks ([128][128] = 32 KiB, rows of 256 bytes) streamed global -> LDS by
//     LDS-DMA through a ring of four slots, three chunks in flight;
//   * per chunk and wave (its rows x 32 columns; the 4 waves of a group split the
//     128 columns) 4 sub-steps of 32 k on 16x16x32 MFMAs, B fragments by
//     ds_read_b64_tr_b16 as in the tile kernel's [K,N] path;
//   * the tile's results staged in LDS (row-major, 16-byte chunks XOR-swizzled by
//     row; two buffers for MT = 64, one for MT = 128) and written during the next
//     tile's chunks, after their barriers: each
//     wave stores MT/waves whole rows of 256 bytes with non-temporal 16-byte stores
//     (full cache lines that go straight to HBM instead of waiting in L2 as dirty
//     lines; measured on MI355X for the 64 x 16384 x 128 x 64 convolution: 62.4
//     us against 84.5 us for the MFMA layout's 64-byte row pieces through L2, and
//     72.3 us for those pieces non-temporal), out-of-range lanes masked by the
//     descriptor, spread evenly over the tile's KC chunks, so that every chunk
//     issues the same number of vector-memory instructions and one
//     "s_waitcnt vmcnt" constant certifies the chunk about to be read.
// Requirements (checked by the selector): K, N, lda, ldb, ldc multiples of 8;
// A, B and C 16-byte aligned; one A for the whole batch (batch 1 or stride_a 0);
// 128 * ldb * 2 and 128 * ldc * 2 below 2^31.
#pragma once

#include <type_traits>

#include "device_common.h"
#include "tile16_kernel.h"

namespace cmpext3 {

constexpr int kStreamN = 128;     // columns per tile
constexpr int kStreamKC = 128;    // k rows per chunk (rows of a ring slot)
// Cache policy of the result stores: non-temporal (the nt bit of the buffer instruction).
constexpr int kStreamStorePolicy = 2;

// BIAS: 0 none, 2 one value per row of C (the convolution's per-channel bias).
// WG: groups of 4 waves, group g computing rows 64 g .. 64 g + 63 of the tile (MT = 64 WG
// rows, M <= MT); KC: chunks of 128 k per tile (K <= 128 KC).
// NT: B read with the non-temporal cache policy (for read-dominated products).
// BNK: B given as [N, K] (rows of K; e.g. an NHWC image: pixels x input channels), stored
// in a slot as [n][k] (rows of 256 bytes, 16-byte chunks XOR-swizzled by n % 16) and read
// with ds_read_b128; otherwise B is [K, N], stored [k][n] and read with transposing reads.
template <typename T, int BIAS, int WG, int KC, bool NT, bool BNK>
__global__ void __launch_bounds__(256 * WG, 1) gemm_stream_kernel(const GemmParams p, int total_tiles) {
  static_assert((WG == 1 || WG == 2) && (KC == 1 || KC == 2), "tile shapes");
  constexpr int RW = 64;                         // rows per wave
  constexpr int MT = RW * WG;                    // rows per tile
  constexpr int NW = 4 * WG;                     // waves
  constexpr int PITCH = kStreamN * 2;            // bytes per k row of a slot
  constexpr int SLOT = kStreamKC * PITCH;        // 32 KiB
  constexpr int P = SLOT / 1024 / NW;            // 1 KiB LDS-DMA loads per wave per chunk
  constexpr int FM = RW / 16, FN = 2, KSC = kStreamKC / 32, KS = KSC * KC;
  constexpr int Q = RW / 16;                     // 16-byte stores per wave per tile (MT/NW = RW/4 rows)
  constexpr int QC = Q / KC;                     // ... per chunk
  constexpr int STG = MT * 256;                  // one tile's results
  // Staging buffers: two for MT = 64 (a tile's results go to one while the other's are
  // stored); one for MT = 128, with a barrier before it is overwritten, so that the ring
  // keeps four slots (three chunks in flight) there too.
  constexpr int SB = MT == 64 ? 2 : 1;
  constexpr int SLOTS = 4;                       // ring depth (chunks)
  static_assert(Q % KC == 0, "stores spread evenly over the chunks");
  static_assert((SLOTS - 2) * (P + QC) <= 63, "vmcnt range");
  static_assert(SLOTS * SLOT + SB * STG <= 160 * 1024, "LDS");
  __shared__ __attribute__((aligned(1024))) unsigned char smem[SLOTS * SLOT + SB * STG];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = wave >> 2, wc = wave & 3;  // row group, column slice
  const int r16 = lane & 15, G = lane >> 4;
  const int N = p.N, K = p.K;
  const int tiles_n = p.tiles_n;
  // Row blocks of MT rows: gridDim.x / row_blocks workgroups per block, each walking the
  // column tiles of its block.  The launcher makes that count a multiple of 8, so workgroup
  // j of every block runs on the same XCD (workgroups go to the XCDs round robin) and, the
  // blocks walking their tiles in step, the later blocks find each B chunk in that L2.
  const int row_blocks = (p.M + MT - 1) / MT;
  const int step = gridDim.x / row_blocks;
  const int rblk = blockIdx.x / step, me = blockIdx.x - rblk * step;
  const int m_base = rblk * MT;
  const int M = min(p.M - m_base, MT);  // rows of this block
  const int ntiles = total_tiles > me ? (total_tiles - me + step - 1) / step : 0;
  const int nchunks = ntiles * KC;

  // ---- A fragments (rows RW grp + 16i + r16, k = 32s + 8G .. +7), zero past M and K ----
  u32x4 fa[FM][KS];
  {
    const __amdgpu_buffer_rsrc_t ra = make_rsrc((const T*)p.A + (int64_t)m_base * p.lda);
    static_for<FM * KS>([&](auto xc) {
      constexpr int x = decltype(xc)::value, i = x / KS, s = x % KS;
      const int m = RW * grp + 16 * i + r16, k = 32 * s + 8 * G;
      fa[i][s] = buf_load16(ra, (m < M && k < K) ? (uint32_t)(m * p.lda + k) * 2u : kBufOOB);
    });
  }
  float bias_m[FM] = {};
  if constexpr (BIAS == 2) {
    const __amdgpu_buffer_rsrc_t rb =
        __builtin_amdgcn_make_buffer_rsrc((T*)const_cast<void*>(p.bias) + m_base, 0, 2 * M, kBufWord3);
#pragma unroll
    for (int i = 0; i < FM; ++i) bias_m[i] = from_bits<T>(buf_load2(rb, (uint32_t)(2 * (RW * grp + 16 * i + r16))));
  }
  // Make these values definitions of an asm statement placed after a full wait: the
  // compiler counts only its own vector-memory instructions, so a wait it derived for
  // them inside the loop would also stall on the ring's loads.
  asm volatile("s_waitcnt vmcnt(0)" : : : "memory");
#pragma unroll
  for (int x = 0; x < FM * KS; ++x) asm volatile("" : "+v"(fa[x / KS][x % KS]));
#pragma unroll
  for (int i = 0; i < FM; ++i) asm volatile("" : "+v"(bias_m[i]));

  // ---- DMA: piece q of wave w fills bytes (w*P + q) KiB of a slot: k rows 4(wP+q) .. +3
  // of the chunk ([K, N]), or n rows 4(wP+q) .. +3 ([N, K]; lane l: row 4(wP+q) + l/16,
  // 16-byte chunk position l % 16, holding k = 8 ((l % 16) ^ (n % 16)) .. +7) ----
  // b_off[h][q]: the piece's offset in chunk h of a tile, or kBufOOB past K
  uint32_t b_off[KC][P];
  int b_n[P];
#pragma unroll
  for (int q = 0; q < P; ++q) {
    int k, n;
    if constexpr (BNK) {
      const int pos = (wave * P + q) * 1024 + 16 * lane;
      n = pos / PITCH;
      k = 8 * (((pos % PITCH) >> 4) ^ (n & 15));
    } else {
      dma_kn_geom(wave * P + q, lane, PITCH, k, n);
    }
#pragma unroll
    for (int h = 0; h < KC; ++h)
      b_off[h][q] = kStreamKC * h + k < K ? (uint32_t)(BNK ? n * p.ldb + k : k * p.ldb + n) * 2u : kBufOOB;
    b_n[q] = n;
  }
  const uint32_t lds_w = lds_addr(smem) + (uint32_t)(wave * P * 1024);
  // Chunk c = KC i + h (tile i, its k rows from 128 h; h known at compile time) of this
  // workgroup into ring slot c % SLOTS; chunks past the end load through an empty
  // descriptor (no memory read, zeros into LDS) so every iteration issues P loads.
  auto issue = [&](int c, auto hc) {
    constexpr int h = decltype(hc)::value;
    const bool live = c < nchunks;
    const int t = live ? me + (c / KC) * step : 0;
    const int bz = t / tiles_n, n0 = (t - bz * tiles_n) * kStreamN;
    i32x4 r = make_rsrc_sgpr((const T*)p.B + (int64_t)bz * p.stride_b +
                             (BNK ? (int64_t)n0 * p.ldb + kStreamKC * h : (int64_t)(kStreamKC * h) * p.ldb + n0));
    r[2] = live ? (int)kBufRecords : 0;
    const uint32_t base = lds_w + (uint32_t)((c % SLOTS) * SLOT);
    static_for<P>([&](auto qc) {
      constexpr int q = decltype(qc)::value;
      const uint32_t voff = n0 + b_n[q] < N ? b_off[h][q] : kBufOOB;
      if constexpr (NT)
        dma_load16_stream(r, voff, base + (uint32_t)(q * 1024));
      else
        dma_load16_m0(r, voff, 0u, base, std::integral_constant<uint32_t, (uint32_t)(q * 1024)>{});
    });
  };

  // ---- fragment addresses: [k][n] slot, transposing reads as in the tile kernel; [n][k]
  // slot, row n = 32 wc + 16 j + r16 (its chunk position added per sub-step) ----
  uint32_t fb_off[FN];
  const int kr = 8 * G + (r16 >> 2);
#pragma unroll
  for (int j = 0; j < FN; ++j)
    fb_off[j] = BNK ? (uint32_t)((32 * wc + 16 * j + r16) * PITCH)
                    : kn_off(kr, PITCH, (32 * wc + 16 * j + 4 * (r16 & 3)) * 2);

  // ---- results: after one permlane16 swap per dword, lane (r16, G) holds row RW grp + 16i + r16,
  // columns col .. col+7 of the tile; they go to staging buffer i % 2 as 16-byte chunk
  // col/8 of the row, at chunk position (col/8) ^ (row % 16) (conflict-free writes and
  // row reads) ----
  const int col = 32 * wc + 16 * (G & 1) + 8 * (G >> 1);
  unsigned char* const stg0 = smem + SLOTS * SLOT;
  // Part `part` of KC of this wave's stores of tile i: QC stores of 4 x 256-byte rows
  // (rows RW/4 wave + 4 QC part .. of the wave's RW/4 rows; an empty descriptor when there
  // is no tile i): always QC instructions.
  auto store = [&](int i, auto partc) {
    constexpr int part = decltype(partc)::value;
    const bool live = i >= 0 && i < ntiles;
    const int t = live ? me + i * step : 0;
    const int bz = t / tiles_n, n0 = (t - bz * tiles_n) * kStreamN;
    T* cb = (T*)p.C + (int64_t)bz * p.stride_c + (int64_t)m_base * p.ldc + n0;
    const __amdgpu_buffer_rsrc_t rc = __builtin_amdgcn_make_buffer_rsrc(cb, 0, live ? (int)kBufRecords : 0, kBufWord3);
    const unsigned char* stg = stg0 + (SB == 2 ? (i & 1) * STG : 0);
    const int ch = lane & 15;
    const bool col_ok = n0 + 8 * ch < N;
    u32x4 v[QC];
#pragma unroll
    for (int q = 0; q < QC; ++q) {
      const int row = (RW / 4) * wave + 4 * (QC * part + q) + (lane >> 4);
      v[q] = *(const u32x4*)(stg + row * 256 + ((ch ^ (row & 15)) << 4));
    }
#pragma unroll
    for (int q = 0; q < QC; ++q) {
      const int row = (RW / 4) * wave + 4 * (QC * part + q) + (lane >> 4);
      const uint32_t off = (col_ok && row < M) ? (uint32_t)(row * p.ldc + 8 * ch) * 2u : kBufOOB;
      __builtin_amdgcn_raw_buffer_store_b128(v[q], rc, off, 0, kStreamStorePolicy);
    }
  };

  static_for<SLOTS - 1>([&](auto cc) {
    constexpr int c = decltype(cc)::value;
    issue(c, std::integral_constant<int, c % KC>{});
  });
  for (int i = 0; i < ntiles; ++i) {
    f32x4 acc[FM][FN];
    static_for<FM * FN>([&](auto xc) {
      constexpr int x = decltype(xc)::value;
      acc[x / FN][x % FN] = f32x4{0.f, 0.f, 0.f, 0.f};
    });
    static_for<KC>([&](auto hc) {
      constexpr int h = decltype(hc)::value;
      const int c = i * KC + h;
      // Chunk c landed: after its loads (issued in iteration c - (SLOTS-1), or before the
      // loop) this wave issued the stores and loads of SLOTS-2 more iterations ((SLOTS-2) x
      // (P + QC) instructions; at least (SLOTS-2) x P in the first iterations, where the
      // loads of later chunks came before the loop), and vector-memory instructions
      // complete in issue order.
      if (c >= SLOTS - 2)
        asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" : : "n"((SLOTS - 2) * (P + QC)) : "memory");
      else
        asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" : : "n"((SLOTS - 2) * P) : "memory");
      // every wave is past chunk c-1's reads (its slot takes chunk c + SLOTS-1) and has
      // staged tile i-1's results
      store(i - 1, hc);
      issue(c + SLOTS - 1, std::integral_constant<int, (h + SLOTS - 1) % KC>{});

      const unsigned char* sb = smem + (c % SLOTS) * SLOT;
      static_for<KSC>([&](auto sc) {  // sub-steps of 32 k: B fragments, then their MFMAs
        constexpr int s = decltype(sc)::value;
        u32x4 fb[FN];
        if constexpr (BNK) {
          // k = 32 s + 8 G .. +7 of row n: chunk 4 s + G at position (4 s + G) ^ (n % 16),
          // n % 16 = r16 (16 distinct positions across the 16 rows: conflict free)
#pragma unroll
          for (int j = 0; j < FN; ++j)
            fb[j] = *(const u32x4*)(sb + fb_off[j] + (((4 * s + G) ^ r16) << 4));
        } else {
          static_for<FN * 2>([&](auto rc) {
            constexpr int r = decltype(rc)::value, j = r / 2, half = r % 2;
            typedef short s16x4 __attribute__((ext_vector_type(4)));
            const unsigned char* q = sb + fb_off[j] + (32 * s + 4 * half) * PITCH;
            const u32x2 v = __builtin_bit_cast(
                u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)q));
            if constexpr (half == 0) {
              fb[j].x = v.x;
              fb[j].y = v.y;
            } else {
              fb[j].z = v.x;
              fb[j].w = v.y;
            }
          });
        }
        static_for<FM * FN>([&](auto xc) {
          constexpr int x = decltype(xc)::value, ii = x / FN, j = x % FN;
          acc[ii][j] = Mfma<T>::mma(fb[j], fa[ii][KSC * h + s], acc[ii][j]);
        });
      });
    });
    // results -> staging: with two buffers, buffer i % 2, last read by the stores of tile
    // i-2 (during the chunks of tile i-1), which every wave finished before this tile's
    // barriers; with one, the buffer the stores of tile i-1 read during this tile's chunks,
    // so every wave first waits for the others to be past those reads
    if constexpr (SB == 1) asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" : : : "memory");
    unsigned char* stg = stg0 + (SB == 2 ? (i & 1) * STG : 0);
#pragma unroll
    for (int ii = 0; ii < FM; ++ii) {
      f32x4 v0 = acc[ii][0], v1 = acc[ii][1];
      if constexpr (BIAS == 2) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v0[e] += bias_m[ii];
          v1[e] += bias_m[ii];
        }
      }
      uint32_t P0[2] = {pack2<T>(v0[0], v0[1]), pack2<T>(v0[2], v0[3])};
      uint32_t P1[2] = {pack2<T>(v1[0], v1[1]), pack2<T>(v1[2], v1[3])};
#pragma unroll
      for (int w = 0; w < 2; ++w) {
        const auto sw = __builtin_amdgcn_permlane16_swap(P0[w], P1[w], false, false);
        P0[w] = sw[0];
        P1[w] = sw[1];
      }
      const int row = RW * grp + 16 * ii + r16;
      *(u32x4*)(stg + row * 256 + (((col >> 3) ^ (row & 15)) << 4)) = u32x4{P0[0], P0[1], P1[0], P1[1]};
    }
  }
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" : : : "memory");  // the last tile is staged
  static_for<KC>([&](auto hc) { store(ntiles - 1, hc); });
  asm volatile("s_waitcnt vmcnt(0)" : : : "memory");  // no LDS DMA may outlive the workgroup
}

}  // namespace cmpext3
