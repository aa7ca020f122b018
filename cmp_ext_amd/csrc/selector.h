// Host-side kernel selector (plain C++, no HIP): validates a GEMM request and
// picks the kernel, tile and launch geometry.
#pragma once

#include <stdint.h>

#include <string>

#include "gemm_params.h"

namespace cmpext3 {

struct Plan {
  KernelId kernel;
  int bm, bn;             // output tile of one workgroup
  int tiles_m, tiles_n;   // tile grid (skinny: tiles_m = 1, tiles_n = strips)
  int group_m;            // tile-order group height
  int mb;                 // skinny: 16-row blocks of M
  int threads;            // workgroup size
  int splits;             // skinny wide: K splits (1 = no workspace)
  int ksplit;             // skinny wide: K range per split (multiple of 64)
  int64_t ws_bytes;       // workspace the plan needs (padded copies first, then split-K partials)
  // 16-bit operands whose rows are not 16-byte aligned (odd K or N, offset views)
  // are copied, zero-padded, into the workspace so that a tiled kernel can run:
  bool pad_a, pad_b;
  int64_t kp;                          // the K the kernel runs with (K rounded up to 8 when padded)
  int64_t lda_p, ldb_p;                // pitches of the copies
  int64_t stride_a_p, stride_b_p;      // their batch strides (0: one copy shared by the batch)
  int64_t pad_a_bytes, pad_b_bytes;    // workspace bytes of each copy (multiples of 256)
  bool dma16;  // fp32: rows 16-byte aligned, K (and N for B as [K,N]) multiples of 4
  bool forced;  // chosen by the CMPEXT3_GEMM_CONFIG override (no padded copies in its place)
};

struct Request {
  int dtype, layout;
  int64_t M, N, K;
  int64_t lda, ldb, ldc;
  int64_t stride_a, stride_b, stride_c;
  int align;  // largest power of two (<= 16) dividing the addresses of A, B and C
  int align_a, align_b, align_c;  // the same for A, B and C alone (0: use `align`); the bias
                                  // address never restricts the kernel choice
  bool b_cols_padded;             // B ([K, N]) has zero columns up to a multiple of 8 (planner use)
  bool has_bias;
  bool bias_row;  // the bias is one value per row of C (a 1x1 convolution's), not per column
  int64_t batch;
  int64_t ws_bytes;  // workspace the caller provides (0: none)
};

// Returns 0 and fills *plan, or a negative CMPEXT3_ERR_* code.
int make_plan(const Request& r, Plan* plan);

// A 16-bit tiled product whose last round of tiles would run mostly empty (rows just
// past a multiple of what one round covers) runs as two launches over its rows: rows
// [0, m_main) with `main`, the remaining rows with `tail` (each planned for its rows of
// the same operands; they write disjoint rows of C).
struct RowSplit {
  int64_t m_main;
  Plan main, tail;
};
// Given the plan for all rows, returns true and fills *out when the two launches are
// modelled to take less than 0.92 of its time.
bool plan_row_split(const Request& r, const Plan& full, RowSplit* out);

// One-line description of a plan, e.g. "tile256x256 f16 KN grid=256x1".
std::string describe(const Request& r, const Plan& p);

// Number of compute units the tile cost model assumes (MI355X: 256).
constexpr int kNumCUs = 256;
// Most rows of C the streaming kernel takes (16 row blocks of 128).
constexpr int kStreamMaxRows = 2048;

}  // namespace cmpext3
