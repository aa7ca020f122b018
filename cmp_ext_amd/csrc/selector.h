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
  int64_t ws_bytes;       // workspace the plan needs
};

struct Request {
  int dtype, layout;
  int64_t M, N, K;
  int64_t lda, ldb, ldc;
  int64_t stride_a, stride_b, stride_c;
  int align;  // largest power of two (<= 16) dividing every operand address
  bool has_bias;
  int64_t batch;
  int64_t ws_bytes;  // workspace the caller provides (0: none)
};

// Returns 0 and fills *plan, or a negative CMPEXT3_ERR_* code.
int make_plan(const Request& r, Plan* plan);

// One-line description of a plan, e.g. "tile256x256 f16 KN grid=256x1".
std::string describe(const Request& r, const Plan& p);

// Number of compute units the tile cost model assumes (MI355X: 256).
constexpr int kNumCUs = 256;

}  // namespace cmpext3
