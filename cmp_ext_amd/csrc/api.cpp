// C ABI of the gfx950 GEMM library (declared in include/cmpext3_gemm.h).
// Validates, asks the selector for a plan and launches one kernel per call
// (or one per 65535 batch entries) on the caller's stream.
#include <hip/hip_runtime_api.h>
#include <string.h>

#include <stdint.h>

#include <algorithm>
#include <string>
#include <type_traits>

#include "../../include/cmpext3_gemm.h"
#include "kernels.h"
#include "selector.h"

using namespace cmpext3;

namespace {

int align_of(const void* ptr) {
  const uintptr_t v = (uintptr_t)ptr;
  if (v == 0) return 16;
  int a = 1;
  while (a < 16 && v % (uintptr_t)(2 * a) == 0) a *= 2;
  return a;
}

// The tile kernel for the element type and B layout, with whole-step loads when K
// (and every split's K range) is a multiple of 64.
hipError_t launch_tile(int dtype, KernelId id, BLayout lay, const GemmParams& p, dim3 grid, hipStream_t s) {
  const bool ragged = p.K % 64 != 0 || (p.splits > 1 && p.ksplit % 64 != 0);
  if (dtype == kF16) {
    if (lay == kKN) return ragged ? launch_tile_f16_kn_ragged(id, p, grid, s) : launch_tile_f16_kn_whole(id, p, grid, s);
    return ragged ? launch_tile_f16_nk_ragged(id, p, grid, s) : launch_tile_f16_nk_whole(id, p, grid, s);
  }
  if (lay == kKN) return ragged ? launch_tile_bf16_kn_ragged(id, p, grid, s) : launch_tile_bf16_kn_whole(id, p, grid, s);
  return ragged ? launch_tile_bf16_nk_ragged(id, p, grid, s) : launch_tile_bf16_nk_whole(id, p, grid, s);
}

hipError_t dispatch(const Plan& plan, int dtype, int layout, const GemmParams& p, dim3 grid, void* ws,
                    hipStream_t s) {
  const BLayout lay = (BLayout)layout;
  switch (plan.kernel) {
    case kSkinnyWide: {
      // split K: the last workgroup of each column strip to finish sums the partials
      // (counters of this stream; a batch entry's partial block addressed with 32-bit
      // byte offsets), else a second launch does
      const bool fuse = plan.splits > 1 && (int64_t)p.M * p.N * 4 < (1ll << 31);
      unsigned int* sem = fuse ? split_counters(s, (int64_t)grid.z * (grid.x / plan.splits)) : nullptr;
      hipError_t e = launch_skinny_wide((DType)dtype, plan.mb, p, (float*)ws, plan.splits, plan.ksplit, grid, s, sem);
      if (e == hipSuccess && plan.splits > 1 && sem == nullptr)
        e = launch_skinny_reduce((DType)dtype, p, (const float*)ws, plan.splits, (int)grid.z, s);
      return e;
    }
    case kTile256x256:
    case kTile256x224:
    case kTile128x128:
      if (plan.splits > 1) {  // split K: fp32 partials, then the reduction adds the bias and rounds
        GemmParams q = p;
        q.splits = plan.splits;
        q.ksplit = plan.ksplit;
        q.partials = (float*)ws;
        const dim3 g(grid.x, grid.y, grid.z * plan.splits);
        hipError_t e = launch_tile(dtype, plan.kernel, lay, q, g, s);
        if (e == hipSuccess) e = launch_skinny_reduce((DType)dtype, p, (const float*)ws, plan.splits, (int)grid.z, s);
        return e;
      }
      [[fallthrough]];
    case kTile64x256:
      return launch_tile(dtype, plan.kernel, lay, p, grid, s);
    case kStream64x128:
    case kStream128x128:
      return launch_stream((DType)dtype, lay, p, grid, s);
    case kSkinny:
      return launch_skinny((DType)dtype, plan.mb, p, grid, s);
    case kSkinnyNK:
    case kTall:
      if (plan.splits > 1) {  // split K: fp32 partials, then the reduction adds the bias and rounds
        GemmParams q = p;
        q.splits = plan.splits;
        q.ksplit = plan.ksplit;
        q.partials = (float*)ws;
        const dim3 g(grid.x, grid.y, grid.z * plan.splits);
        hipError_t e = plan.kernel == kTall ? launch_tall((DType)dtype, lay, plan.mb, plan.bm, q, g, s)
                                            : launch_skinny_nk((DType)dtype, plan.mb, plan.bn, q, g, s);
        if (e == hipSuccess) e = launch_skinny_reduce((DType)dtype, p, (const float*)ws, plan.splits, (int)grid.z, s);
        return e;
      }
      return plan.kernel == kTall ? launch_tall((DType)dtype, lay, plan.mb, plan.bm, p, grid, s)
                                  : launch_skinny_nk((DType)dtype, plan.mb, plan.bn, p, grid, s);
    case kF32Tile128:
    case kF32Tile64:
    case kF32Tile96x64:
    case kF32Tile64K4:
    case kF32Tile16K4:
      if (plan.splits > 1) {  // split K: fp32 partials, then the reduction adds the bias
        GemmParams q = p;
        q.splits = plan.splits;
        q.ksplit = plan.ksplit;
        q.partials = (float*)ws;
        hipError_t e = launch_f32(plan.kernel, lay, plan.dma16, q, dim3(grid.x, grid.y, grid.z * plan.splits), s);
        if (e == hipSuccess) e = launch_skinny_reduce(kF32, p, (const float*)ws, plan.splits, (int)grid.z, s);
        return e;
      }
      return launch_f32(plan.kernel, lay, plan.dma16, p, grid, s);
    case kGeneric16:
      return launch_generic((DType)dtype, lay, p, grid, s);
    default:
      return hipErrorInvalidValue;
  }
}

// A plan's description; for a row split, both launches'.
std::string describe_rows(const Request& r, const Plan& plan, int64_t m_main, const Plan& tail) {
  if (m_main <= 0) return describe(r, plan);
  Request head = r, rest = r;
  head.M = m_main;
  rest.M = r.M - m_main;
  return describe(head, plan) + " rows=" + std::to_string(m_main) + " | rows " + std::to_string(m_main) + ".." +
         std::to_string(r.M - 1) + ": " + describe(rest, tail);
}

constexpr int64_t kMaxGridZ = 65535;
constexpr uint64_t kCallMagic = 0x636d7065787433ull;  // "cmpext3"

// The contents of a cmpext3_gemm_call: one validated, planned GEMM.
struct Prepared {
  uint64_t magic;
  Request r;
  Plan plan;
  // rows [0, m_main) run with `plan`, the rest with `tail` (0: one launch for all rows)
  int64_t m_main;
  Plan tail;
  const void* A;
  const void* B;
  void* C;
  const void* bias;
  int bias_row;
  bool empty;  // M, N or batch is 0: nothing to launch
};
static_assert(sizeof(Prepared) <= sizeof(cmpext3_gemm_call), "cmpext3_gemm_call too small");
static_assert(std::is_trivially_copyable<Prepared>::value, "cmpext3_gemm_call is copied bytewise");

int prepare(Prepared* pc, int dtype, int b_layout, const void* A, int64_t lda, int64_t stride_a, const void* B,
            int64_t ldb, int64_t stride_b, void* C, int64_t ldc, int64_t stride_c, const void* bias, int bias_row,
            int M, int N, int K, int batch, int64_t workspace_limit) {
  Request r{};
  r.dtype = dtype;
  r.layout = b_layout;
  r.M = M;
  r.N = N;
  r.K = K;
  r.lda = lda;
  r.ldb = ldb;
  r.ldc = ldc;
  r.stride_a = stride_a;
  r.stride_b = stride_b;
  r.stride_c = stride_c;
  // the bias is read element by element where its address needs it (tile kernels:
  // GemmParams::bias_vec), so only A, B and C steer the kernel choice
  r.align_a = align_of(A);
  r.align_b = align_of(B);
  r.align_c = align_of(C);
  r.align = std::min(std::min(r.align_a, r.align_b), r.align_c);
  r.has_bias = bias != nullptr;
  r.bias_row = bias != nullptr && bias_row != 0;
  r.batch = batch;
  r.ws_bytes = std::max<int64_t>(0, workspace_limit);
  Plan plan;
  const int st = make_plan(r, &plan);
  if (st != CMPEXT3_OK) return st;
  const bool empty = M == 0 || N == 0 || batch == 0;
  if (!empty && (C == nullptr || (K > 0 && (A == nullptr || B == nullptr)))) return CMPEXT3_ERR_INVALID_ARG;
  if (empty) plan.ws_bytes = 0;
  Prepared p{};
  p.magic = kCallMagic;
  p.r = r;
  p.plan = plan;
  RowSplit rs;
  if (!empty && plan_row_split(r, plan, &rs)) {
    p.plan = rs.main;
    p.m_main = rs.m_main;
    p.tail = rs.tail;
  }
  p.A = A;
  p.B = B;
  p.C = C;
  p.bias = bias;
  p.bias_row = bias_row;
  p.empty = empty;
  *pc = p;
  return CMPEXT3_OK;
}

const Prepared* as_prepared(const cmpext3_gemm_call* call) {
  if (call == nullptr) return nullptr;
  const Prepared* pc = reinterpret_cast<const Prepared*>(call);
  return pc->magic == kCallMagic ? pc : nullptr;
}

// Enqueues a prepared call: the zero-padded operand copies it planned, then its
// kernel(s), batch entries in chunks of at most 65535 grid rows.
int run(const Prepared& pc, void* workspace, int64_t workspace_bytes, hipStream_t s) {
  const Plan& plan = pc.plan;
  if (pc.empty) return CMPEXT3_OK;
  if (pc.m_main > 0) {  // two launches over the rows, one after the other on the stream
    const int64_t esz = pc.r.dtype == kF32 ? 4 : 2;
    Prepared head = pc, rest = pc;
    head.m_main = rest.m_main = 0;
    head.r.M = pc.m_main;
    rest.r.M = pc.r.M - pc.m_main;
    rest.plan = pc.tail;
    rest.A = (const char*)pc.A + pc.m_main * pc.r.lda * esz;
    rest.C = (char*)pc.C + pc.m_main * pc.r.ldc * esz;
    if (pc.bias != nullptr && pc.bias_row) rest.bias = (const char*)pc.bias + pc.m_main * esz;
    const int st = run(head, workspace, workspace_bytes, s);
    return st != CMPEXT3_OK ? st : run(rest, workspace, workspace_bytes, s);
  }
  if (plan.ws_bytes > 0 && (workspace == nullptr || align_of(workspace) < 16 || workspace_bytes < plan.ws_bytes))
    return CMPEXT3_ERR_WORKSPACE;
  const int dtype = pc.r.dtype, b_layout = pc.r.layout;
  const int M = (int)pc.r.M, N = (int)pc.r.N, batch = (int)pc.r.batch;
  int K = (int)pc.r.K;
  const void* A = pc.A;
  const void* B = pc.B;
  int64_t lda = pc.r.lda, ldb = pc.r.ldb, stride_a = pc.r.stride_a, stride_b = pc.r.stride_b;
  const int64_t esz = dtype == kF32 ? 4 : 2;
  char* ws = (char*)workspace;
  const bool kn = b_layout == CMPEXT3_B_KN;
  if (plan.pad_a) {
    const int64_t copies = (batch > 1 && stride_a != 0) ? batch : 1;
    const hipError_t e = launch_pad_copy(A, lda, stride_a, M, K, ws, plan.lda_p, plan.stride_a_p, M, (int)plan.kp,
                                         copies, (int)esz, s);
    if (e != hipSuccess) return (int)e;
    A = ws;
    lda = plan.lda_p;
    stride_a = plan.stride_a_p;
    ws += plan.pad_a_bytes;
  }
  if (plan.pad_b) {
    const int64_t copies = (batch > 1 && stride_b != 0) ? batch : 1;
    const int rows = kn ? K : N, cols = kn ? N : K;
    const int dst_rows = kn ? (int)plan.kp : N;
    const hipError_t e = launch_pad_copy(B, ldb, stride_b, rows, cols, ws, plan.ldb_p, plan.stride_b_p, dst_rows,
                                         (int)plan.ldb_p, copies, (int)esz, s);
    if (e != hipSuccess) return (int)e;
    B = ws;
    ldb = plan.ldb_p;
    stride_b = plan.stride_b_p;
    ws += plan.pad_b_bytes;
  }
  if (plan.pad_a || plan.pad_b) K = (int)plan.kp;
  GemmParams p{};
  p.bias = pc.bias;
  p.bias_row = pc.bias_row;
  p.bias_vec = pc.bias != nullptr && align_of(pc.bias) >= 8;
  p.lda = lda;
  p.ldb = ldb;
  p.ldc = pc.r.ldc;
  p.stride_a = stride_a;
  p.stride_b = stride_b;
  p.stride_c = pc.r.stride_c;
  p.M = M;
  p.N = N;
  p.K = K;
  p.tiles_m = plan.tiles_m;
  p.tiles_n = plan.tiles_n;
  p.group_m = plan.group_m;
  // kernels whose K split multiplies grid.z (the skinny_wide split goes along grid.x)
  const bool split_z = plan.kernel == kTile256x256 || plan.kernel == kTile256x224 || plan.kernel == kTile128x128 ||
                     plan.kernel == kF32Tile128 || plan.kernel == kF32Tile96x64 || plan.kernel == kF32Tile64 ||
                     plan.kernel == kF32Tile64K4 || plan.kernel == kF32Tile16K4 || plan.kernel == kSkinnyNK ||
                     plan.kernel == kTall;
  const int64_t zmax = kMaxGridZ / std::max(1, split_z ? plan.splits : 1);
  for (int64_t b0 = 0; b0 < batch; b0 += zmax) {
    const int64_t nb = std::min<int64_t>(zmax, batch - b0);
    p.A = (const char*)A + b0 * stride_a * esz;
    p.B = (const char*)B + b0 * stride_b * esz;
    p.C = (char*)pc.C + b0 * pc.r.stride_c * esz;
    const dim3 grid((unsigned)(plan.tiles_m * plan.tiles_n), 1, (unsigned)nb);
    const hipError_t e = dispatch(plan, dtype, b_layout, p, grid, ws, s);
    if (e != hipSuccess) return (int)e;
  }
  return CMPEXT3_OK;
}

// Shared body of cmpext3_gemm_ex (bias per column) and cmpext3_conv2d_1x1
// (bias per row): prepare with the workspace at hand, then run.
int run_gemm(int dtype, int b_layout, const void* A, int64_t lda, int64_t stride_a, const void* B, int64_t ldb,
             int64_t stride_b, void* C, int64_t ldc, int64_t stride_c, const void* bias, int bias_row, int M, int N,
             int K, int batch, void* workspace, int64_t workspace_bytes, void* stream) {
  Prepared pc;
  const int64_t limit = (workspace != nullptr && align_of(workspace) >= 16) ? workspace_bytes : 0;
  const int st = prepare(&pc, dtype, b_layout, A, lda, stride_a, B, ldb, stride_b, C, ldc, stride_c, bias, bias_row,
                         M, N, K, batch, limit);
  if (st != CMPEXT3_OK) return st;
  return run(pc, workspace, workspace_bytes, (hipStream_t)stream);
}

}  // namespace

extern "C" int cmpext3_gemm_ex(int dtype, int b_layout, const void* A, int64_t lda, int64_t stride_a,
                               const void* B, int64_t ldb, int64_t stride_b, void* C, int64_t ldc,
                               int64_t stride_c, const void* bias, int M, int N, int K, int batch,
                               void* workspace, int64_t workspace_bytes, void* stream) {
  return run_gemm(dtype, b_layout, A, lda, stride_a, B, ldb, stride_b, C, ldc, stride_c, bias, 0, M, N, K, batch,
                  workspace, workspace_bytes, stream);
}

extern "C" int cmpext3_gemm_prepare(cmpext3_gemm_call* call, int dtype, int b_layout, const void* A, int64_t lda,
                                    int64_t stride_a, const void* B, int64_t ldb, int64_t stride_b, void* C,
                                    int64_t ldc, int64_t stride_c, const void* bias, int flags, int M, int N, int K,
                                    int batch, int64_t workspace_limit) {
  if (call == nullptr || (flags & ~CMPEXT3_BIAS_PER_ROW) != 0) return CMPEXT3_ERR_INVALID_ARG;
  memset(call, 0, sizeof *call);
  Prepared pc;
  const int st = prepare(&pc, dtype, b_layout, A, lda, stride_a, B, ldb, stride_b, C, ldc, stride_c, bias,
                         (flags & CMPEXT3_BIAS_PER_ROW) ? 1 : 0, M, N, K, batch, workspace_limit);
  if (st != CMPEXT3_OK) return st;
  memcpy(call, &pc, sizeof pc);
  return CMPEXT3_OK;
}

extern "C" int64_t cmpext3_gemm_call_workspace_size(const cmpext3_gemm_call* call) {
  const Prepared* pc = as_prepared(call);
  if (pc == nullptr) return (int64_t)CMPEXT3_ERR_INVALID_ARG;
  // the two launches of a row split share the workspace, one after the other
  return pc->m_main > 0 ? std::max(pc->plan.ws_bytes, pc->tail.ws_bytes) : pc->plan.ws_bytes;
}

extern "C" int cmpext3_gemm_call_describe(const cmpext3_gemm_call* call, char* buf, int buflen) {
  const Prepared* pc = as_prepared(call);
  if (pc == nullptr) return CMPEXT3_ERR_INVALID_ARG;
  if (buf && buflen > 0) {
    const std::string d = describe_rows(pc->r, pc->plan, pc->m_main, pc->tail);
    strncpy(buf, d.c_str(), (size_t)buflen - 1);
    buf[buflen - 1] = '\0';
  }
  return (int)pc->plan.kernel;
}

extern "C" int cmpext3_gemm_run(const cmpext3_gemm_call* call, void* workspace, int64_t workspace_bytes,
                                void* stream) {
  const Prepared* pc = as_prepared(call);
  if (pc == nullptr) return CMPEXT3_ERR_INVALID_ARG;
  return run(*pc, workspace, workspace_bytes, (hipStream_t)stream);
}

// NCHW 1x1 convolution = `batch` GEMMs out_b[c_out, hw] = W[c_out, c_in] * in_b[c_in, hw]
// that share A (stride_a = 0), with B in the [K, N] layout and the bias per row.
extern "C" int cmpext3_conv2d_1x1(int dtype, const void* input, const void* weight, const void* bias, void* output,
                                  int batch, int c_in, int c_out, int hw, void* workspace, int64_t workspace_bytes,
                                  void* stream) {
  if (batch < 0 || c_in < 0 || c_out < 0 || hw < 0) return CMPEXT3_ERR_INVALID_ARG;
  return run_gemm(dtype, CMPEXT3_B_KN, weight, c_in > 1 ? c_in : 1, 0, input, hw > 1 ? hw : 1, (int64_t)c_in * hw,
                  output, hw > 1 ? hw : 1, (int64_t)c_out * hw, bias, 1, c_out, hw, c_in, batch, workspace,
                  workspace_bytes, stream);
}

extern "C" int cmpext3_matmul_fp16(const void* A, const void* B, void* C, int M, int N, int K, void* stream) {
  return cmpext3_gemm_ex(CMPEXT3_F16, CMPEXT3_B_KN, A, K > 1 ? K : 1, 0, B, N > 1 ? N : 1, 0, C, N > 1 ? N : 1, 0,
                         nullptr, M, N, K, 1, nullptr, 0, stream);
}

extern "C" int cmpext3_matmul_bf16(const void* A, const void* B, void* C, int M, int N, int K, void* stream) {
  return cmpext3_gemm_ex(CMPEXT3_BF16, CMPEXT3_B_KN, A, K > 1 ? K : 1, 0, B, N > 1 ? N : 1, 0, C, N > 1 ? N : 1, 0,
                         nullptr, M, N, K, 1, nullptr, 0, stream);
}

extern "C" int cmpext3_matmul_fp32(const float* A, const float* B, float* C, int M, int N, int K, void* stream) {
  return cmpext3_gemm_ex(CMPEXT3_F32, CMPEXT3_B_KN, A, K > 1 ? K : 1, 0, B, N > 1 ? N : 1, 0, C, N > 1 ? N : 1, 0,
                         nullptr, M, N, K, 1, nullptr, 0, stream);
}

extern "C" int cmpext3_gemm_f16(const void* A, int64_t lda, const void* B, int64_t ldb, void* C, int64_t ldc,
                                int M, int N, int K, void* stream) {
  return cmpext3_gemm_ex(CMPEXT3_F16, CMPEXT3_B_KN, A, lda, 0, B, ldb, 0, C, ldc, 0, nullptr, M, N, K, 1, nullptr,
                         0, stream);
}

extern "C" int cmpext3_gemm_bf16(const void* A, int64_t lda, const void* B, int64_t ldb, void* C, int64_t ldc,
                                 int M, int N, int K, void* stream) {
  return cmpext3_gemm_ex(CMPEXT3_BF16, CMPEXT3_B_KN, A, lda, 0, B, ldb, 0, C, ldc, 0, nullptr, M, N, K, 1, nullptr,
                         0, stream);
}

extern "C" int cmpext3_gemm_f32(const float* A, int64_t lda, const float* B, int64_t ldb, float* C, int64_t ldc,
                                int M, int N, int K, void* stream) {
  return cmpext3_gemm_ex(CMPEXT3_F32, CMPEXT3_B_KN, A, lda, 0, B, ldb, 0, C, ldc, 0, nullptr, M, N, K, 1, nullptr,
                         0, stream);
}

namespace {
Request plan_request(int dtype, int b_layout, int M, int N, int K, int64_t lda, int64_t ldb, int64_t ldc, int align,
                     int has_bias, int batch, int64_t ws_bytes) {
  Request r{};
  r.dtype = dtype;
  r.layout = b_layout;
  r.M = M;
  r.N = N;
  r.K = K;
  r.lda = lda;
  r.ldb = ldb;
  r.ldc = ldc;
  r.stride_a = (int64_t)M * lda;
  r.stride_b = (int64_t)(b_layout == CMPEXT3_B_KN ? K : N) * ldb;
  r.stride_c = (int64_t)M * ldc;
  r.align = align;
  r.has_bias = has_bias != 0;
  r.batch = batch;
  r.ws_bytes = ws_bytes;
  return r;
}
}  // namespace

extern "C" int64_t cmpext3_gemm_workspace_size(int dtype, int b_layout, int M, int N, int K, int batch) {
  const int64_t ldb = b_layout == CMPEXT3_B_KN ? N : K;
  const Request r = plan_request(dtype, b_layout, M, N, K, K > 1 ? K : 1, ldb > 1 ? ldb : 1, N > 1 ? N : 1, 16, 0,
                                 batch, INT64_MAX);
  Plan plan;
  const int st = make_plan(r, &plan);
  if (st != CMPEXT3_OK) return st;
  RowSplit rs;
  return plan_row_split(r, plan, &rs) ? std::max(rs.main.ws_bytes, rs.tail.ws_bytes) : plan.ws_bytes;
}

extern "C" int cmpext3_gemm_plan(int dtype, int b_layout, int M, int N, int K, int64_t lda, int64_t ldb,
                                 int64_t ldc, int align, int has_bias, int batch, int64_t workspace_bytes, char* buf,
                                 int buflen) {
  const Request r = plan_request(dtype, b_layout, M, N, K, lda, ldb, ldc, align, has_bias, batch, workspace_bytes);
  Plan plan;
  const int st = make_plan(r, &plan);
  if (st != CMPEXT3_OK) return st;
  RowSplit rs;
  const bool split = M > 0 && N > 0 && batch > 0 && plan_row_split(r, plan, &rs);
  if (buf && buflen > 0) {
    const std::string d = split ? describe_rows(r, rs.main, rs.m_main, rs.tail) : describe(r, plan);
    strncpy(buf, d.c_str(), (size_t)buflen - 1);
    buf[buflen - 1] = '\0';
  }
  return (int)(split ? rs.main.kernel : plan.kernel);
}

extern "C" const char* cmpext3_status_string(int status) {
  switch (status) {
    case CMPEXT3_OK: return "success";
    case CMPEXT3_ERR_INVALID_ARG: return "invalid argument (null pointer, negative size or leading dimension too small)";
    case CMPEXT3_ERR_UNSUPPORTED: return "unsupported dtype or B layout";
    case CMPEXT3_ERR_TOO_LARGE: return "size or leading dimension exceeds the kernels' 32-bit offset range";
    case CMPEXT3_ERR_WORKSPACE:
      return "workspace missing, not 16-byte aligned or smaller than the prepared call needs "
             "(cmpext3_gemm_call_workspace_size)";
    case CMPEXT3_ERR_SCRATCH:
      return "the call needs more workspace than the library's static scratch buffer holds "
             "(CMPEXT3_SCRATCH_BYTES); use cmpext3_gemm_ex with a workspace";
    default:
      if (status > 0) return hipGetErrorString((hipError_t)status);
      return "unknown status";
  }
}

extern "C" const char* cmpext3_version(void) { return "cmpext3-mi355x 0.1.0 (gfx950)"; }
