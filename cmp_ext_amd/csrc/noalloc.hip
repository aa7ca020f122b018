// cmpext3_gemm_ex_noalloc (include/cmpext3_gemm.h): cmpext3_gemm_ex with the
// library's own device scratch buffer as the workspace, for callers that may
// not allocate device memory (code under HIP graph capture, tight serving
// loops, harnesses that forbid hipMalloc).  The scratch buffer is a file-scope
// device array of CMPEXT3_SCRATCH_BYTES; every GPU the library runs on holds
// its own copy until the process ends.  Its device address on each GPU is
// looked up once, with that GPU current, and used for every later call whose
// stream belongs to that GPU.  Nothing here allocates or frees.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>

#include "../../include/cmpext3_gemm.h"

namespace {

// The scratch buffer.  In host code `scratch` names a host-side stand-in, not
// device memory: only its looked-up device address (scratch_ptr) is passed on.
static __device__ __align__(256) unsigned char scratch[CMPEXT3_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
void* g_ptr[kMaxDevices];
hipError_t g_err[kMaxDevices];
std::once_flag g_once[kMaxDevices];

// The GPU whose queue `stream` is (the current GPU for the null stream).
int stream_device(hipStream_t stream, int* dev) {
  hipError_t e = stream == nullptr ? hipGetDevice(dev) : hipStreamGetDevice(stream, dev);
  if (e != hipSuccess) return (int)e;
  return *dev >= 0 && *dev < kMaxDevices ? CMPEXT3_OK : CMPEXT3_ERR_INVALID_ARG;
}

// Device address of `scratch` on GPU `dev`: hipGetSymbolAddress once per GPU, made
// with that GPU current (and the caller's current GPU restored after it).
int scratch_ptr(int dev, void** out) {
  std::call_once(g_once[dev], [dev]() {
    int cur = -1;
    g_err[dev] = hipGetDevice(&cur);
    if (g_err[dev] != hipSuccess) return;
    if (cur != dev && (g_err[dev] = hipSetDevice(dev)) != hipSuccess) return;
    void* p = nullptr;
    g_err[dev] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    g_ptr[dev] = g_err[dev] == hipSuccess ? p : nullptr;
    if (cur != dev) {
      const hipError_t back = hipSetDevice(cur);
      if (g_err[dev] == hipSuccess && back != hipSuccess) g_err[dev] = back;
    }
  });
  if (g_err[dev] != hipSuccess) return (int)g_err[dev];
  if (g_ptr[dev] == nullptr) return (int)hipErrorInvalidSymbol;
  *out = g_ptr[dev];
  return CMPEXT3_OK;
}

}  // namespace

extern "C" int cmpext3_gemm_ex_noalloc(int dtype, int b_layout, const void* A, int64_t lda, int64_t stride_a,
                                       const void* B, int64_t ldb, int64_t stride_b, void* C, int64_t ldc,
                                       int64_t stride_c, const void* bias, int M, int N, int K, int batch,
                                       void* stream) {
  // the plan cmpext3_gemm_ex would run with all the workspace it asks for; when that
  // is more than the scratch holds, the plan for a workspace of the scratch's size
  // (fewer K splits, no padded copies: what cmpext3_gemm_ex runs with that much)
  cmpext3_gemm_call call;
  int st = cmpext3_gemm_prepare(&call, dtype, b_layout, A, lda, stride_a, B, ldb, stride_b, C, ldc, stride_c, bias, 0,
                                M, N, K, batch, INT64_MAX);
  if (st != CMPEXT3_OK) return st;
  int64_t need = cmpext3_gemm_call_workspace_size(&call);
  if (need < 0) return (int)need;
  if (need > (int64_t)CMPEXT3_SCRATCH_BYTES) {
    st = cmpext3_gemm_prepare(&call, dtype, b_layout, A, lda, stride_a, B, ldb, stride_b, C, ldc, stride_c, bias, 0,
                              M, N, K, batch, (int64_t)CMPEXT3_SCRATCH_BYTES);
    if (st != CMPEXT3_OK) return st;
    need = cmpext3_gemm_call_workspace_size(&call);
    if (need < 0) return (int)need;
    if (need > (int64_t)CMPEXT3_SCRATCH_BYTES) return CMPEXT3_ERR_SCRATCH;
  }
  void* ws = nullptr;
  if (need > 0) {
    int dev = -1;
    st = stream_device((hipStream_t)stream, &dev);
    if (st != CMPEXT3_OK) return st;
    st = scratch_ptr(dev, &ws);
    if (st != CMPEXT3_OK) return st;
  }
  // The kernels read back every workspace byte they write within the call, so
  // the scratch needs no clearing between calls.
  return cmpext3_gemm_run(&call, ws, need, stream);
}
