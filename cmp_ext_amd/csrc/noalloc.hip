// cmpext3_gemm_ex_noalloc (include/cmpext3_gemm.h): cmpext3_gemm_ex with the
// library's own device scratch buffer as the workspace, for callers that may
// not allocate device memory (code under HIP graph capture, tight serving
// loops, harnesses that forbid hipMalloc).  The scratch buffer is a file-scope
// device array of CMPEXT3_SCRATCH_BYTES; every GPU the library runs on holds
// its own copy until the process ends.  Its device address on each GPU is
// looked up once, on the first call made with that GPU current, and used for
// every later call there.  Nothing here allocates or frees.
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

// Device address of `scratch` on the current device (hipGetSymbolAddress, once
// per device, with that device current), or a status.
int scratch_ptr(void** out) {
  int dev = -1;
  const hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kMaxDevices) return CMPEXT3_ERR_INVALID_ARG;
  std::call_once(g_once[dev], [dev]() {
    void* p = nullptr;
    g_err[dev] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    g_ptr[dev] = g_err[dev] == hipSuccess ? p : nullptr;
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
  // the plan cmpext3_gemm_ex would run with all the workspace it asks for
  cmpext3_gemm_call call;
  int st = cmpext3_gemm_prepare(&call, dtype, b_layout, A, lda, stride_a, B, ldb, stride_b, C, ldc, stride_c, bias, 0,
                                M, N, K, batch, INT64_MAX);
  if (st != CMPEXT3_OK) return st;
  const int64_t need = cmpext3_gemm_call_workspace_size(&call);
  if (need < 0) return (int)need;
  if (need > (int64_t)CMPEXT3_SCRATCH_BYTES) return CMPEXT3_ERR_SCRATCH;
  void* ws = nullptr;
  if (need > 0) {
    st = scratch_ptr(&ws);
    if (st != CMPEXT3_OK) return st;
  }
  // The kernels read back every workspace byte they write within the call, so
  // the scratch needs no clearing between calls.
  return cmpext3_gemm_run(&call, ws, need, stream);
}
