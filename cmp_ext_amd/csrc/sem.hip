// Counters of the split-K reductions done inside the splitting kernel: the
// workgroups of one output strip (or tile) that sum disjoint K ranges each
// write their fp32 partial block, count themselves in on the strip's counter,
// and the last to arrive sums the partials in split order, adds the bias,
// rounds, stores C and puts the counter back to zero.  No second launch.
//
// The counters live in a file-scope device array, zero when the code object
// is loaded on a GPU and zero again after every kernel that used them.  It is
// split into slots of kSemCounters counters; a slot belongs to one stream of
// one GPU (the first kSemSlots streams of a GPU to ask get one each, in
// order), because kernels of one stream never overlap while kernels of two
// streams may.  Calls on a further stream, on hipStreamPerThread (one handle for
// a different stream per host thread), or under graph capture (whose kernels
// may later replay on any stream), get no slot: they reduce in a second launch
// instead.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>

#include "kernels.h"

namespace cmpext3 {
namespace {

constexpr int kMaxDevices = 64;

// In host code `split_sem` names a host-side stand-in; its device address is looked
// up per GPU (Table::base) and only that is passed to kernels.
static __device__ __align__(256) unsigned int split_sem[kSemSlots * kSemCounters];

struct Table {
  std::mutex mu;
  bool looked_up = false;
  unsigned int* base = nullptr;
  hipStream_t owner[kSemSlots];
  int used = 0;
};
Table g_tab[kMaxDevices];

}  // namespace

unsigned int* split_counters(hipStream_t s, int64_t count) {
  // hipStreamPerThread names a different stream on every host thread: no slot can be its own
  if (count <= 0 || count > kSemCounters || s == hipStreamPerThread) return nullptr;
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(s, &cap) != hipSuccess || cap != hipStreamCaptureStatusNone) return nullptr;
  int dev = -1;
  if ((s == nullptr ? hipGetDevice(&dev) : hipStreamGetDevice(s, &dev)) != hipSuccess) return nullptr;
  if (dev < 0 || dev >= kMaxDevices) return nullptr;
  Table& t = g_tab[dev];
  std::lock_guard<std::mutex> lock(t.mu);
  if (!t.looked_up) {  // once per GPU, with that GPU current
    t.looked_up = true;
    int cur = -1;
    if (hipGetDevice(&cur) != hipSuccess) return nullptr;
    if (cur != dev && hipSetDevice(dev) != hipSuccess) return nullptr;
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(split_sem)) == hipSuccess) t.base = (unsigned int*)p;
    if (cur != dev) (void)hipSetDevice(cur);
  }
  if (t.base == nullptr) return nullptr;
  for (int i = 0; i < t.used; ++i)
    if (t.owner[i] == s) return t.base + (int64_t)i * kSemCounters;
  if (t.used == kSemSlots) return nullptr;
  t.owner[t.used] = s;
  return t.base + (int64_t)(t.used++) * kSemCounters;
}

}  // namespace cmpext3
