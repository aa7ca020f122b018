// The streaming kernel's instantiations for B given as [N, K] (e.g. NHWC images in a 1x1
// convolution), in a translation unit of their own so that the two layouts build in parallel.
#include "stream_launch.h"

namespace cmpext3 {

hipError_t launch_stream_nk(DType dt, const GemmParams& p, int total, unsigned wgs, hipStream_t s) {
  return launch_stream_layout<true>(dt, p, total, wgs, s);
}

}  // namespace cmpext3
