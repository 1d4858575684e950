// Flash-Sinkhorn forward, stream mode (sinkhorn_fwd_kernel.h): long sequences
// whose Q and K do not fit in LDS.  A translation unit of its own so that the
// two modes compile in parallel.
#include "sinkhorn_fwd_kernel.h"

namespace dfl {

hipError_t launch_sinkhorn_fwd_stream(const SinkFwdArgs& a, bool bf16_in, int DP, size_t lds, hipStream_t stream,
                                      bool coop) {
  return launch_fwd_mode<true>(a, bf16_in, DP, lds, stream, coop);
}

}  // namespace dfl
