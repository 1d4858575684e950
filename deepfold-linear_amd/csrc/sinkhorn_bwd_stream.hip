// Flash-Sinkhorn IFT backward, stream mode (sinkhorn_bwd_kernel.h): long
// sequences whose operands and vectors do not fit in LDS.  A translation unit of
// its own so that the two modes compile in parallel.
#include "sinkhorn_bwd_kernel.h"

namespace dfl {

hipError_t launch_sinkhorn_bwd_stream(const SinkBwdArgs& a, bool bf16_in, int DP, size_t lds, hipStream_t stream,
                                      bool coop) {
  return launch_bwd_mode<true>(a, bf16_in, DP, lds, stream, coop);
}

}  // namespace dfl
