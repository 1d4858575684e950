// Flash-Sinkhorn forward, resident layout with register storage (sinkhorn_fwd_kernel.h,
// FWD_UOT_REG): a translation unit of its own so that it compiles in parallel with the
// other modes.
#include "sinkhorn_fwd_kernel.h"

namespace dfl {

hipError_t launch_sinkhorn_fwd_reg(const SinkFwdArgs& a, bool bf16_in, int DP, size_t lds, hipStream_t stream,
                                   bool coop) {
  if (a.balanced || a.hist || a.K_iter < 1 || !reg_fits(a.N, a.G)) return hipErrorInvalidValue;
  const bool gen = (a.bins8 && a.pos_w) || (a.x && a.w_dist);
  return gen ? launch_fwd_reg_dt<true>(a, bf16_in, DP, lds, stream, coop)
             : launch_fwd_reg_dt<false>(a, bf16_in, DP, lds, stream, coop);
}

bool sinkhorn_fwd_reg_fits(int N, int G) { return reg_fits(N, G); }

size_t sinkhorn_fwd_reg_lds_bytes(int N, int DP, int elem, int G) {
  return sinkhorn_fwd_lds_bytes_t(N, DP, elem, G, false, true);
}

}  // namespace dfl
