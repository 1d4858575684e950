// Register-storage flash-Sinkhorn forward (sinkhorn_fwd_blk.h): instantiations,
// launch and the host-side fit check.
#include "sinkhorn_fwd_blk.h"

namespace dfl {

template <typename T, int DP, bool HIST, bool GEN>
static hipError_t launch_blk_t(const SinkFwdArgs& a, size_t lds, int L, hipStream_t stream, bool coop) {
  auto kern = sinkhorn_fwd_blk_kernel<T, DP, HIST, GEN>;
  hipError_t e = set_lds_limit((const void*)kern, lds);
  if (e != hipSuccess) return e;
  dim3 grid(8 * L), block(BLK_NT);
  SinkFwdArgs copy = a;
  if (coop) {
    void* args[] = {&copy};
    return hipLaunchCooperativeKernel((const void*)kern, grid, block, args, (unsigned)lds, stream);
  }
  hipLaunchKernelGGL(kern, grid, block, lds, stream, copy);
  return hipGetLastError();
}

template <bool HIST, bool GEN>
static hipError_t launch_blk_dt(const SinkFwdArgs& a, bool bf16_in, int DP, size_t lds, int L, hipStream_t stream,
                                bool coop) {
  if (bf16_in) {
    if (DP == 32) return launch_blk_t<bf16, 32, HIST, GEN>(a, lds, L, stream, coop);
    if (DP == 64) return launch_blk_t<bf16, 64, HIST, GEN>(a, lds, L, stream, coop);
  } else {
    if (DP == 32) return launch_blk_t<float, 32, HIST, GEN>(a, lds, L, stream, coop);
    if (DP == 64) return launch_blk_t<float, 64, HIST, GEN>(a, lds, L, stream, coop);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_sinkhorn_fwd_blk(const SinkFwdArgs& a, bool bf16_in, int DP, size_t lds, int L, hipStream_t stream,
                                   bool coop) {
  if (a.balanced || a.K_iter < 1) return hipErrorInvalidValue;
  const bool gen = (a.bins8 && a.pos_w) || (a.x && a.w_dist);
  if (a.hist)
    return gen ? launch_blk_dt<true, true>(a, bf16_in, DP, lds, L, stream, coop)
               : launch_blk_dt<true, false>(a, bf16_in, DP, lds, L, stream, coop);
  return gen ? launch_blk_dt<false, true>(a, bf16_in, DP, lds, L, stream, coop)
             : launch_blk_dt<false, false>(a, bf16_in, DP, lds, L, stream, coop);
}

size_t sinkhorn_fwd_blk_lds_bytes(int N, int DP, int elem) { return blk_lds_bytes(N, DP, elem); }

bool sinkhorn_fwd_blk_fits(int B, int H, int N, int L) { return blk_fits(B, H, N, L); }

}  // namespace dfl

namespace dfl {
// Exchange words the register-storage forward uses: BLK_XCH_VECS vectors of Np words
// per (b,h), then BLK_MAXL placement words per (b,h).
size_t sinkhorn_fwd_blk_xch_words(int B, int H, int N) {
  const size_t np = (size_t)((N + 31) / 32) * 32;
  return (size_t)B * H * (BLK_XCH_VECS * np + BLK_MAXL);
}
}  // namespace dfl
