// Flash-Sinkhorn forward, resident mode (sinkhorn_fwd_kernel.h), plus the
// stream-mode operand padding kernel and the LDS sizing used by the C ABI.
#include "sinkhorn_fwd_kernel.h"

namespace dfl {

size_t sinkhorn_fwd_lds_bytes(int N, int DP, int elem, int G, bool stream) {
  return sinkhorn_fwd_lds_bytes_t(N, DP, elem, G, stream);
}

hipError_t launch_sinkhorn_fwd(const SinkFwdArgs& a, bool bf16_in, int DP, size_t lds, hipStream_t stream,
                               bool coop) {
  return launch_fwd_mode<false>(a, bf16_in, DP, lds, stream, coop);
}

template <typename T, int DP>
static hipError_t launch_pad_t(const PadArgs& p, hipStream_t stream) {
  const size_t Np = ((p.N + 31) / 32) * 32;
  const size_t threads = (size_t)p.B * p.H * Np * DP;  // multiple of 1024
  hipLaunchKernelGGL((sinkhorn_pad_kernel<T, DP>), dim3((unsigned)(threads / 256)), dim3(256), 0, stream, p);
  return hipGetLastError();
}

hipError_t launch_sinkhorn_pad(const PadArgs& p, bool bf16_in, int DP, hipStream_t stream) {
  if (bf16_in) {
    if (DP == 32) return launch_pad_t<bf16, 32>(p, stream);
    if (DP == 64) return launch_pad_t<bf16, 64>(p, stream);
  } else {
    if (DP == 32) return launch_pad_t<float, 32>(p, stream);
    if (DP == 64) return launch_pad_t<float, 64>(p, stream);
  }
  return hipErrorInvalidValue;
}

}  // namespace dfl
