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

// Padded uint8 bin copies (see Bias): one thread per (b, i, j) of (B, Np, Np).
__global__ void __launch_bounds__(256) bins8_kernel(const int* __restrict__ bins, int B, int N, int Np,
                                                    uint8_t* __restrict__ b8, uint8_t* __restrict__ b8t) {
  const size_t e = (size_t)blockIdx.x * 256 + threadIdx.x;
  const size_t per = (size_t)Np * Np;
  if (e >= (size_t)B * per) return;
  const int b = (int)(e / per);
  const int i = (int)((e % per) / Np), j = (int)(e % Np);
  int v = (int)BIN_NONE;
  if (i < N && j < N) {
    const int k = bins[((size_t)b * N + i) * N + j];
    v = (k >= 0 && k < 68) ? k : (int)BIN_NONE;
  }
  b8[e] = (uint8_t)v;
  b8t[(size_t)b * per + (size_t)j * Np + i] = (uint8_t)v;
}

hipError_t launch_bins8(const int* bins, int B, int N, uint8_t* b8, uint8_t* b8t, hipStream_t stream) {
  const int Np = ((N + 31) / 32) * 32;
  const size_t total = (size_t)B * Np * Np;
  hipLaunchKernelGGL(bins8_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream, bins, B, N, Np, b8, b8t);
  return hipGetLastError();
}

// Zero fill of n 64-bit words (workspace exchange regions): a kernel rather than
// hipMemsetAsync, so that a caller may capture the launch in a HIP graph.
__global__ void __launch_bounds__(256) fill_u64_kernel(uint64_t* __restrict__ p, size_t n) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) p[i] = 0;
}

hipError_t launch_fill_u64(uint64_t* p, size_t n, hipStream_t stream) {
  if (n == 0) return hipSuccess;
  const size_t blocks = (n + 255) / 256;
  hipLaunchKernelGGL(fill_u64_kernel, dim3((unsigned)(blocks < 1024 ? blocks : 1024)), dim3(256), 0, stream, p, n);
  return hipGetLastError();
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
