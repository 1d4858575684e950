// Flash-Sinkhorn IFT backward, resident mode (sinkhorn_bwd_kernel.h), plus the
// prep and finalize kernels shared by both storage modes and the LDS sizing used
// by the C ABI.
#include "sinkhorn_bwd_kernel.h"

namespace dfl {

// Prep: per (b,h) and row i < Np, with gO = sigma(G) dO on valid rows (0 elsewhere):
//   go_hi = T(gO), go_lo = T(gO - T(gO)), go_t = go_hi transposed, dG = sigma(1-sigma) O_avg dO,
//   D_i = sum_c gO_ic O_avg_ic + dxc_i . xc_i   (flash_sinkhorn_attn.py:278-292).
// One thread per (b, h, i, c), c < DP; the DP lanes of a row are contiguous in a wave.
template <typename T, int DP>
__global__ void __launch_bounds__(256) sinkhorn_bwd_prep_kernel(SinkBwdArgs a) {
  const int N = a.N, d = a.d;
  const int Np = ((N + 31) / 32) * 32;
  const size_t e = (size_t)blockIdx.x * 256 + threadIdx.x;  // grid covers B*H*Np*DP exactly
  const size_t row = e / DP;
  const int c = (int)(e % DP);
  const int bh = (int)(row / Np), i = (int)(row % Np);
  const int b = bh / a.H, h = bh % a.H;
  const bool ok = i < N && (a.mask ? a.mask[(size_t)b * N + i] > 0.5f : true);
  float go = 0.f, oa = 0.f, s = 1.f;
  if (ok && c < d) {
    go = a.grad_o[((size_t)b * N + i) * a.H * d + (size_t)h * d + c];
    oa = a.o_avg[((size_t)bh * N + i) * d + c];
    if (a.g) {
      const T* Gg = reinterpret_cast<const T*>(a.g) + (size_t)b * a.sb + (size_t)h * a.sh;
      s = sigm(to_f32(Gg[(size_t)i * a.sn + c]));
      put_grad<T>(a.dg, ((size_t)bh * N + i) * d + c, s * (1.f - s) * oa * go);
    }
  } else if (a.g && i < N && c < d) {
    put_grad<T>(a.dg, ((size_t)bh * N + i) * d + c, 0.f);
  }
  const float g = s * go;
  const T hi = from_f32<T>(g);
  reinterpret_cast<T*>(a.go_hi)[row * DP + c] = hi;
  reinterpret_cast<T*>(a.go_lo)[row * DP + c] = from_f32<T>(g - to_f32(hi));
  reinterpret_cast<T*>(a.go_t)[((size_t)bh * DP + c) * Np + i] = hi;
  float part = g * oa;
#pragma unroll
  for (int o = DP / 2; o >= 1; o >>= 1) part += __shfl_xor(part, o, WAVE);
  if (c == 0) {
    if (ok && a.grad_xc) {
      const float* dxc = a.grad_xc + ((size_t)bh * N + i) * 3;
      const float* xc = a.x_centroid + ((size_t)bh * N + i) * 3;
      part += dxc[0] * xc[0] + dxc[1] * xc[1] + dxc[2] * xc[2];
    }
    a.dcoef[row] = ok ? part : 0.f;
  }
}

// dx_res[b,i,:] = sum_h dx_part[b,h,i,:] on valid rows; dpw / dw summed over
// (b, member) partials in a fixed order.
__global__ void sinkhorn_bwd_finalize_kernel(SinkBwdArgs a, float* dx, float* dpw, float* dw) {
  const int tid = blockIdx.x * blockDim.x + threadIdx.x;
  const int total_x = a.B * a.N * 3;
  if (dx && a.x && tid < total_x) {
    const int b = tid / (a.N * 3);
    const int rem = tid - b * a.N * 3;
    const int i = rem / 3;
    const bool ok = a.mask ? a.mask[(size_t)b * a.N + i] > 0.5f : true;
    float s = 0.f;
    if (ok)
      for (int h = 0; h < a.H; ++h) s += a.dx_part[(((size_t)b * a.H + h) * a.N) * 3 + rem];
    dx[tid] = s;
  }
  if (tid < a.H * 68) {
    const int h = tid / 68, k = tid % 68;
    float s = 0.f;
    for (int b = 0; b < a.B; ++b)
      for (int m = 0; m < a.G; ++m) s += a.dpw_part[(((size_t)b * a.H + h) * a.G + m) * 68 + k];
    if (dpw) dpw[tid] = s;  // zeros without position bins (their partials are zero)
  }
  if (tid < a.H) {
    float s = 0.f;
    for (int b = 0; b < a.B; ++b)
      for (int m = 0; m < a.G; ++m) s += a.dw_part[((size_t)b * a.H + tid) * a.G + m];
    if (dw) dw[tid] = s;
  }
}

// ---------------------------------------------------------------------------
// ---------------------------------------------------------------------------
size_t sinkhorn_bwd_lds_bytes(int N, int DP, int elem, int G, int CH, bool stream) {
  return sinkhorn_bwd_lds_bytes_t(N, DP, elem, G, CH, stream);
}

hipError_t launch_sinkhorn_bwd(const SinkBwdArgs& a, bool bf16_in, int DP, size_t lds, hipStream_t stream,
                               bool coop) {
  return launch_bwd_mode<false>(a, bf16_in, DP, lds, stream, coop);
}

template <typename T, int DP>
static hipError_t launch_prep_t(const SinkBwdArgs& a, hipStream_t stream) {
  const size_t Np = ((a.N + 31) / 32) * 32;
  const size_t threads = (size_t)a.B * a.H * Np * DP;  // multiple of 1024
  hipLaunchKernelGGL((sinkhorn_bwd_prep_kernel<T, DP>), dim3((unsigned)(threads / 256)), dim3(256), 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_sinkhorn_bwd_prep(const SinkBwdArgs& a, bool bf16_in, int DP, hipStream_t stream) {
  if (bf16_in) {
    if (DP == 32) return launch_prep_t<bf16, 32>(a, stream);
    if (DP == 64) return launch_prep_t<bf16, 64>(a, stream);
  } else {
    if (DP == 32) return launch_prep_t<float, 32>(a, stream);
    if (DP == 64) return launch_prep_t<float, 64>(a, stream);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_sinkhorn_bwd_finalize(const SinkBwdArgs& a, float* dx, float* dpw, float* dw, hipStream_t stream) {
  const int total = std::max(a.B * a.N * 3, a.H * 68);
  const int threads = 256;
  const int blocks = (total + threads - 1) / threads;
  hipLaunchKernelGGL(sinkhorn_bwd_finalize_kernel, dim3(blocks), dim3(threads), 0, stream, a, dx, dpw, dw);
  return hipGetLastError();
}

}  // namespace dfl
