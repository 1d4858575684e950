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
    if (ok) s = ordered_sum(a.dx_part + ((size_t)b * a.H * a.N) * 3 + rem, (size_t)a.N * 3, a.H, 0.f);
    dx[tid] = s;
  }
  if (tid < a.H * 68) {
    const int h = tid / 68, k = tid % 68;
    float s = 0.f;
    for (int b = 0; b < a.B; ++b)
      s = ordered_sum(a.dpw_part + (((size_t)b * a.H + h) * a.G) * 68 + k, 68, a.G, s);
    if (dpw) dpw[tid] = s;  // zeros without position bins (their partials are zero)
  }
  if (tid < a.H) {
    float s = 0.f;
    for (int b = 0; b < a.B; ++b) s = ordered_sum(a.dw_part + ((size_t)b * a.H + tid) * a.G, 1, a.G, s);
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

// The cost bias of every (b,h), once per backward call, in the backward's sweep
// orientations: mat[bh][i][j] = bias(i, j) and matT[bh][i][j] = bias(j, i), i, j < Np,
// from Bias::quads with the coordinates and tables a backward workgroup stages (x of
// rows below the batch row's last valid token, else 0), so the sweeps read exactly the
// values they would compute.  Block: 16 rows i of one (b,h); thread: 4 columns at a time.
constexpr int BIAS_ROWS = 16;
__global__ void __launch_bounds__(256) bias_mat_kernel(SinkBwdArgs a, float* mat, float* matT) {
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ float posw[BIN_NONE + 1];
  __shared__ int s_tmp;
  const int N = a.N, Np = ((N + 31) / 32) * 32;
  const int bh = blockIdx.y, b = bh / a.H, h = bh % a.H;
  float* xs = reinterpret_cast<float*>(smem);                       // [Np][3]
  unsigned char* valid = smem + (size_t)Np * 3 * sizeof(float);     // [Np]
  const int n = mask_setup(a.mask ? a.mask + (size_t)b * N : nullptr, N, valid, &s_tmp);
  const float eps = a.eps[h];
  const float w_h = a.w_dist ? a.w_dist[h] : 0.f;
  const bool use_geo = a.x != nullptr && w_h != 0.f;
  const bool use_pos = a.bins8 != nullptr && a.pos_w != nullptr;
  for (int k = threadIdx.x; k <= (int)BIN_NONE; k += blockDim.x)
    posw[k] = (use_pos && k < (int)BIN_NONE) ? -LOG2E * a.pos_w[h * 68 + k] / eps : 0.f;
  for (int e = threadIdx.x; e < 3 * Np; e += blockDim.x) {
    const int i = e / 3, c = e - 3 * i;
    xs[e] = (a.x && i < n) ? a.x[((size_t)b * N + i) * 3 + c] : 0.f;
  }
  __syncthreads();
  Bias bias;
  bias.b8 = use_pos ? a.bins8 + (size_t)b * Np * Np : nullptr;
  bias.b8t = use_pos ? a.bins8t + (size_t)b * Np * Np : nullptr;
  bias.posw = posw;
  bias.xs = use_geo ? xs : nullptr;
  bias.geo_scale = -LOG2E * w_h / eps;
  bias.r0 = a.r0;
  bias.Np = Np;
  // Bias::quads itself in both orientations (a distance evaluated separately and added
  // afterwards would round differently from the fused form the sweeps use)
  const int q4 = Np / 4;
  for (int e = threadIdx.x; e < BIAS_ROWS * q4; e += blockDim.x) {
    const int i = blockIdx.x * BIAS_ROWS + e / q4, j0 = 4 * (e % q4);
    if (i >= Np) break;
    const int s0[1] = {j0};
    f32x4 o[1], ot[1];
    bias.template quads<false, 1>(i, s0, o);
    bias.template quads<true, 1>(i, s0, ot);
    const size_t off = ((size_t)bh * Np + i) * Np + j0;
    *reinterpret_cast<f32x4*>(mat + off) = o[0];
    *reinterpret_cast<f32x4*>(matT + off) = ot[0];
  }
}

hipError_t launch_bias_mat(const SinkBwdArgs& a, float* mat, float* matT, hipStream_t stream) {
  const int Np = ((a.N + 31) / 32) * 32;
  const size_t lds = (size_t)Np * 3 * sizeof(float) + Np;
  hipError_t e = set_lds_limit((const void*)bias_mat_kernel, lds);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(bias_mat_kernel, dim3((unsigned)((Np + BIAS_ROWS - 1) / BIAS_ROWS), (unsigned)(a.B * a.H)),
                     dim3(256), lds, stream, a, mat, matT);
  return hipGetLastError();
}

hipError_t launch_sinkhorn_bwd_finalize(const SinkBwdArgs& a, float* dx, float* dpw, float* dw, hipStream_t stream) {
  const int total = std::max(a.B * a.N * 3, a.H * 68);
  const int threads = 256;
  const int blocks = (total + threads - 1) / threads;
  hipLaunchKernelGGL(sinkhorn_bwd_finalize_kernel, dim3(blocks), dim3(threads), 0, stream, a, dx, dpw, dw);
  return hipGetLastError();
}

}  // namespace dfl
