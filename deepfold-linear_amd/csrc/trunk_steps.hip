// The TokenOTBlock steps either side of the balanced transport
// (src/deepfold/model/trunk_block.py):
//
//   before (:165-175)  h_s = LayerNorm(h); Q_s, K_s, V_s = h_s W_q^T, h_s W_k^T, h_s W_v^T;
//                      Q_s, K_s L2-normalised per head (F.normalize, eps 1e-12).  One fused
//                      kernel: the LayerNorm of a 64-token block goes to LDS, the projection
//                      runs on MFMA against weight rows streamed from L2, and the head norms
//                      are taken in the epilogue.  The outputs are (M, C) = (B, N, H, d) fp32,
//                      which the transport's C ABI reads in place through its strides.
//   after (:189-204)   x <- x + mask * sigmoid(w_gate . LN_gate(h) + b) * sum_h tanh(lam_h)/H (x_c,h - x).
//                      One wave per token.
//
// Backward: normalisation backward (elementwise, per head), the weight and input
// gradients as fp32 MFMA GEMMs over LDS-staged tiles, LayerNorm backward; parameter
// gradients are summed over tokens in per-workgroup partials, then in a fixed order.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>

#include "common.h"
#include "trunk_args.h"

namespace dfl {

constexpr int TS_NT = 256;          // threads of every kernel here (4 waves)
constexpr int TS_PARTS = 64;        // workgroups of the per-token kernels (partials rows)
constexpr float TS_LN_EPS = 1e-5f;  // nn.LayerNorm default
constexpr float TS_NORM_EPS = 1e-12f;  // F.normalize default
constexpr int TS_MAXE = 16;         // C / 64 elements per lane (C <= 1024)

template <typename T> constexpr int xs_pad() { return 16 / (int)sizeof(T); }

size_t proj_fwd_lds_bytes(int C, bool bf16_in) {
  const int e = bf16_in ? 2 : 4;
  return (size_t)64 * (C + 16 / e) * e;
}

// ---------------------------------------------------------------------------
// Forward projections.  Grid (ceil(M/64), C/64, n_proj); workgroup = 64 tokens x 64
// output columns of projection p; wave w owns columns [o0 + 16w, o0 + 16w + 16) for all
// 64 tokens (4 MFMA tiles), so its weight fragment is loaded once per k-step and the
// LayerNorm'd token fragments come from LDS.
template <typename T>
__global__ void __launch_bounds__(TS_NT) proj_fwd_kernel(ProjArgs a) {
  using M = Mfma<T, 32>;
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ float ss_l[4][64];
  T* xs = reinterpret_cast<T*>(smem);
  const int C = a.C, ldx = C + xs_pad<T>();
  const int m0 = blockIdx.x * 64, o0 = blockIdx.y * 64, p = blockIdx.z;
  const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE, g = lane >> 4;
  const T* h = static_cast<const T*>(a.h);
  const int E = C / 64;

  // LayerNorm of the block's rows (biased variance, as nn.LayerNorm)
  for (int r = wave; r < 64; r += 4) {
    const int m = m0 + r;
    float v[TS_MAXE];
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < TS_MAXE; ++e) {
      v[e] = (e < E && m < a.M) ? to_f32(h[(size_t)m * C + e * 64 + lane]) : 0.f;
      s += v[e];
    }
    const float mean = wave_sum(s) / C;
    float q = 0.f;
#pragma unroll
    for (int e = 0; e < TS_MAXE; ++e)
      if (e < E) q += (v[e] - mean) * (v[e] - mean);
    const float rstd = rsqrtf(wave_sum(q) / C + TS_LN_EPS);
#pragma unroll
    for (int e = 0; e < TS_MAXE; ++e)
      if (e < E) {
        const int c = e * 64 + lane;
        const float y = m < a.M ? (v[e] - mean) * rstd * a.ln_w[c] + a.ln_b[c] : 0.f;
        xs[(size_t)r * ldx + c] = from_f32<T>(y);
      }
    if (p == 0 && blockIdx.y == 0 && lane == 0 && m < a.M) {
      a.mean[m] = mean;
      a.rstd[m] = rstd;
    }
  }
  __syncthreads();

  // projection: lane holds token 16t + l%16, output columns o0 + 16w + 4g + e
  const T* W = static_cast<const T*>(a.w[p]);
  const T* wrow = W + (size_t)(o0 + 16 * wave + (lane & 15)) * C;
  f32x4 acc[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll 4  // C % 128 == 0 is not required: the remainder loop handles C = 64 (mod 128)
  for (int kc = 0; kc < C; kc += 32) {
    typename M::Frag wf;
    M::load(wf, wrow + kc, lane);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      typename M::Frag xf;
      M::load(xf, xs + (size_t)(16 * t + (lane & 15)) * ldx + kc, lane);
      acc[t] = M::qk(wf, xf, acc[t]);
    }
  }

  // per-head norms of q and k: head = dh consecutive columns, i.e. dh/16 waves
  const int dh = C / a.H;
  float scale[4] = {1.f, 1.f, 1.f, 1.f}, nrm[4] = {0.f, 0.f, 0.f, 0.f};
  if (p < 2) {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      float s = acc[t][0] * acc[t][0] + acc[t][1] * acc[t][1] + acc[t][2] * acc[t][2] + acc[t][3] * acc[t][3];
      s = sum_groups(s);
      if (g == 0) ss_l[wave][16 * t + lane] = s;
    }
    __syncthreads();
    const int wph = dh / 16, w0 = (wave / wph) * wph;  // waves of this head
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      float s = 0.f;
      for (int w = w0; w < w0 + wph; ++w) s += ss_l[w][16 * t + (lane & 15)];
      nrm[t] = sqrtf(s);
      scale[t] = 1.f / fmaxf(nrm[t], TS_NORM_EPS);
    }
  }
  float* y = a.y[p];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const int m = m0 + 16 * t + (lane & 15);
    if (m >= a.M) continue;
    const int o = o0 + 16 * wave + 4 * g;
    const f32x4 out = {acc[t][0] * scale[t], acc[t][1] * scale[t], acc[t][2] * scale[t], acc[t][3] * scale[t]};
    *reinterpret_cast<f32x4*>(y + (size_t)m * C + o) = out;
    if (p < 2 && g == 0 && (16 * wave) % dh == 0) a.norm[p][(size_t)m * a.H + (o0 + 16 * wave) / dh] = nrm[t];
  }
}

// ---------------------------------------------------------------------------
// Backward of y = u / max(|u|, eps) per head: du = (dy - y (y . dy)) / |u| where
// |u| > eps, else dy / eps.  One thread per element of projection blockIdx.y; the dh
// lanes of a head are consecutive (C % 64 == 0, dh | 64).
__global__ void __launch_bounds__(TS_NT) proj_dnorm_kernel(ProjArgs a) {
  const size_t t = (size_t)blockIdx.x * TS_NT + threadIdx.x;
  const int p = blockIdx.y;
  if (t >= (size_t)a.M * a.C) return;  // M*C is a multiple of 64: whole waves leave
  const float dy = a.dy[p] ? a.dy[p][t] : 0.f;
  float du = dy;
  if (p < 2) {
    const int dh = a.C / a.H;
    const int m = (int)(t / a.C), c = (int)(t % a.C);
    const float y = a.y[p][t];
    float dot = y * dy;
    for (int s = 1; s < dh; s <<= 1) dot += __shfl_xor(dot, s);
    const float n = a.norm[p][(size_t)m * a.H + c / dh];
    du = n > TS_NORM_EPS ? (dy - y * dot) / n : dy / TS_NORM_EPS;
  }
  a.du[p][t] = du;
}

// LayerNorm output and normalised input, recomputed from the saved statistics.
template <typename T>
__global__ void __launch_bounds__(TS_NT) proj_ln_recompute_kernel(ProjArgs a) {
  const size_t t = (size_t)blockIdx.x * TS_NT + threadIdx.x;
  if (t >= (size_t)a.M * a.C) return;
  const int m = (int)(t / a.C), c = (int)(t % a.C);
  const float xn = (to_f32(static_cast<const T*>(a.h)[t]) - a.mean[m]) * a.rstd[m];
  a.xn[t] = xn;
  a.xa[t] = xn * a.ln_w[c] + a.ln_b[c];
}

// ---------------------------------------------------------------------------
// fp32 GEMM on MFMA (16x16x4 f32) for the backward's small products (M ~ 10^2-10^3
// tokens, C ~ 512): 32 x 32 output tiles (one 16 x 16 tile per wave), so that even
// M = 256 gives 128+ workgroups; k-steps of 64 staged in LDS in the row-over-k layout
// of Mfma<float, 64> (K-major operands transposed on the way in), with the next step's
// global loads issued before the current step's MFMAs.
constexpr int GB = 32;  // output tile edge
constexpr int GK = 64;  // k-step
constexpr int GQ = GB * GK / TS_NT;  // elements of one operand tile per thread (8)

template <bool KMAJ, typename TS>
__device__ __forceinline__ void gemm_fetch(float (&v)[GQ], const TS* __restrict__ src, long long ld, int r0, int k0,
                                           int nr, int kend) {
#pragma unroll
  for (int q = 0; q < GQ; ++q) {
    // consecutive threads walk the contiguous dimension of the source
    const int e = threadIdx.x + q * TS_NT;
    const int r = KMAJ ? (e % GB) : (e / GK);
    const int k = KMAJ ? (e / GB) : (e % GK);
    const int gr = r0 + r, gk = k0 + k;
    v[q] = (gr < nr && gk < kend) ? to_f32(KMAJ ? src[(size_t)gk * ld + gr] : src[(size_t)gr * ld + gk]) : 0.f;
  }
}
template <bool KMAJ>
__device__ __forceinline__ void gemm_put(float (*S)[GK + 4], const float (&v)[GQ]) {
#pragma unroll
  for (int q = 0; q < GQ; ++q) {
    const int e = threadIdx.x + q * TS_NT;
    const int r = KMAJ ? (e % GB) : (e / GK);
    const int k = KMAJ ? (e / GB) : (e % GK);
    S[r][k] = v[q];
  }
}

template <bool AK, bool BK, typename TB>
__global__ void __launch_bounds__(TS_NT) gemm_kernel(GemmArgs a) {
  using MF = Mfma<float, GK>;
  __shared__ __align__(16) float As[GB][GK + 4];
  __shared__ __align__(16) float Bs[GB][GK + 4];
  const int z = blockIdx.z;
  const int i0 = blockIdx.x * GB, j0 = blockIdx.y * GB;
  const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE, g = lane >> 4;
  const int ti = 16 * (wave >> 1), tj = 16 * (wave & 1);
  const int sps = (a.kseg + GK - 1) / GK, steps = a.nseg * sps;
  float va[GQ], vb[GQ];
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int t = 0; t < steps; ++t) {
    if (t == 0) {
      gemm_fetch<AK>(va, a.A[z], a.lda, i0, 0, a.m, a.kseg);
      gemm_fetch<BK>(vb, static_cast<const TB*>(a.B[z]), a.ldb, j0, 0, a.n, a.kseg);
    }
    gemm_put<AK>(As, va);
    gemm_put<BK>(Bs, vb);
    __syncthreads();
    if (t + 1 < steps) {  // next step's loads in flight during this step's MFMAs
      const int s = (t + 1) / sps, kl = (t + 1 - s * sps) * GK;
      gemm_fetch<AK>(va, a.A[z + s], a.lda, i0, kl, a.m, a.kseg);
      gemm_fetch<BK>(vb, static_cast<const TB*>(a.B[z + s]), a.ldb, j0, kl, a.n, a.kseg);
    }
    MF::Frag af, bf;
    MF::load(af, &As[ti + (lane & 15)][0], lane);
    MF::load(bf, &Bs[tj + (lane & 15)][0], lane);
    acc = MF::qk(bf, af, acc);  // lane: row ti + l%16, columns tj + 4g + e
    __syncthreads();
  }
  const int i = i0 + ti + (lane & 15);
  if (i >= a.m) return;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int j = j0 + tj + 4 * g + e;
    if (j < a.n) a.C[z][(size_t)i * a.ldc + j] = acc[e];
  }
}

// ---------------------------------------------------------------------------
// LayerNorm backward of the projection path: dh = rstd (g - mean(g) - xn mean(g xn)),
// g = dxa * w; per-workgroup partials of dln_w = sum dxa xn and dln_b = sum dxa.
__global__ void __launch_bounds__(TS_NT) proj_ln_bwd_kernel(ProjArgs a) {
  __shared__ float s_dw[1024], s_db[1024];
  const int C = a.C, E = C / 64;
  const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;
  for (int c = threadIdx.x; c < C; c += TS_NT) s_dw[c] = s_db[c] = 0.f;
  __syncthreads();
  float pw[TS_MAXE], pb[TS_MAXE];
#pragma unroll
  for (int e = 0; e < TS_MAXE; ++e) pw[e] = pb[e] = 0.f;
  for (int m = blockIdx.x * 4 + wave; m < a.M; m += gridDim.x * 4) {
    float gv[TS_MAXE], xv[TS_MAXE];
    float s1 = 0.f, s2 = 0.f;
#pragma unroll
    for (int e = 0; e < TS_MAXE; ++e) {
      gv[e] = xv[e] = 0.f;
      if (e < E) {
        const size_t t = (size_t)m * C + e * 64 + lane;
        const float gd = a.dxa[t];
        xv[e] = a.xn[t];
        gv[e] = gd * a.ln_w[e * 64 + lane];
        pw[e] += gd * xv[e];
        pb[e] += gd;
        s1 += gv[e];
        s2 += gv[e] * xv[e];
      }
    }
    const float a1 = wave_sum(s1) / C, a2 = wave_sum(s2) / C, r = a.rstd[m];
#pragma unroll
    for (int e = 0; e < TS_MAXE; ++e)
      if (e < E) a.dh[(size_t)m * C + e * 64 + lane] = r * (gv[e] - a1 - xv[e] * a2);
  }
#pragma unroll
  for (int e = 0; e < TS_MAXE; ++e)
    if (e < E) {
      atomicAdd(&s_dw[e * 64 + lane], pw[e]);
      atomicAdd(&s_db[e * 64 + lane], pb[e]);
    }
  __syncthreads();
  for (int c = threadIdx.x; c < C; c += TS_NT) {
    a.part[(size_t)blockIdx.x * 2 * C + c] = s_dw[c];
    a.part[(size_t)blockIdx.x * 2 * C + C + c] = s_db[c];
  }
}

// Column sums of the partial rows (rows split over the 4 waves, combined in a fixed
// order), scattered to the segments' outputs.  One thread column per lane.
__global__ void __launch_bounds__(TS_NT) sum_segs_kernel(SumSegs a) {
  __shared__ float red[4][WAVE];
  const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;
  const int c = blockIdx.x * WAVE + lane;
  float s = 0.f;
  if (c < a.width)
    for (int r = wave; r < a.rows; r += 4) s += a.part[(size_t)r * a.width + c];
  red[wave][lane] = s;
  __syncthreads();
  if (wave != 0 || c >= a.width) return;
  const float tot = (red[0][lane] + red[1][lane]) + (red[2][lane] + red[3][lane]);
  for (int sg = 0; sg < a.nseg; ++sg)
    if (c >= a.off[sg] && c < a.off[sg] + a.n[sg] && a.out[sg]) a.out[sg][c - a.off[sg]] = tot;
}

// ---------------------------------------------------------------------------
// Gated coordinate update, one wave per token (grid-stride).
template <typename T, bool BWD>
__global__ void __launch_bounds__(TS_NT) coord_kernel(CoordArgs a) {
  __shared__ float s_red[3 * 1024 + 64 + 1];
  const int C = a.C, E = C / 64, H = a.H;
  const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;
  const int width = 3 * C + H + 1;  // dw_gate | dln_w | dln_b | dlam_raw | db_gate
  if (BWD) {
    for (int c = threadIdx.x; c < width; c += TS_NT) s_red[c] = 0.f;
    __syncthreads();
  }
  float p_wg[TS_MAXE], p_lw[TS_MAXE], p_lb[TS_MAXE];
#pragma unroll
  for (int e = 0; e < TS_MAXE; ++e) p_wg[e] = p_lw[e] = p_lb[e] = 0.f;
  float p_lam = 0.f, p_b = 0.f;
  const T* h = static_cast<const T*>(a.h);
  const int NT = a.B * a.N;
  for (int tok = blockIdx.x * 4 + wave; tok < NT; tok += gridDim.x * 4) {
    const int b = tok / a.N, n = tok - b * a.N;
    float xv[TS_MAXE];
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < TS_MAXE; ++e) {
      xv[e] = e < E ? to_f32(h[(size_t)tok * C + e * 64 + lane]) : 0.f;
      s += xv[e];
    }
    const float mean = wave_sum(s) / C;
    float q = 0.f;
#pragma unroll
    for (int e = 0; e < TS_MAXE; ++e)
      if (e < E) q += (xv[e] - mean) * (xv[e] - mean);
    const float rstd = rsqrtf(wave_sum(q) / C + TS_LN_EPS);
    float z = 0.f;
#pragma unroll
    for (int e = 0; e < TS_MAXE; ++e)
      if (e < E) {
        const int c = e * 64 + lane;
        xv[e] = (xv[e] - mean) * rstd;  // normalised input
        z += (xv[e] * a.ln_w[c] + a.ln_b[c]) * a.w_gate[c];
      }
    z = wave_sum(z) + a.b_gate[0];
    const float gate = 1.f / (1.f + __expf(-z));
    const float mk = a.mask ? a.mask[tok] : 1.f;
    const float* xt = a.x + (size_t)tok * 3;
    const float x0 = xt[0], x1 = xt[1], x2 = xt[2];
    // lane hd < H carries head hd
    float th = 0.f, d0 = 0.f, d1 = 0.f, d2 = 0.f;
    if (lane < H) {
      th = tanhf(a.lam_raw[lane]);
      const float* c = a.xc + (((size_t)b * H + lane) * a.N + n) * 3;
      d0 = c[0] - x0;
      d1 = c[1] - x1;
      d2 = c[2] - x2;
    }
    const float lam = th / H;
    const float w0 = wave_sum(lam * d0), w1 = wave_sum(lam * d1), w2 = wave_sum(lam * d2);
    const float mg = mk * gate;
    if (!BWD) {
      if (lane < 3) {
        const float w = lane == 0 ? w0 : (lane == 1 ? w1 : w2);
        a.x_out[(size_t)tok * 3 + lane] = xt[lane] + mg * w;
      }
      continue;
    }
    const float* go = a.dx_out + (size_t)tok * 3;
    const float g0 = go[0], g1 = go[1], g2 = go[2];
    const float L = wave_sum(lam);
    if (lane < 3) {
      const float gl = lane == 0 ? g0 : (lane == 1 ? g1 : g2);
      a.dx[(size_t)tok * 3 + lane] = gl * (1.f - mg * L);
    }
    if (lane < H) {
      float* c = a.dxc + (((size_t)b * H + lane) * a.N + n) * 3;
      c[0] = g0 * mg * lam;
      c[1] = g1 * mg * lam;
      c[2] = g2 * mg * lam;
      p_lam += mg * (g0 * d0 + g1 * d1 + g2 * d2) * (1.f - th * th) / H;
    }
    const float dz = mk * (g0 * w0 + g1 * w1 + g2 * w2) * gate * (1.f - gate);
    p_b += dz;
    float s1 = 0.f, s2 = 0.f, gv[TS_MAXE];
#pragma unroll
    for (int e = 0; e < TS_MAXE; ++e) {
      gv[e] = 0.f;
      if (e < E) {
        const int c = e * 64 + lane;
        const float dl = dz * a.w_gate[c];  // gradient of the LayerNorm output
        p_wg[e] += dz * (xv[e] * a.ln_w[c] + a.ln_b[c]);
        p_lw[e] += dl * xv[e];
        p_lb[e] += dl;
        gv[e] = dl * a.ln_w[c];
        s1 += gv[e];
        s2 += gv[e] * xv[e];
      }
    }
    const float a1 = wave_sum(s1) / C, a2 = wave_sum(s2) / C;
#pragma unroll
    for (int e = 0; e < TS_MAXE; ++e)
      if (e < E) a.dh[(size_t)tok * C + e * 64 + lane] = rstd * (gv[e] - a1 - xv[e] * a2);
  }
  if (BWD) {
#pragma unroll
    for (int e = 0; e < TS_MAXE; ++e)
      if (e < E) {
        atomicAdd(&s_red[e * 64 + lane], p_wg[e]);
        atomicAdd(&s_red[C + e * 64 + lane], p_lw[e]);
        atomicAdd(&s_red[2 * C + e * 64 + lane], p_lb[e]);
      }
    if (lane < H) atomicAdd(&s_red[3 * C + lane], p_lam);
    if (lane == 0) atomicAdd(&s_red[3 * C + H], p_b);
    __syncthreads();
    for (int c = threadIdx.x; c < width; c += TS_NT) a.part[(size_t)blockIdx.x * width + c] = s_red[c];
  }
}

// ---------------------------------------------------------------------------
// Launchers.
static hipError_t sum_segs(const SumSegs& g, hipStream_t s) {
  hipLaunchKernelGGL(sum_segs_kernel, dim3((unsigned)((g.width + WAVE - 1) / WAVE)), dim3(TS_NT), 0, s, g);
  return hipGetLastError();
}

hipError_t launch_proj_fwd(const ProjArgs& a, bool bf16_in, hipStream_t s) {
  const size_t lds = proj_fwd_lds_bytes(a.C, bf16_in);
  const dim3 grid((unsigned)((a.M + 63) / 64), (unsigned)(a.C / 64), a.w[2] ? 3u : 2u);
  if (bf16_in) {
    hipError_t e = set_lds_limit((const void*)proj_fwd_kernel<bf16>, lds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(proj_fwd_kernel<bf16>, grid, dim3(TS_NT), lds, s, a);
  } else {
    hipError_t e = set_lds_limit((const void*)proj_fwd_kernel<float>, lds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(proj_fwd_kernel<float>, grid, dim3(TS_NT), lds, s, a);
  }
  return hipGetLastError();
}

template <bool AK, bool BK, typename TB>
static hipError_t gemm(const GemmArgs& g, int batch, hipStream_t s) {
  hipLaunchKernelGGL((gemm_kernel<AK, BK, TB>), dim3((unsigned)((g.m + GB - 1) / GB), (unsigned)((g.n + GB - 1) / GB),
                     (unsigned)batch), dim3(TS_NT), 0, s, g);
  return hipGetLastError();
}

hipError_t launch_proj_bwd(const ProjArgs& a, bool bf16_in, hipStream_t s) {
  const int np = a.w[2] ? 3 : 2;
  const size_t tot = (size_t)a.M * a.C;
  const unsigned blocks = (unsigned)((tot + TS_NT - 1) / TS_NT);
  hipLaunchKernelGGL(proj_dnorm_kernel, dim3(blocks, (unsigned)np), dim3(TS_NT), 0, s, a);
  if (bf16_in) hipLaunchKernelGGL(proj_ln_recompute_kernel<bf16>, dim3(blocks), dim3(TS_NT), 0, s, a);
  else hipLaunchKernelGGL(proj_ln_recompute_kernel<float>, dim3(blocks), dim3(TS_NT), 0, s, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  // dxa (M x C) = sum_p du_p (M x C, row layout over o) . W_p (o-major: a K-major operand)
  GemmArgs gx;
  memset(&gx, 0, sizeof(gx));
  for (int p = 0; p < np; ++p) {
    gx.A[p] = a.du[p];
    gx.B[p] = a.w[p];
  }
  gx.C[0] = a.dxa;
  gx.lda = gx.ldb = gx.ldc = a.C;
  gx.m = a.M; gx.n = a.C; gx.kseg = a.C; gx.nseg = np;
  e = bf16_in ? gemm<false, true, bf16>(gx, 1, s) : gemm<false, true, float>(gx, 1, s);
  if (e != hipSuccess) return e;
  // dW_p (C x C) = du_p^T . xa (both operands token-major), one launch for the requested ones
  GemmArgs gw;
  memset(&gw, 0, sizeof(gw));
  int nw = 0;
  for (int p = 0; p < np; ++p)
    if (a.dw[p]) {
      gw.A[nw] = a.du[p];
      gw.B[nw] = a.xa;
      gw.C[nw] = a.dw[p];
      ++nw;
    }
  gw.lda = gw.ldb = gw.ldc = a.C;
  gw.m = a.C; gw.n = a.C; gw.kseg = a.M; gw.nseg = 1;
  if (nw > 0 && (e = gemm<true, true, float>(gw, nw, s)) != hipSuccess) return e;
  hipLaunchKernelGGL(proj_ln_bwd_kernel, dim3(TS_PARTS), dim3(TS_NT), 0, s, a);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  SumSegs sg;
  memset(&sg, 0, sizeof(sg));
  sg.part = a.part; sg.rows = TS_PARTS; sg.width = 2 * a.C; sg.nseg = 2;
  sg.off[0] = 0; sg.n[0] = a.C; sg.out[0] = a.dln_w;
  sg.off[1] = a.C; sg.n[1] = a.C; sg.out[1] = a.dln_b;
  return sum_segs(sg, s);
}

hipError_t launch_coord(const CoordArgs& a, bool bf16_in, bool bwd, hipStream_t s) {
  const int tokens = a.B * a.N;
  const unsigned blocks = (unsigned)std::min(TS_PARTS, (tokens + 3) / 4);
  if (bwd) {
    if (bf16_in) hipLaunchKernelGGL((coord_kernel<bf16, true>), dim3(TS_PARTS), dim3(TS_NT), 0, s, a);
    else hipLaunchKernelGGL((coord_kernel<float, true>), dim3(TS_PARTS), dim3(TS_NT), 0, s, a);
  } else {
    if (bf16_in) hipLaunchKernelGGL((coord_kernel<bf16, false>), dim3(blocks), dim3(TS_NT), 0, s, a);
    else hipLaunchKernelGGL((coord_kernel<float, false>), dim3(blocks), dim3(TS_NT), 0, s, a);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || !bwd) return e;
  const int C = a.C, H = a.H;
  SumSegs sg;
  memset(&sg, 0, sizeof(sg));
  sg.part = a.part; sg.rows = TS_PARTS; sg.width = 3 * C + H + 1; sg.nseg = 5;
  const int off[5] = {0, C, 2 * C, 3 * C, 3 * C + H}, n[5] = {C, C, C, H, 1};
  float* out[5] = {a.dw_gate, a.dln_w, a.dln_b, a.dlam_raw, a.db_gate};
  for (int i = 0; i < 5; ++i) {
    sg.off[i] = off[i];
    sg.n[i] = n[i];
    sg.out[i] = out[i];
  }
  return sum_segs(sg, s);
}

}  // namespace dfl
