// Dense, materialised-cost Sinkhorn on gfx950: the restatement of
// vv137/deepfold-linear src/deepfold/model/sinkhorn.py.
//
//   sinkhorn_solve (:17-112)            K log-domain UOT iterations on a given cost
//                                       C (B,H,N,N): u = kappa (log mu - LSE_j(L + v + cb)),
//                                       v = kappa (log nu - LSE_i(L + u + rb)), L = -C/eps,
//                                       masks as -1e9 biases, early stop on the L-inf change;
//                                       backward = autograd through the executed iterations.
//   compute_transport_output (:115-198) T_norm = exp(ls - max)/(sum + 1e-6), O = T_norm V,
//                                       sigmoid gate, EGNN centroid; backward of those ops.
//
// Every pass streams C (or T_norm / dC) once, so all kernels are bound by
// HBM / Infinity-cache bandwidth; fp32 throughout (the reference's dtype).
// Row passes: one wave per row, lanes stride the columns (coalesced).
// Column passes: one 256-thread workgroup per 64 columns, lane = column, the
// four waves split the rows and combine in LDS (coalesced row segments, no
// transposed copy of C).
#include "dense_args.h"
#include "common.h"

#include <algorithm>

namespace dfl {

constexpr int DN_NT = 256;
constexpr int DN_NW = DN_NT / WAVE;
constexpr float MASK_BIAS = -1e9f;  // sinkhorn.py:79-80, 151

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x = fmaxf(x, __shfl_xor(x, o, WAVE));
  return x;
}
__device__ __forceinline__ float mask_bias(const float* mask, int b, int N, int j) {
  return mask ? (1.f - mask[(size_t)b * N + j]) * MASK_BIAS : 0.f;
}
// |x| as ordered bits for an atomic max over non-negative floats (NaN -> +inf bits)
__device__ __forceinline__ unsigned abs_bits(float x) {
  const float a = fabsf(x);
  return a == a ? __float_as_uint(a) : 0x7f800000u;
}

// ---------------------------------------------------------------------------
// Row update of iteration k: r_i = LSE_j(-C_ij/eps + v_j + cb_j), u_i = kappa (log mu_i - r_i).
// One wave per row; 4 rows per workgroup.  v = hist_v[k-1]; writes hist_r[k], hist_u[k].
__global__ void __launch_bounds__(DN_NT) dense_row_update_kernel(DenseSinkArgs a, int k) {
  const int lane = threadIdx.x & (WAVE - 1);
  const size_t row = (size_t)blockIdx.x * DN_NW + threadIdx.x / WAVE;  // (bh, i)
  const int N = a.N;
  const size_t BHN = (size_t)a.B * a.H * N;
  if (row >= BHN) return;
  const int bh = (int)(row / N), i = (int)(row % N), b = bh / a.H, h = bh % a.H;
  const float eps = a.eps[h];
  const float kappa = a.lam / (a.lam + eps);
  const float* Cr = a.C + row * N;
  const float* v = a.hist_v + (size_t)(k - 1) * BHN + (size_t)bh * N;
  float m = -INFINITY, s = 0.f;
  for (int j = lane; j < N; j += WAVE) {
    const float x = -Cr[j] / eps + v[j] + mask_bias(a.mask, b, N, j);
    const float mn = fmaxf(m, x);
    s = s * __expf(m - mn) + __expf(x - mn);
    m = mn;
  }
  const float mm = wave_max(m);
  const float ss = wave_sum(s * __expf(m - mm));
  if (lane == 0) {
    const float r = mm + __logf(ss);
    const float u = kappa * (a.log_mu[row] - r);
    a.hist_r[(size_t)k * BHN + row] = r;
    a.hist_u[(size_t)k * BHN + row] = u;
    if (a.delta) atomicMax(a.delta + 2 * k, abs_bits(u - a.hist_u[(size_t)(k - 1) * BHN + row]));
  }
}

// Column update of iteration k: c_j = LSE_i(-C_ij/eps + u_i + rb_i), v_j = kappa (log nu_j - c_j).
// Workgroup per 64 columns of one (b,h); wave w takes rows w, w + 4, ...
__global__ void __launch_bounds__(DN_NT) dense_col_update_kernel(DenseSinkArgs a, int k) {
  __shared__ float s_m[DN_NW][WAVE], s_s[DN_NW][WAVE];
  const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;
  const int N = a.N;
  const int nblk = (N + WAVE - 1) / WAVE;
  const int bh = blockIdx.x / nblk, j = (blockIdx.x % nblk) * WAVE + lane;
  const int b = bh / a.H, h = bh % a.H;
  const size_t BHN = (size_t)a.B * a.H * N;
  const float eps = a.eps[h];
  const float kappa = a.lam / (a.lam + eps);
  const float* Cb = a.C + (size_t)bh * N * N;
  const float* u = a.hist_u + (size_t)k * BHN + (size_t)bh * N;
  float m = -INFINITY, s = 0.f;
  if (j < N)
    for (int i = wave; i < N; i += DN_NW) {
      const float x = -Cb[(size_t)i * N + j] / eps + u[i] + mask_bias(a.mask, b, N, i);
      const float mn = fmaxf(m, x);
      s = s * __expf(m - mn) + __expf(x - mn);
      m = mn;
    }
  s_m[wave][lane] = m;
  s_s[wave][lane] = s;
  __syncthreads();
  if (wave == 0 && j < N) {
    float mm = -INFINITY;
#pragma unroll
    for (int w = 0; w < DN_NW; ++w) mm = fmaxf(mm, s_m[w][lane]);
    float ss = 0.f;
#pragma unroll
    for (int w = 0; w < DN_NW; ++w) ss += s_s[w][lane] * __expf(s_m[w][lane] - mm);
    const float c = mm + __logf(ss);
    const size_t col = (size_t)bh * N + j;
    const float vv = kappa * (a.log_nu[col] - c);
    a.hist_c[(size_t)k * BHN + col] = c;
    a.hist_v[(size_t)k * BHN + col] = vv;
    if (a.delta) atomicMax(a.delta + 2 * k + 1, abs_bits(vv - a.hist_v[(size_t)(k - 1) * BHN + col]));
  }
}

// Final potentials (masked) and the iteration-0 entries of the history.
__global__ void dense_init_kernel(DenseSinkArgs a) {
  const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const size_t BHN = (size_t)a.B * a.H * a.N;
  if (t < BHN) {
    a.hist_u[t] = a.u_init ? a.u_init[t] : 0.f;
    a.hist_v[t] = a.v_init ? a.v_init[t] : 0.f;
  }
  if (a.delta && t < (size_t)2 * (a.K + 1)) a.delta[t] = 0u;
}
__global__ void dense_finish_kernel(DenseSinkArgs a, int k) {
  const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const size_t BHN = (size_t)a.B * a.H * a.N;
  if (t >= BHN) return;
  const int bh = (int)(t / a.N), i = (int)(t % a.N), b = bh / a.H;
  const float mk = a.mask ? a.mask[(size_t)b * a.N + i] : 1.f;
  a.log_u[t] = a.hist_u[(size_t)k * BHN + t] * mk;
  a.log_v[t] = a.hist_v[(size_t)k * BHN + t] * mk;
}

// ---------------------------------------------------------------------------
// Backward of iteration k (autograd through the executed iterations).
// Row pass, one wave per row i, with bvec = -kappa g_v(k) (all j):
//   P_col_ij = exp(L_ij + u_k,i + rb_i - c_k,j),   t_i = sum_j P_col_ij bvec_j
//   g_u(k)_i = [k == K] g_up_u_i + t_i,  avec_i = -kappa g_u(k)_i
//   P_row_ij = exp(L_ij + v_{k-1},j + cb_j - r_k,i)
//   dL_ij += P_col_ij bvec_j + P_row_ij avec_i;   d log mu_i += kappa g_u(k)_i
// dL accumulates in dC; the pass of k = 1 writes the final dC = -dL / eps.
__global__ void __launch_bounds__(DN_NT) dense_bwd_row_kernel(DenseSinkBwdArgs a, int k) {
  const int lane = threadIdx.x & (WAVE - 1);
  const size_t row = (size_t)blockIdx.x * DN_NW + threadIdx.x / WAVE;
  const int N = a.N;
  const size_t BHN = (size_t)a.B * a.H * N;
  if (row >= BHN) return;
  const int bh = (int)(row / N), i = (int)(row % N), b = bh / a.H, h = bh % a.H;
  const float eps = a.eps[h];
  const float kappa = a.lam / (a.lam + eps);
  const float* Cr = a.C + row * N;
  float* dCr = a.dC + row * N;
  const float* ck = a.hist_c + (size_t)k * BHN + (size_t)bh * N;
  const float* vprev = a.hist_v + (size_t)(k - 1) * BHN + (size_t)bh * N;
  const float* gv = a.gv + (size_t)bh * N;
  const float uk = a.hist_u[(size_t)k * BHN + row];
  const float rk = a.hist_r[(size_t)k * BHN + row];
  const float rb = mask_bias(a.mask, b, N, i);
  // t_i
  float t = 0.f;
  for (int j = lane; j < N; j += WAVE) {
    const float L = -Cr[j] / eps;
    t += __expf(L + uk + rb - ck[j]) * (-kappa * gv[j]);
  }
  t = wave_sum(t);
  const float gu = (k == a.K && a.grad_u ? a.grad_u[row] * (a.mask ? a.mask[(size_t)b * N + i] : 1.f) : 0.f) + t;
  const float av = -kappa * gu;
  const bool first = k == a.K, last = k == 1;
  const float inv_eps = 1.f / eps;
  for (int j = lane; j < N; j += WAVE) {
    const float L = -Cr[j] / eps;
    const float pc = __expf(L + uk + rb - ck[j]);
    const float pr = __expf(L + vprev[j] + mask_bias(a.mask, b, N, j) - rk);
    float dl = pc * (-kappa * gv[j]) + pr * av;
    if (!first) dl += dCr[j];
    dCr[j] = last ? -dl * inv_eps : dl;
  }
  if (lane == 0) {
    a.avec[row] = av;
    const float dmu = kappa * gu;
    a.dlog_mu[row] = first ? dmu : a.dlog_mu[row] + dmu;
  }
}

// Column pass of iteration k: g_v(k-1)_j = sum_i P_row_ij avec_i, d log nu_j += kappa g_v(k)_j.
__global__ void __launch_bounds__(DN_NT) dense_bwd_col_kernel(DenseSinkBwdArgs a, int k) {
  __shared__ float s_t[DN_NW][WAVE];
  const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;
  const int N = a.N;
  const int nblk = (N + WAVE - 1) / WAVE;
  const int bh = blockIdx.x / nblk, j = (blockIdx.x % nblk) * WAVE + lane;
  const int b = bh / a.H, h = bh % a.H;
  const size_t BHN = (size_t)a.B * a.H * N;
  const float eps = a.eps[h];
  const float kappa = a.lam / (a.lam + eps);
  const float* Cb = a.C + (size_t)bh * N * N;
  const float* rk = a.hist_r + (size_t)k * BHN + (size_t)bh * N;
  const float* av = a.avec + (size_t)bh * N;
  float t = 0.f;
  if (j < N) {
    const float vj = a.hist_v[(size_t)(k - 1) * BHN + (size_t)bh * N + j] + mask_bias(a.mask, b, N, j);
    for (int i = wave; i < N; i += DN_NW) t += __expf(-Cb[(size_t)i * N + j] / eps + vj - rk[i]) * av[i];
  }
  s_t[wave][lane] = t;
  __syncthreads();
  if (wave == 0 && j < N) {
    float tt = 0.f;
#pragma unroll
    for (int w = 0; w < DN_NW; ++w) tt += s_t[w][lane];
    const size_t col = (size_t)bh * N + j;
    const float gvk = a.gv[col];
    const float dnu = kappa * gvk;
    a.dlog_nu[col] = k == a.K ? dnu : a.dlog_nu[col] + dnu;
    a.gv[col] = tt;  // g_v(k-1)
  }
}

// g_v(K) = grad_v * mask into the workspace vector.
__global__ void dense_bwd_init_kernel(DenseSinkBwdArgs a) {
  const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const size_t BHN = (size_t)a.B * a.H * a.N;
  if (t >= BHN) return;
  const int bh = (int)(t / a.N), i = (int)(t % a.N), b = bh / a.H;
  const float mk = a.mask ? a.mask[(size_t)b * a.N + i] : 1.f;
  a.gv[t] = a.grad_v ? a.grad_v[t] * mk : 0.f;
}
// After the last pass: d log_v_init = g_v(0); d log_u_init = 0 (u_0 feeds nothing for
// K >= 1; for K = 0 the output is the masked initial potential itself).
__global__ void dense_bwd_finish_kernel(DenseSinkBwdArgs a) {
  const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const size_t BHN = (size_t)a.B * a.H * a.N;
  if (t >= BHN) return;
  if (a.dlog_v_init) a.dlog_v_init[t] = a.gv[t];
  if (a.dlog_u_init) {
    float g = 0.f;
    if (a.K == 0 && a.grad_u) {
      const int bh = (int)(t / a.N), i = (int)(t % a.N), b = bh / a.H;
      g = a.grad_u[t] * (a.mask ? a.mask[(size_t)b * a.N + i] : 1.f);
    }
    a.dlog_u_init[t] = g;
  }
}

__global__ void dense_zero_kernel(float* p, size_t n) {
  const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t < n) p[t] = 0.f;
}

// ---------------------------------------------------------------------------
// Transport output, forward.  One wave per row i of one (b,h):
//   ls_j = u_i - C_ij/eps + v_j + cb_j, T = exp(ls - max), Tn = T / (sum T + 1e-6) * mask_i,
//   O_i = sum_j Tn_j V_j (lane = column c, Tn broadcast through LDS), x_c = sum_j Tn_j x_j,
//   o = sigma(G) O (permuted to (B,N,H*d)) * mask_i.  Saves O_avg for the backward.
__global__ void __launch_bounds__(DN_NT) dense_transport_fwd_kernel(DenseTransportArgs a) {
  __shared__ float s_t[DN_NW][WAVE];
  const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;
  const size_t row = (size_t)blockIdx.x * DN_NW + wave;
  const int N = a.N, d = a.d;
  const size_t BHN = (size_t)a.B * a.H * N;
  const bool live = row < BHN;
  const size_t rr = live ? row : 0;
  const int bh = (int)(rr / N), i = (int)(rr % N), b = bh / a.H, h = bh % a.H;
  const float eps = a.eps[h];
  const float* Cr = a.C + rr * N;
  const float* v = a.log_v + (size_t)bh * N;
  const float ui = a.log_u[rr];
  const float mi = a.mask ? a.mask[(size_t)b * N + i] : 1.f;
  float m = -INFINITY;
  for (int j = lane; j < N; j += WAVE) m = fmaxf(m, ui + (-Cr[j] / eps) + v[j] + mask_bias(a.mask, b, N, j));
  m = wave_max(m);
  float s = 0.f;
  for (int j = lane; j < N; j += WAVE) s += __expf(ui + (-Cr[j] / eps) + v[j] + mask_bias(a.mask, b, N, j) - m);
  s = wave_sum(s);
  const float scale = mi / (s + 1e-6f);
  float* Tr = a.T_norm + rr * N;
  const float* Vb = a.V + (size_t)bh * N * d;
  const float* xb = a.x_res ? a.x_res + (size_t)b * N * 3 : nullptr;
  float oacc = 0.f, x0 = 0.f, x1 = 0.f, x2 = 0.f;
  for (int j0 = 0; j0 < N; j0 += WAVE) {
    const int j = j0 + lane;
    float tn = 0.f;
    if (j < N) {
      tn = __expf(ui + (-Cr[j] / eps) + v[j] + mask_bias(a.mask, b, N, j) - m) * scale;
      if (live) Tr[j] = tn;
      if (xb) {
        x0 = __builtin_fmaf(tn, xb[3 * j], x0);
        x1 = __builtin_fmaf(tn, xb[3 * j + 1], x1);
        x2 = __builtin_fmaf(tn, xb[3 * j + 2], x2);
      }
    }
    s_t[wave][lane] = tn;  // wave-private slice: no block barrier needed
    const int jn = min(WAVE, N - j0);
    if (lane < d)
      for (int jj = 0; jj < jn; ++jj) oacc = __builtin_fmaf(s_t[wave][jj], Vb[(size_t)(j0 + jj) * d + lane], oacc);
  }
  if (!live) return;
  if (lane < d) {
    a.o_avg[rr * d + lane] = oacc;
    const float g = a.G ? 1.f / (1.f + __expf(-a.G[rr * d + lane])) : 1.f;
    a.o[((size_t)b * N + i) * (size_t)(a.H * d) + (size_t)h * d + lane] = g * oacc * mi;
  }
  if (a.x_centroid) {
    x0 = wave_sum(x0);
    x1 = wave_sum(x1);
    x2 = wave_sum(x2);
    if (lane == 0) {
      a.x_centroid[rr * 3 + 0] = x0;
      a.x_centroid[rr * 3 + 1] = x1;
      a.x_centroid[rr * 3 + 2] = x2;
    }
  }
}

// Transport backward, row pass (wave per row i):
//   gOa_i = sigma(G) gO_i mask_i,  dG_i = sigma (1 - sigma) O_avg_i gO_i mask_i
//   dTn_ij = (gOa_i . V_j + gxc_i . x_j + gT_ij) * mask_i
//   dT_j = (dTn_j - dot) / (S + 1e-6) with dot = sum_j' dTn_j' T_j' / (S + 1e-6);  dls_j = dT_j T_j
//   plus, at the first argmax (torch max semantics), the row max's gradient
//   -sum_j dT_j T_j = -dot 1e-6 / (S + 1e-6)
//   dC_ij = -dls_ij / eps,  d log_u_i = sum_j dls_ij.  Writes gOa for the column pass.
__global__ void __launch_bounds__(DN_NT) dense_transport_bwd_row_kernel(DenseTransportArgs a) {
  __shared__ float s_g[DN_NW][64 + 4];
  const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;
  const size_t row = (size_t)blockIdx.x * DN_NW + wave;
  const int N = a.N, d = a.d;
  const size_t BHN = (size_t)a.B * a.H * N;
  if (row >= BHN) return;
  const int bh = (int)(row / N), i = (int)(row % N), b = bh / a.H, h = bh % a.H;
  const float eps = a.eps[h];
  const float* Cr = a.C + row * N;
  const float* v = a.log_v + (size_t)bh * N;
  const float ui = a.log_u[row];
  const float mi = a.mask ? a.mask[(size_t)b * N + i] : 1.f;
  // gated output gradient of this row (lane = column)
  float goa = 0.f;
  if (lane < d) {
    const float go = a.grad_o ? a.grad_o[((size_t)b * N + i) * (size_t)(a.H * d) + (size_t)h * d + lane] * mi : 0.f;
    const float sg = a.G ? 1.f / (1.f + __expf(-a.G[row * d + lane])) : 1.f;
    goa = sg * go;
    if (a.dG) a.dG[row * d + lane] = sg * (1.f - sg) * a.o_avg[row * d + lane] * go;
    a.goa[row * d + lane] = goa;
  }
  s_g[wave][lane] = goa;
  const float* gxc = a.grad_xc ? a.grad_xc + row * 3 : nullptr;
  if (lane < 3) s_g[wave][64 + lane] = gxc ? gxc[lane] : 0.f;
  // recompute the row statistics of the forward
  float m = -INFINITY;
  int am = N;  // first argmax
  for (int j = lane; j < N; j += WAVE) {
    const float x = ui + (-Cr[j] / eps) + v[j] + mask_bias(a.mask, b, N, j);
    if (x > m) { m = x; am = j; }
  }
  const float mw = wave_max(m);
  int amw = m == mw ? am : N;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) amw = min(amw, __shfl_xor(amw, o, WAVE));
  float s = 0.f;
  for (int j = lane; j < N; j += WAVE) s += __expf(ui + (-Cr[j] / eps) + v[j] + mask_bias(a.mask, b, N, j) - mw);
  s = wave_sum(s);
  const float den = s + 1e-6f;
  const float* Vb = a.V + (size_t)bh * N * d;
  const float* xb = a.x_res ? a.x_res + (size_t)b * N * 3 : nullptr;
  const float* gT = a.grad_T ? a.grad_T + row * N : nullptr;
  // pass 1: sum_j dTn_j Tn_j with Tn the unmasked normalised plan
  auto dtn_of = [&](int j) {
    float acc = gT ? gT[j] : 0.f;
    const float* Vj = Vb + (size_t)j * d;
    for (int c = 0; c < d; ++c) acc = __builtin_fmaf(s_g[wave][c], Vj[c], acc);
    if (xb) acc += s_g[wave][64] * xb[3 * j] + s_g[wave][65] * xb[3 * j + 1] + s_g[wave][66] * xb[3 * j + 2];
    return acc * mi;
  };
  float dot = 0.f;
  for (int j = lane; j < N; j += WAVE) {
    const float T = __expf(ui + (-Cr[j] / eps) + v[j] + mask_bias(a.mask, b, N, j) - mw);
    dot += dtn_of(j) * (T / den);
  }
  dot = wave_sum(dot);
  // pass 2: dls_j (with the row max's gradient at the first argmax), dC, d log_u
  const float dmax = -dot * 1e-6f / den;
  float du = 0.f;
  float* dCr = a.dC + row * N;
  for (int j = lane; j < N; j += WAVE) {
    const float T = __expf(ui + (-Cr[j] / eps) + v[j] + mask_bias(a.mask, b, N, j) - mw);
    float dls = (dtn_of(j) - dot) / den * T;
    if (j == amw) dls += dmax;
    du += dls;
    dCr[j] = -dls / eps;
  }
  du = wave_sum(du);
  if (lane == 0) a.dlog_u[row] = du;
}

// Transport backward, column pass (workgroup per 64 columns, lane = column j):
//   dV_j = sum_i Tn_ij gOa_i,  dx_j (this head) = sum_i Tn_ij gxc_i,  d log_v_j = sum_i dls_ij
//   with dls_ij = -eps dC_ij (dC already holds the argmax term).
__global__ void __launch_bounds__(DN_NT) dense_transport_bwd_col_kernel(DenseTransportArgs a) {
  __shared__ float s_acc[DN_NW][WAVE][17];
  const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;
  const int N = a.N, d = a.d;
  const int nblk = (N + WAVE - 1) / WAVE;
  const int bh = blockIdx.x / nblk, j = (blockIdx.x % nblk) * WAVE + lane;
  const int b = bh / a.H, h = bh % a.H;
  const float eps = a.eps[h];
  const float* Tb = a.T_norm + (size_t)bh * N * N;
  const float* dCb = a.dC + (size_t)bh * N * N;
  const float* goa = a.goa + (size_t)bh * N * d;
  const float* gxc = a.grad_xc ? a.grad_xc + (size_t)bh * N * 3 : nullptr;
  float dv[64];
#pragma unroll
  for (int c = 0; c < 64; ++c) dv[c] = 0.f;
  float dlv = 0.f, dx0 = 0.f, dx1 = 0.f, dx2 = 0.f;
  if (j < N)
    for (int i = wave; i < N; i += DN_NW) {
      const float tn = Tb[(size_t)i * N + j];
      dlv += -eps * dCb[(size_t)i * N + j];
      const float* gi = goa + (size_t)i * d;
#pragma unroll
      for (int c = 0; c < 64; ++c)
        if (c < d) dv[c] = __builtin_fmaf(tn, gi[c], dv[c]);
      if (gxc) {
        dx0 = __builtin_fmaf(tn, gxc[3 * i], dx0);
        dx1 = __builtin_fmaf(tn, gxc[3 * i + 1], dx1);
        dx2 = __builtin_fmaf(tn, gxc[3 * i + 2], dx2);
      }
    }
  // combine the four waves, 16 accumulator columns at a time
  float* dVj = a.dV + ((size_t)bh * N + j) * d;
#pragma unroll
  for (int c0 = 0; c0 < 64; c0 += 16) {
    if (c0 < d) {  // uniform
      __syncthreads();
#pragma unroll
      for (int cc = 0; cc < 16; ++cc) s_acc[wave][lane][cc] = dv[c0 + cc];
      __syncthreads();
      if (wave == 0 && j < N)
        for (int cc = 0; cc < 16 && c0 + cc < d; ++cc) {
          float t = 0.f;
#pragma unroll
          for (int w = 0; w < DN_NW; ++w) t += s_acc[w][lane][cc];
          dVj[c0 + cc] = t;
        }
    }
  }
  __syncthreads();
  s_acc[wave][lane][0] = dlv;
  s_acc[wave][lane][1] = dx0;
  s_acc[wave][lane][2] = dx1;
  s_acc[wave][lane][3] = dx2;
  __syncthreads();
  if (wave == 0 && j < N) {
    float t[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < DN_NW; ++w)
#pragma unroll
      for (int cc = 0; cc < 4; ++cc) t[cc] += s_acc[w][lane][cc];
    const size_t col = (size_t)bh * N + j;
    a.dlog_v[col] = t[0];
    if (a.dx_part) {
      a.dx_part[col * 3 + 0] = t[1];
      a.dx_part[col * 3 + 1] = t[2];
      a.dx_part[col * 3 + 2] = t[3];
    }
  }
}

// dx_res[b, j] = sum_h dx_part[b, h, j] (fixed order).
__global__ void dense_transport_dx_kernel(DenseTransportArgs a) {
  const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (size_t)a.B * a.N * 3) return;
  const int b = (int)(t / ((size_t)a.N * 3));
  const size_t rem = t - (size_t)b * a.N * 3;
  float s = 0.f;
  for (int h = 0; h < a.H; ++h) s += a.dx_part[((size_t)b * a.H + h) * a.N * 3 + rem];
  a.dx_res[t] = s;
}

// ---------------------------------------------------------------------------
static unsigned blocks_for(size_t n, int per) { return (unsigned)((n + per - 1) / per); }

hipError_t dense_sinkhorn_init(const DenseSinkArgs& a, hipStream_t s) {
  const size_t BHN = (size_t)a.B * a.H * a.N;
  const size_t n = std::max(BHN, (size_t)2 * (a.K + 1));
  hipLaunchKernelGGL(dense_init_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, s, a);
  return hipGetLastError();
}
hipError_t dense_sinkhorn_iteration(const DenseSinkArgs& a, int k, hipStream_t s) {
  const size_t BHN = (size_t)a.B * a.H * a.N;
  hipLaunchKernelGGL(dense_row_update_kernel, dim3(blocks_for(BHN, DN_NW)), dim3(DN_NT), 0, s, a, k);
  const int nblk = (a.N + WAVE - 1) / WAVE;
  hipLaunchKernelGGL(dense_col_update_kernel, dim3((unsigned)(a.B * a.H * nblk)), dim3(DN_NT), 0, s, a, k);
  return hipGetLastError();
}
hipError_t dense_sinkhorn_finish(const DenseSinkArgs& a, int k, hipStream_t s) {
  const size_t BHN = (size_t)a.B * a.H * a.N;
  hipLaunchKernelGGL(dense_finish_kernel, dim3(blocks_for(BHN, 256)), dim3(256), 0, s, a, k);
  return hipGetLastError();
}
hipError_t dense_sinkhorn_backward(const DenseSinkBwdArgs& a, hipStream_t s) {
  const size_t BHN = (size_t)a.B * a.H * a.N;
  const int nblk = (a.N + WAVE - 1) / WAVE;
  hipLaunchKernelGGL(dense_bwd_init_kernel, dim3(blocks_for(BHN, 256)), dim3(256), 0, s, a);
  for (int k = a.K; k >= 1; --k) {
    hipLaunchKernelGGL(dense_bwd_row_kernel, dim3(blocks_for(BHN, DN_NW)), dim3(DN_NT), 0, s, a, k);
    hipLaunchKernelGGL(dense_bwd_col_kernel, dim3((unsigned)(a.B * a.H * nblk)), dim3(DN_NT), 0, s, a, k);
  }
  hipLaunchKernelGGL(dense_bwd_finish_kernel, dim3(blocks_for(BHN, 256)), dim3(256), 0, s, a);
  return hipGetLastError();
}
hipError_t dense_zero(float* p, size_t n, hipStream_t s) {
  hipLaunchKernelGGL(dense_zero_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, s, p, n);
  return hipGetLastError();
}
hipError_t dense_transport_forward(const DenseTransportArgs& a, hipStream_t s) {
  const size_t BHN = (size_t)a.B * a.H * a.N;
  hipLaunchKernelGGL(dense_transport_fwd_kernel, dim3(blocks_for(BHN, DN_NW)), dim3(DN_NT), 0, s, a);
  return hipGetLastError();
}
hipError_t dense_transport_backward(const DenseTransportArgs& a, hipStream_t s) {
  const size_t BHN = (size_t)a.B * a.H * a.N;
  const int nblk = (a.N + WAVE - 1) / WAVE;
  hipLaunchKernelGGL(dense_transport_bwd_row_kernel, dim3(blocks_for(BHN, DN_NW)), dim3(DN_NT), 0, s, a);
  hipLaunchKernelGGL(dense_transport_bwd_col_kernel, dim3((unsigned)(a.B * a.H * nblk)), dim3(DN_NT), 0, s, a);
  if (a.dx_res && a.dx_part)
    hipLaunchKernelGGL(dense_transport_dx_kernel, dim3(blocks_for((size_t)a.B * a.N * 3, 256)), dim3(256), 0, s, a);
  return hipGetLastError();
}

}  // namespace dfl
