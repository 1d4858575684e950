// Softmax attention kernels on gfx950 for the layers next to the Sinkhorn path:
//
//   flash_diffusion_attn  (flash_diffusion_attn.py:440-622)  bins / dense pair bias, optional gate
//   flash_atom_attn       (flash_atom_attn.py:215-354)       32-query windows over 128 keys
//   token_to_atom_attn    (cross_attn_kernel.py:460-696)     dense cross attention
//   atom_to_token_attn    (cross_attn_kernel.py:424-661)     per-token atom ranges (a2t_* kernels)
//
// The first three run on the streaming engine of attn_engine.h: forward, a
// query-resident pass for dQ and the bias gradients, and a key-resident pass for
// dK / dV (optionally split over query ranges with fp32 partials); the dQ pass runs
// first and also does the backward prep of its rows (D_i = dO_i.O_i, sigma(G) dO, dG).
// This file holds the finalize of the partial sums, the atom-to-token kernels and
// the launchers.  No atomics in HBM except in the atom-to-token backward, whose
// atom ranges may overlap.
#include "attn_args.h"
#include "attn_engine.h"
#include "common.h"

#include <algorithm>

namespace dfl {

// dK / dV from query-split partials; d pos_weight from per-workgroup partials; the
// window-bias gradient from per-batch-row slabs (all sums in a fixed order).
template <typename T, int DP>
__global__ void __launch_bounds__(256) attn_bwd_finalize_kernel(AttnArgs a, int n_qblocks) {
  const size_t e = (size_t)blockIdx.x * 256 + threadIdx.x;
  const size_t nslab = (size_t)((a.Mq + ATTN_WQ - 1) / ATTN_WQ) * a.H * ATTN_WQ * ATTN_WK;
  if (a.dbias_rows && e < nslab) {
    const T* rows = reinterpret_cast<const T*>(a.dbias_rows);
    float s = 0.f;
    for (int b = 0; b < a.B; ++b) s += to_f32(rows[(size_t)b * nslab + e]);
    reinterpret_cast<T*>(a.dbias)[e] = from_f32<T>(s);
  }
  const size_t nkv = (size_t)a.B * a.H * a.Nk * a.d;
  if (a.qsplit > 1 && e < nkv) {
    const size_t row = e / a.d;
    const int col = (int)(e % a.d);
    float sk = 0.f, sv = 0.f;
    for (int s = 0; s < a.qsplit; ++s) {
      const float* part = a.kv_part + ((size_t)s * a.B * a.H * a.Nk + row) * 2 * DP;
      sk += part[col];
      sv += part[DP + col];
    }
    reinterpret_cast<T*>(a.dk)[e] = from_f32<T>(sk);
    reinterpret_cast<T*>(a.dv)[e] = from_f32<T>(sv);
  }
  if (a.dpos_w && e < (size_t)a.H * 68) {
    const int h = (int)(e / 68), k = (int)(e % 68);
    float s = 0.f;
    for (int b = 0; b < a.B; ++b)
      for (int qb = 0; qb < n_qblocks; ++qb) s += a.dpw_part[(((size_t)b * a.H + h) * n_qblocks + qb) * 68 + k];
    a.dpos_w[e] = s;
  }
}

// ===========================================================================
// Atom-to-token (cross_attn_kernel.py:424-457): token n attends to atoms
// [starts[n], starts[n] + counts[n]).  One wave per (b, h, n); lanes take atoms
// for the scores and head-dim columns for the output.
// Atom range of token (b, n), clipped to [0, M); count 0 if the token is masked.
__device__ __forceinline__ void a2t_range(const A2TArgs& a, int b, int n, int& st, int& cnt) {
  st = a.starts[(size_t)b * a.N + n];
  cnt = (st < 0 || st >= a.M) ? 0 : min(a.counts[(size_t)b * a.N + n], a.M - st);
  if (a.tmask && a.tmask[(size_t)b * a.N + n] == 0.f) cnt = 0;
  if (cnt < 0) cnt = 0;
}

// Forward: atoms stream in chunks of 64 (one per lane) with an online softmax;
// the output accumulates with lane = head-dim column.
template <typename T>
__global__ void __launch_bounds__(256) a2t_fwd_kernel(A2TArgs a) {
  __shared__ float s_p[4][WAVE];
  __shared__ float s_q[4][64];
  const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;
  const size_t tok = (size_t)blockIdx.x * 4 + wave;  // over B*H*N
  if (tok >= (size_t)a.B * a.H * a.N) return;
  const int bh = (int)(tok / a.N), n = (int)(tok % a.N), b = bh / a.H;
  int st, cnt;
  a2t_range(a, b, n, st, cnt);
  const T* K = reinterpret_cast<const T*>(a.k) + (size_t)bh * a.M * a.d;
  const T* V = reinterpret_cast<const T*>(a.v) + (size_t)bh * a.M * a.d;
  if (lane < a.d) s_q[wave][lane] = to_f32(reinterpret_cast<const T*>(a.q)[tok * a.d + lane]);
  const float sc = a.scale * LOG2E;
  float m = NEG_BIG, l = 0.f, acc = 0.f;
  for (int j0 = 0; j0 < cnt; j0 += WAVE) {
    const int j = j0 + lane;
    float s = NEG_BIG;
    if (j < cnt) {
      const T* kr = K + (size_t)(st + j) * a.d;
      float dot = 0.f;
      for (int c = 0; c < a.d; ++c) dot = __builtin_fmaf(s_q[wave][c], to_f32(kr[c]), dot);
      s = dot * sc;
    }
    float mt = s;
    for (int o = 32; o >= 1; o >>= 1) mt = fmaxf(mt, __shfl_xor(mt, o, WAVE));
    const float mn = fmaxf(m, mt);
    const float alpha = fast_exp2(m - mn);
    const float p = j < cnt ? fast_exp2(s - mn) : 0.f;
    s_p[wave][lane] = p;
    float lp = p;
    for (int o = 32; o >= 1; o >>= 1) lp += __shfl_xor(lp, o, WAVE);
    l = l * alpha + lp;
    acc *= alpha;
    const int nj = min(WAVE, cnt - j0);
    if (lane < a.d)
      for (int jj = 0; jj < nj; ++jj)
        acc = __builtin_fmaf(s_p[wave][jj], to_f32(V[(size_t)(st + j0 + jj) * a.d + lane]), acc);
    m = mn;
  }
  const bool ok = cnt > 0 && l > 0.f;
  if (lane < a.d) reinterpret_cast<T*>(a.o)[tok * a.d + lane] = from_f32<T>(ok ? acc / l : 0.f);
  if (lane == 0) a.lse[tok] = ok ? (m + fast_log2(l)) * LN2 : 0.f;
}

// Backward: p and dS per atom chunk from the saved LSE; dQ with lane = column;
// dK / dV accumulate with fp32 atomics (token atom ranges may overlap).
template <typename T>
__global__ void __launch_bounds__(256) a2t_bwd_kernel(A2TArgs a) {
  __shared__ float s_p[4][WAVE];
  __shared__ float s_ds[4][WAVE];
  __shared__ float s_q[4][64];
  __shared__ float s_do[4][64];
  const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;
  const size_t tok = (size_t)blockIdx.x * 4 + wave;
  if (tok >= (size_t)a.B * a.H * a.N) return;
  const int bh = (int)(tok / a.N), n = (int)(tok % a.N), b = bh / a.H;
  int st, cnt;
  a2t_range(a, b, n, st, cnt);
  T* dQ = reinterpret_cast<T*>(a.dq) + tok * a.d;
  if (cnt == 0) {
    if (lane < a.d) dQ[lane] = from_f32<T>(0.f);
    return;
  }
  const T* K = reinterpret_cast<const T*>(a.k) + (size_t)bh * a.M * a.d;
  const T* V = reinterpret_cast<const T*>(a.v) + (size_t)bh * a.M * a.d;
  const float l2 = a.lse[tok] * LOG2E;
  const float sc = a.scale * LOG2E;
  float Dp = 0.f;
  if (lane < a.d) {
    s_q[wave][lane] = to_f32(reinterpret_cast<const T*>(a.q)[tok * a.d + lane]);
    const float dov = to_f32(reinterpret_cast<const T*>(a.dout)[tok * a.d + lane]);
    s_do[wave][lane] = dov;
    Dp = dov * to_f32(reinterpret_cast<const T*>(a.o)[tok * a.d + lane]);
  }
  for (int o = 32; o >= 1; o >>= 1) Dp += __shfl_xor(Dp, o, WAVE);
  float dq = 0.f;
  for (int j0 = 0; j0 < cnt; j0 += WAVE) {
    const int j = j0 + lane;
    float p = 0.f, ds = 0.f;
    if (j < cnt) {
      const T* kr = K + (size_t)(st + j) * a.d;
      const T* vr = V + (size_t)(st + j) * a.d;
      float s = 0.f, dp = 0.f;
      for (int c = 0; c < a.d; ++c) {
        s = __builtin_fmaf(s_q[wave][c], to_f32(kr[c]), s);
        dp = __builtin_fmaf(s_do[wave][c], to_f32(vr[c]), dp);
      }
      p = fast_exp2(s * sc - l2);
      ds = p * (dp - Dp);
    }
    s_p[wave][lane] = p;
    s_ds[wave][lane] = ds;
    const int nj = min(WAVE, cnt - j0);
    if (lane < a.d)
      for (int jj = 0; jj < nj; ++jj) {
        const size_t atom = (size_t)bh * a.M + st + j0 + jj;
        dq = __builtin_fmaf(s_ds[wave][jj], to_f32(K[(atom - (size_t)bh * a.M) * a.d + lane]), dq);
        float* acc_kv = a.dkv + atom * 2 * a.d;
        atomicAdd(acc_kv + lane, a.scale * s_ds[wave][jj] * s_q[wave][lane]);
        atomicAdd(acc_kv + a.d + lane, s_p[wave][jj] * s_do[wave][lane]);
      }
  }
  if (lane < a.d) dQ[lane] = from_f32<T>(a.scale * dq);
}

__global__ void __launch_bounds__(256) a2t_zero_kernel(float* p, size_t n) {
  const size_t e = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (e < n) p[e] = 0.f;
}

template <typename T>
__global__ void __launch_bounds__(256) a2t_bwd_finalize_kernel(A2TArgs a) {
  const size_t e = (size_t)blockIdx.x * 256 + threadIdx.x;
  const size_t total = (size_t)a.B * a.H * a.M * a.d;
  if (e >= total) return;
  const size_t row = e / a.d;
  const int c = (int)(e % a.d);
  reinterpret_cast<T*>(a.dk)[e] = from_f32<T>(a.dkv[row * 2 * a.d + c]);
  reinterpret_cast<T*>(a.dv)[e] = from_f32<T>(a.dkv[row * 2 * a.d + a.d + c]);
}

// ===========================================================================
// Launchers
// Fast staging: 16-byte aligned key / value rows and bias rows (and query, dO, O and
// gate rows when with_q), head dim a multiple of the 16-byte element count, key
// count a multiple of 8 when a bias is read.
template <typename T>
static bool attn_fast(const AttnArgs& a, bool with_q) {
  constexpr int VEC = 16 / (int)sizeof(T);
  auto al = [](const void* p) { return ((uintptr_t)p & 15u) == 0; };
  auto st = [](long long s) { return ((s * (long long)sizeof(T)) & 15) == 0; };
  bool ok = a.d % VEC == 0 && al(a.k) && al(a.v) && st(a.ksb) && st(a.ksh) && st(a.ksn);
  if (with_q) ok = ok && al(a.q) && st(a.qsb) && st(a.qsh) && st(a.qsn);
  if (with_q) ok = ok && al(a.dout) && al(a.o) && (!a.g || al(a.g));  // row loads of the forward and dQ pass
  if (a.bias_mode == ATTN_BIAS_DENSE || a.bias_mode == ATTN_BIAS_WINDOW)
    ok = ok && al(a.bias) && (!a.dbias || al(a.dbias)) && a.Nk % 8 == 0;
  if (a.bias_mode == ATTN_BIAS_BINS) ok = ok && al(a.bins) && a.Nk % 8 == 0;
  return ok;
}

template <typename T, int DP, int BIAS, bool WIN, bool FAST>
static hipError_t attn_fwd_f(const AttnArgs& a, hipStream_t s) {
  using E = Eng<T, DP, WIN>;
  const int lds = attn_fwd_lds<T, DP, WIN>() + (a.g ? attn_fwd_gate_lds<T, DP, WIN>() : 0);
  auto kern = attn_fwd2_kernel<T, DP, BIAS, WIN, FAST>;
  const hipError_t attr = set_lds_limit((const void*)kern, lds);
  if (attr != hipSuccess) return attr;
  const int nqb = (a.Mq + E::RQ - 1) / E::RQ;
  hipLaunchKernelGGL(kern, dim3((unsigned)(nqb * a.B * a.H)), dim3(E::NT), lds, s, a);
  return hipGetLastError();
}
template <typename T, int DP, int BIAS, bool WIN>
static hipError_t attn_fwd_w(const AttnArgs& a, hipStream_t s) {
  return attn_fast<T>(a, true) ? attn_fwd_f<T, DP, BIAS, WIN, true>(a, s) : attn_fwd_f<T, DP, BIAS, WIN, false>(a, s);
}
template <typename T, int DP, int BIAS>
static hipError_t attn_fwd_t(const AttnArgs& a, hipStream_t s) {
  return a.window ? attn_fwd_w<T, DP, BIAS, true>(a, s) : attn_fwd_w<T, DP, BIAS, false>(a, s);
}
template <typename T, int DP>
static hipError_t attn_fwd_b(const AttnArgs& a, hipStream_t s) {
  switch (a.bias_mode) {
    case ATTN_BIAS_NONE: return attn_fwd_t<T, DP, ATTN_BIAS_NONE>(a, s);
    case ATTN_BIAS_BINS: return attn_fwd_t<T, DP, ATTN_BIAS_BINS>(a, s);
    case ATTN_BIAS_DENSE: return attn_fwd_t<T, DP, ATTN_BIAS_DENSE>(a, s);
    case ATTN_BIAS_WINDOW: return attn_fwd_t<T, DP, ATTN_BIAS_WINDOW>(a, s);
  }
  return hipErrorInvalidValue;
}
hipError_t launch_attn_fwd(const AttnArgs& a, bool bf16_in, int DP, hipStream_t s) {
  if (bf16_in) return DP == 32 ? attn_fwd_b<bf16, 32>(a, s) : attn_fwd_b<bf16, 64>(a, s);
  return DP == 32 ? attn_fwd_b<float, 32>(a, s) : attn_fwd_b<float, 64>(a, s);
}

template <typename T, int DP, int BIAS, bool WIN, bool FAST>
static hipError_t attn_bwd_f(const AttnArgs& a, hipStream_t s) {
  using E = Eng<T, DP, WIN>;
  using K = EngKV<T, DP>;
  constexpr int lkv = attn_bwdkv_lds<T, DP>(), lq = attn_bwdq_lds<T, DP, WIN>();
  auto kkv = attn_bwd_kv2_kernel<T, DP, BIAS, WIN, FAST>;
  auto kq = attn_bwd_q2_kernel<T, DP, BIAS, WIN, FAST>;
  const hipError_t attr = set_lds_limit((const void*)kkv, lkv) != hipSuccess ? hipErrorInvalidValue
                                                                             : set_lds_limit((const void*)kq, lq);
  if (attr != hipSuccess) return attr;
  const int BH = a.B * a.H;
  // the dQ pass first: it also writes do_w and D of every query, which the dK/dV pass streams
  const int nqb = (a.Mq + E::RQ - 1) / E::RQ;
  hipLaunchKernelGGL(kq, dim3((unsigned)(nqb * BH)), dim3(E::NT), lq, s, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int nkb = (a.Nk + K::RK - 1) / K::RK;
  hipLaunchKernelGGL(kkv, dim3((unsigned)(nkb * a.qsplit * BH)), dim3(K::NT), lkv, s, a);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  if (a.qsplit > 1 || (BIAS == ATTN_BIAS_BINS && a.dpos_w) || a.dbias_rows) {
    const size_t nslab = a.dbias_rows ? (size_t)((a.Mq + ATTN_WQ - 1) / ATTN_WQ) * a.H * ATTN_WQ * ATTN_WK : 0;
    const size_t n = std::max(std::max((size_t)BH * a.Nk * a.d, (size_t)a.H * 68), nslab);
    hipLaunchKernelGGL((attn_bwd_finalize_kernel<T, DP>), dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, a,
                       nqb);
    e = hipGetLastError();
  }
  return e;
}
template <typename T, int DP, int BIAS, bool WIN>
static hipError_t attn_bwd_w(const AttnArgs& a, hipStream_t s) {
  return attn_fast<T>(a, true) ? attn_bwd_f<T, DP, BIAS, WIN, true>(a, s) : attn_bwd_f<T, DP, BIAS, WIN, false>(a, s);
}
template <typename T, int DP, int BIAS>
static hipError_t attn_bwd_t(const AttnArgs& a, hipStream_t s) {
  return a.window ? attn_bwd_w<T, DP, BIAS, true>(a, s) : attn_bwd_w<T, DP, BIAS, false>(a, s);
}
template <typename T, int DP>
static hipError_t attn_bwd_b(const AttnArgs& a, hipStream_t s) {
  switch (a.bias_mode) {
    case ATTN_BIAS_NONE: return attn_bwd_t<T, DP, ATTN_BIAS_NONE>(a, s);
    case ATTN_BIAS_BINS: return attn_bwd_t<T, DP, ATTN_BIAS_BINS>(a, s);
    case ATTN_BIAS_DENSE: return attn_bwd_t<T, DP, ATTN_BIAS_DENSE>(a, s);
    case ATTN_BIAS_WINDOW: return attn_bwd_t<T, DP, ATTN_BIAS_WINDOW>(a, s);
  }
  return hipErrorInvalidValue;
}
hipError_t launch_attn_bwd(const AttnArgs& a, bool bf16_in, int DP, hipStream_t s) {
  if (bf16_in) return DP == 32 ? attn_bwd_b<bf16, 32>(a, s) : attn_bwd_b<bf16, 64>(a, s);
  return DP == 32 ? attn_bwd_b<float, 32>(a, s) : attn_bwd_b<float, 64>(a, s);
}

hipError_t launch_a2t_fwd(const A2TArgs& a, bool bf16_in, hipStream_t s) {
  const size_t toks = (size_t)a.B * a.H * a.N;
  dim3 grid((unsigned)((toks + 3) / 4));
  if (bf16_in) hipLaunchKernelGGL(a2t_fwd_kernel<bf16>, grid, dim3(256), 0, s, a);
  else hipLaunchKernelGGL(a2t_fwd_kernel<float>, grid, dim3(256), 0, s, a);
  return hipGetLastError();
}
hipError_t launch_a2t_bwd(const A2TArgs& a, bool bf16_in, hipStream_t s) {
  const size_t nacc = (size_t)a.B * a.H * a.M * 2 * a.d;
  hipLaunchKernelGGL(a2t_zero_kernel, dim3((unsigned)((nacc + 255) / 256)), dim3(256), 0, s, a.dkv, nacc);
  const size_t toks = (size_t)a.B * a.H * a.N;
  dim3 grid((unsigned)((toks + 3) / 4));
  if (bf16_in) hipLaunchKernelGGL(a2t_bwd_kernel<bf16>, grid, dim3(256), 0, s, a);
  else hipLaunchKernelGGL(a2t_bwd_kernel<float>, grid, dim3(256), 0, s, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const size_t n = (size_t)a.B * a.H * a.M * a.d;
  dim3 g2((unsigned)((n + 255) / 256));
  if (bf16_in) hipLaunchKernelGGL(a2t_bwd_finalize_kernel<bf16>, g2, dim3(256), 0, s, a);
  else hipLaunchKernelGGL(a2t_bwd_finalize_kernel<float>, g2, dim3(256), 0, s, a);
  return hipGetLastError();
}

}  // namespace dfl
