// Softmax attention kernels on gfx950 for the layers next to the Sinkhorn path:
//
//   flash_diffusion_attn  (flash_diffusion_attn.py:440-622)  bins / dense pair bias, optional gate
//   flash_atom_attn       (flash_atom_attn.py:215-354)       32-query windows over 128 keys
//   token_to_atom_attn    (cross_attn_kernel.py:460-696)     dense cross attention
//   atom_to_token_attn    (cross_attn_kernel.py:424-661)     per-token atom ranges (a2t_* kernels)
//
// One engine serves the first three.  A wave owns 16 queries (or 16 keys in the
// dK/dV pass) whose MFMA fragments stay in registers; the other operand streams
// through LDS in chunks of 32-128 rows.  Scores are formed transposed
// (S^T = K Q^T) so that each lane holds one resident row and 4+4 streamed
// columns of a 32-wide tile pair: row statistics of the online softmax stay in
// the lane (plus two lane-group exchanges), and the output is accumulated
// transposed (O^T = V^T P) with the same lane <-> row mapping, so the running
// rescale needs no lane shuffles.  Exponentials are base 2 (scores scaled by
// log2 e).
//
// Backward: prep (D_i = dO_i.O_i, sigma(G) dO, dG), a key-resident pass for dK /
// dV (optionally split over query ranges with fp32 partials), and a
// query-resident pass for dQ and the bias gradients.  No atomics in HBM except
// in the atom-to-token backward, whose atom ranges may overlap.
#include "attn_args.h"
#include "common.h"

#include <algorithm>

namespace dfl {

constexpr int AT_NT = 256;             // 4 waves
constexpr int AT_NW = AT_NT / WAVE;
constexpr int AT_RB = 16 * AT_NW;      // resident rows per workgroup
// Streamed rows per LDS chunk (a multiple of 32) and the row stride of transposed
// chunks, which leaves room to read one tile pair past the chunk end.
template <typename T, int DP> struct AtGeo {
  static constexpr int CH = sizeof(T) * DP <= 64 ? 128 : (sizeof(T) * DP <= 128 ? 64 : 32);
  static constexpr int TS = CH + 40;
};
constexpr float POS_BIG = 1.0e30f;     // LSE of a masked query: every P becomes exp2(-huge) = 0

__device__ __forceinline__ float sigm(float x) { return 1.f / (1.f + __expf(-x)); }

// 16-row fragment (row = r0 + l%16) from strided global memory, zero outside rows < n, cols < d.
template <typename T, int DP>
__device__ __forceinline__ void frag_rows(typename Mfma<T, DP>::Frag& f, const T* __restrict__ src, long long sn,
                                          int row, int n, int d, int lane) {
  constexpr int RUN = Mfma<T, DP>::RUN;
  T tmp[RUN];
  const int c0 = (lane >> 4) * RUN;
#pragma unroll
  for (int e = 0; e < RUN; ++e) {
    const int col = c0 + e;
    tmp[e] = (row < n && col < d) ? src[(size_t)row * sn + col] : from_f32<T>(0.f);
  }
  Mfma<T, DP>::from_run(f, tmp);
}

// Rows [r0, r0 + CH) of a strided operand into dst[CH][DP] (zero outside rows < n, cols < d).
template <typename T, int DP>
__device__ __forceinline__ void stage_rm(T* dst, const T* __restrict__ src, long long sn, int r0, int n, int d) {
  constexpr int CH = AtGeo<T, DP>::CH;
  for (int e = threadIdx.x; e < CH * DP; e += AT_NT) {
    const int row = e / DP, col = e - row * DP;
    const int i = r0 + row;
    dst[e] = (i < n && col < d) ? src[(size_t)i * sn + col] : from_f32<T>(0.f);
  }
}
// Same rows transposed into dst[DP][TS] (columns [CH, TS) zero).
template <typename T, int DP>
__device__ __forceinline__ void stage_tr(T* dst, const T* __restrict__ src, long long sn, int r0, int n, int d) {
  constexpr int CH = AtGeo<T, DP>::CH, TS = AtGeo<T, DP>::TS;
  for (int e = threadIdx.x; e < TS * DP; e += AT_NT) {
    const int col = e / TS, row = e - col * TS;
    const int i = r0 + row;
    dst[e] = (row < CH && i < n && col < d) ? src[(size_t)i * sn + col] : from_f32<T>(0.f);
  }
}

// Additive score bias in log2 units for (query i, key j) of head h.
template <typename T, int BIAS>
struct ScoreBias {
  const int* bins;      // row i at bins + i*Nk
  const float* pw2;     // LDS, pos_weight[h] * log2 e
  const T* bias;        // dense: row i at bias + i*Nk;  window: (W,H,32,128) base
  int Nk, H, h;
  __device__ __forceinline__ float operator()(int i, int j) const {
    if (BIAS == ATTN_BIAS_BINS) {
      const unsigned k = (unsigned)bins[(size_t)i * Nk + j];
      return k < 68u ? pw2[k] : 0.f;  // bins outside [0, 68) carry no bias
    }
    if (BIAS == ATTN_BIAS_DENSE) return LOG2E * to_f32(bias[(size_t)i * Nk + j]);
    if (BIAS == ATTN_BIAS_WINDOW) {
      const int w = i / ATTN_WQ;
      const int c = j - (ATTN_WQ * w - ATTN_WOFF);
      return LOG2E * to_f32(bias[(((size_t)w * H + h) * ATTN_WQ + (i - ATTN_WQ * w)) * ATTN_WK + c]);
    }
    return 0.f;
  }
};

// Key range [lo, hi) of the query tile starting at q (windowed: its window).
__device__ __forceinline__ void window_keys(int q, int Nk, int& lo, int& hi) {
  const int w = q / ATTN_WQ;
  lo = max(0, ATTN_WQ * w - ATTN_WOFF);
  hi = min(Nk, ATTN_WQ * w + ATTN_WQ + ATTN_WOFF);
}
__device__ __forceinline__ int floordiv(int x, int y) { return x >= 0 ? x / y : -((-x + y - 1) / y); }
// Query range [lo, hi) of the windows that contain any key of [k0, k1):
// key j is in window w  <=>  32w - 48 <= j < 32w + 80  <=>  floor((j - 80)/32) < w <= floor((j + 48)/32).
__device__ __forceinline__ void window_queries(int k0, int k1, int Mq, int& lo, int& hi) {
  const int wlo = max(0, floordiv(k0 - (ATTN_WQ + ATTN_WOFF), ATTN_WQ) + 1);
  const int whi = floordiv(k1 - 1 + ATTN_WOFF, ATTN_WQ);
  lo = min(Mq, ATTN_WQ * wlo);
  hi = min(Mq, ATTN_WQ * (whi + 1));
}

// ===========================================================================
// Forward
template <typename T, int DP, int BIAS>
__global__ void __launch_bounds__(AT_NT) attn_fwd_kernel(AttnArgs a) {
  using M = Mfma<T, DP>;
  constexpr int CH = AtGeo<T, DP>::CH, TS = AtGeo<T, DP>::TS;
  constexpr int NC = DP / 16;
  __shared__ __align__(16) T Ks[CH * DP];
  __shared__ __align__(16) T VTs[DP * TS];
  __shared__ __align__(16) float kb[CH + 32];
  __shared__ float s_pw[68];
  const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE, g = lane >> 4;
  const int bh = blockIdx.y, b = bh / a.H, h = bh % a.H;
  const int q0 = blockIdx.x * AT_RB;
  const int qt = q0 + 16 * wave;
  const int qi = qt + (lane & 15);
  const T* Qg = reinterpret_cast<const T*>(a.q) + (size_t)b * a.qsb + (size_t)h * a.qsh;
  const T* Kg = reinterpret_cast<const T*>(a.k) + (size_t)b * a.ksb + (size_t)h * a.ksh;
  const T* Vg = reinterpret_cast<const T*>(a.v) + (size_t)b * a.ksb + (size_t)h * a.ksh;
  const float sc = a.scale * LOG2E;
  const int Nk = a.Nk;

  int k_lo = 0, k_hi = Nk, wk_lo = 0, wk_hi = Nk;
  if (a.window) {
    int l1, h1, l2, h2;
    window_keys(q0, Nk, l1, h1);
    window_keys(min(q0 + AT_RB, a.Mq) - 1, Nk, l2, h2);
    k_lo = l1;
    k_hi = h2;
    window_keys(qt, Nk, wk_lo, wk_hi);
  }
  if (BIAS == ATTN_BIAS_BINS)
    for (int k = threadIdx.x; k < 68; k += AT_NT) s_pw[k] = LOG2E * a.pos_w[h * 68 + k];
  ScoreBias<T, BIAS> bias;
  bias.bins = a.bins ? a.bins + (size_t)b * a.Mq * Nk : nullptr;
  bias.pw2 = s_pw;
  bias.bias = nullptr;
  if (BIAS == ATTN_BIAS_DENSE) bias.bias = reinterpret_cast<const T*>(a.bias) + (size_t)bh * a.Mq * Nk;
  if (BIAS == ATTN_BIAS_WINDOW) bias.bias = reinterpret_cast<const T*>(a.bias);
  bias.Nk = Nk;
  bias.H = a.H;
  bias.h = h;

  typename M::Frag qf;
  frag_rows<T, DP>(qf, Qg, a.qsn, qi, a.Mq, a.d, lane);
  const bool active = qt < a.Mq;
  const bool qrow = qi < a.Mq;
  float m = NEG_BIG, lsum = 0.f;
  f32x4 oacc[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) oacc[c] = f32x4{0.f, 0.f, 0.f, 0.f};
  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};

  for (int c0 = k_lo; c0 < k_hi; c0 += CH) {
    __syncthreads();
    stage_rm<T, DP>(Ks, Kg, a.ksn, c0, Nk, a.d);
    stage_tr<T, DP>(VTs, Vg, a.ksn, c0, Nk, a.d);
    for (int j = threadIdx.x; j < CH + 32; j += AT_NT) {
      const int key = c0 + j;
      const bool ok = j < CH && key < k_hi && (!a.kmask || a.kmask[(size_t)b * Nk + key] > 0.5f);
      kb[j] = ok ? 0.f : NEG_BIG;
    }
    __syncthreads();
    if (!active) continue;
    const int t_lo = max(c0, wk_lo), t_hi = min(c0 + CH, wk_hi);
    for (int kp = t_lo; kp < t_hi; kp += 32) {
      f32x4 x[2];
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        const int kt = kp + 16 * hf;
        x[hf] = f32x4{NEG_BIG, NEG_BIG, NEG_BIG, NEG_BIG};
        if (kt < t_hi) {
          typename M::Frag kf;
          M::load(kf, Ks + (size_t)(kt - c0 + (lane & 15)) * DP, lane);
          const f32x4 acc = M::qk(kf, qf, zero);
          const f32x4 kbv = *reinterpret_cast<const f32x4*>(kb + kt - c0 + 4 * g);
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            float xv = __builtin_fmaf(acc[r], sc, kbv[r]);
            if (BIAS != ATTN_BIAS_NONE && qrow && kbv[r] == 0.f) xv += bias(qi, kt + 4 * g + r);
            x[hf][r] = (kt + 4 * g + r < t_hi) ? xv : NEG_BIG;
          }
        }
      }
      float mt = fmaxf(fmaxf(fmaxf(x[0][0], x[0][1]), fmaxf(x[0][2], x[0][3])),
                       fmaxf(fmaxf(x[1][0], x[1][1]), fmaxf(x[1][2], x[1][3])));
      mt = max_groups(mt);
      const float mn = fmaxf(m, mt);
      const float alpha = fast_exp2(m - mn);
      f32x4 p[2];
      float ps = 0.f;
#pragma unroll
      for (int hf = 0; hf < 2; ++hf)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float pv = x[hf][r] > 0.5f * NEG_BIG ? fast_exp2(x[hf][r] - mn) : 0.f;
          p[hf][r] = pv;
          ps += pv;
        }
      lsum = __builtin_fmaf(lsum, alpha, ps);
#pragma unroll
      for (int c = 0; c < NC; ++c) {
#pragma unroll
        for (int r = 0; r < 4; ++r) oacc[c][r] *= alpha;
        oacc[c] = M::pvt(p[0], p[1], VTs + (size_t)(c * 16 + (lane & 15)) * TS + (kp - c0), lane, oacc[c]);
      }
      m = mn;
    }
  }
  if (!active) return;
  lsum = sum_groups(lsum);
  const bool qok = qrow && (!a.qmask || a.qmask[(size_t)b * a.Mq + qi] > 0.5f) && lsum > 0.f;
  const float inv = qok ? 1.f / lsum : 0.f;
  if (!qrow) return;
  T* O = reinterpret_cast<T*>(a.o) + ((size_t)bh * a.Mq + qi) * a.d;
  const T* Gr = a.g ? reinterpret_cast<const T*>(a.g) + (size_t)b * a.qsb + (size_t)h * a.qsh + (size_t)qi * a.qsn
                    : nullptr;
  // lane holds O^T[col = c*16 + 4g + r][query qi]
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int col = c * 16 + 4 * g + r;
      if (col < a.d) {
        float o = oacc[c][r] * inv;
        if (Gr) o *= sigm(to_f32(Gr[col]));
        O[col] = from_f32<T>(o);
      }
    }
  if (g == 0) a.lse[(size_t)bh * a.Mq + qi] = qok ? (m + fast_log2(lsum)) * LN2 : 0.f;
}

// ===========================================================================
// Backward prep: one thread per (b,h,i,c), the DP lanes of a row contiguous in a wave.
//   do_w = sigma(G) dO (or dO), D_i = sum_c dO_ic O_ic, dG = (1 - sigma) O dO  (O is the gated output)
template <typename T, int DP>
__global__ void __launch_bounds__(256) attn_bwd_prep_kernel(AttnArgs a) {
  const size_t e = (size_t)blockIdx.x * 256 + threadIdx.x;
  const size_t rows = (size_t)a.B * a.H * a.Mq;
  const size_t row = e / DP;
  const int c = (int)(e % DP);
  const bool in = row < rows;
  const int bh = in ? (int)(row / a.Mq) : 0, i = in ? (int)(row % a.Mq) : 0;
  const int b = bh / a.H, h = bh % a.H;
  const bool ok = in && (!a.qmask || a.qmask[(size_t)b * a.Mq + i] > 0.5f);
  float dov = 0.f, ov = 0.f, s = 1.f;
  if (ok && c < a.d) {
    dov = to_f32(reinterpret_cast<const T*>(a.dout)[row * a.d + c]);
    ov = to_f32(reinterpret_cast<const T*>(a.o)[row * a.d + c]);
    if (a.g) {
      s = sigm(to_f32(reinterpret_cast<const T*>(a.g)[(size_t)b * a.qsb + (size_t)h * a.qsh + (size_t)i * a.qsn + c]));
      if (a.dg) reinterpret_cast<T*>(a.dg)[row * a.d + c] = from_f32<T>((1.f - s) * ov * dov);
    }
  } else if (in && a.g && a.dg && c < a.d) {
    reinterpret_cast<T*>(a.dg)[row * a.d + c] = from_f32<T>(0.f);
  }
  if (in) reinterpret_cast<T*>(a.do_w)[row * DP + c] = from_f32<T>(s * dov);
  float part = dov * ov;
#pragma unroll
  for (int o = DP / 2; o >= 1; o >>= 1) part += __shfl_xor(part, o, WAVE);
  if (in && c == 0) a.dcoef[row] = part;
}

// ===========================================================================
// dK / dV: a wave owns a 16-key tile; queries stream.  grid (ceil(Nk/64), B*H, qsplit).
template <typename T, int DP, int BIAS>
__global__ void __launch_bounds__(AT_NT) attn_bwd_kv_kernel(AttnArgs a) {
  using M = Mfma<T, DP>;
  constexpr int CH = AtGeo<T, DP>::CH, TS = AtGeo<T, DP>::TS;
  constexpr int NC = DP / 16;
  __shared__ __align__(16) T Qs[CH * DP];
  __shared__ __align__(16) T dOs[CH * DP];
  __shared__ __align__(16) T QTs[DP * TS];
  __shared__ __align__(16) T dOTs[DP * TS];
  __shared__ __align__(16) float lse2[CH + 32];
  __shared__ __align__(16) float Dq[CH + 32];
  __shared__ float s_pw[68];
  const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE, g = lane >> 4;
  const int bh = blockIdx.y, b = bh / a.H, h = bh % a.H;
  const int Mq = a.Mq, Nk = a.Nk;
  const int k0 = blockIdx.x * AT_RB;
  const int kt = k0 + 16 * wave;
  const int kj = kt + (lane & 15);
  const T* Qg = reinterpret_cast<const T*>(a.q) + (size_t)b * a.qsb + (size_t)h * a.qsh;
  const T* Kg = reinterpret_cast<const T*>(a.k) + (size_t)b * a.ksb + (size_t)h * a.ksh;
  const T* Vg = reinterpret_cast<const T*>(a.v) + (size_t)b * a.ksb + (size_t)h * a.ksh;
  const T* dOw = reinterpret_cast<const T*>(a.do_w) + (size_t)bh * Mq * DP;
  const float sc = a.scale * LOG2E;

  // query range: this split of [0, Mq), intersected with the windows of the block's keys
  const int per = (((Mq + a.qsplit - 1) / a.qsplit) + 15) / 16 * 16;
  int q_lo = blockIdx.z * per, q_hi = min(Mq, q_lo + per);
  int wq_lo = q_lo, wq_hi = q_hi;
  if (a.window) {
    int l1, h1;
    window_queries(k0, min(Nk, k0 + AT_RB), Mq, l1, h1);
    q_lo = max(q_lo, l1);
    q_hi = min(q_hi, h1);
    window_queries(kt, min(Nk, kt + 16), Mq, l1, h1);
    wq_lo = max(wq_lo, l1);
    wq_hi = min(wq_hi, h1);
  }
  if (BIAS == ATTN_BIAS_BINS)
    for (int k = threadIdx.x; k < 68; k += AT_NT) s_pw[k] = LOG2E * a.pos_w[h * 68 + k];
  ScoreBias<T, BIAS> bias;
  bias.bins = a.bins ? a.bins + (size_t)b * Mq * Nk : nullptr;
  bias.pw2 = s_pw;
  bias.bias = nullptr;
  if (BIAS == ATTN_BIAS_DENSE) bias.bias = reinterpret_cast<const T*>(a.bias) + (size_t)bh * Mq * Nk;
  if (BIAS == ATTN_BIAS_WINDOW) bias.bias = reinterpret_cast<const T*>(a.bias);
  bias.Nk = Nk;
  bias.H = a.H;
  bias.h = h;

  typename M::Frag kf, vf;
  frag_rows<T, DP>(kf, Kg, a.ksn, kj, Nk, a.d, lane);
  frag_rows<T, DP>(vf, Vg, a.ksn, kj, Nk, a.d, lane);
  const bool active = kt < Nk;
  const bool kok = kj < Nk && (!a.kmask || a.kmask[(size_t)b * Nk + kj] > 0.5f);
  f32x4 dk[NC], dv[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) dk[c] = dv[c] = f32x4{0.f, 0.f, 0.f, 0.f};
  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};

  for (int c0 = q_lo; c0 < q_hi; c0 += CH) {
    __syncthreads();
    stage_rm<T, DP>(Qs, Qg, a.qsn, c0, Mq, a.d);
    stage_rm<T, DP>(dOs, dOw, DP, c0, Mq, DP);
    stage_tr<T, DP>(QTs, Qg, a.qsn, c0, Mq, a.d);
    stage_tr<T, DP>(dOTs, dOw, DP, c0, Mq, DP);
    for (int j = threadIdx.x; j < CH + 32; j += AT_NT) {
      const int q = c0 + j;
      const bool ok = j < CH && q < q_hi && (!a.qmask || a.qmask[(size_t)b * Mq + q] > 0.5f);
      lse2[j] = ok ? a.lse[(size_t)bh * Mq + q] * LOG2E : POS_BIG;
      Dq[j] = ok ? a.dcoef[(size_t)bh * Mq + q] : 0.f;
    }
    __syncthreads();
    if (!active) continue;
    const int t_lo = max(c0, wq_lo), t_hi = min(c0 + CH, wq_hi);
    for (int qp = t_lo; qp < t_hi; qp += 32) {
      f32x4 p[2], ds[2];
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        const int qt2 = qp + 16 * hf;
        p[hf] = ds[hf] = zero;
        if (qt2 < t_hi) {
          typename M::Frag qa, da;
          M::load(qa, Qs + (size_t)(qt2 - c0 + (lane & 15)) * DP, lane);
          M::load(da, dOs + (size_t)(qt2 - c0 + (lane & 15)) * DP, lane);
          const f32x4 s = M::qk(qa, kf, zero);
          const f32x4 dp = M::qk(da, vf, zero);
          const f32x4 l2 = *reinterpret_cast<const f32x4*>(lse2 + qt2 - c0 + 4 * g);
          const f32x4 dd = *reinterpret_cast<const f32x4*>(Dq + qt2 - c0 + 4 * g);
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int q = qt2 + 4 * g + r;
            float pv = 0.f;
            if (kok && l2[r] < 0.5f * POS_BIG && q < t_hi) {
              float xv = s[r] * sc;
              if (BIAS != ATTN_BIAS_NONE) xv += bias(q, kj);
              pv = fast_exp2(xv - l2[r]);
            }
            p[hf][r] = pv;
            ds[hf][r] = pv * (dp[r] - dd[r]);
          }
        }
      }
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        dv[c] = M::pvt(p[0], p[1], dOTs + (size_t)(c * 16 + (lane & 15)) * TS + (qp - c0), lane, dv[c]);
        dk[c] = M::pvt(ds[0], ds[1], QTs + (size_t)(c * 16 + (lane & 15)) * TS + (qp - c0), lane, dk[c]);
      }
    }
  }
  if (!active || kj >= Nk) return;
  // lane holds dK^T / dV^T [col = c*16 + 4g + r][key kj]
  if (a.qsplit > 1) {
    float* part = a.kv_part + (((size_t)blockIdx.z * a.B * a.H + bh) * Nk + kj) * 2 * DP;
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int col = c * 16 + 4 * g + r;
        part[col] = a.scale * dk[c][r];
        part[DP + col] = dv[c][r];
      }
    return;
  }
  T* dK = reinterpret_cast<T*>(a.dk) + ((size_t)bh * Nk + kj) * a.d;
  T* dV = reinterpret_cast<T*>(a.dv) + ((size_t)bh * Nk + kj) * a.d;
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int col = c * 16 + 4 * g + r;
      if (col < a.d) {
        dK[col] = from_f32<T>(a.scale * dk[c][r]);
        dV[col] = from_f32<T>(dv[c][r]);
      }
    }
}

// ===========================================================================
// dQ and bias gradients: a wave owns a 16-query tile; keys stream.  grid (ceil(Mq/64), B*H).
template <typename T, int DP, int BIAS>
__global__ void __launch_bounds__(AT_NT) attn_bwd_q_kernel(AttnArgs a) {
  using M = Mfma<T, DP>;
  constexpr int CH = AtGeo<T, DP>::CH, TS = AtGeo<T, DP>::TS;
  constexpr int NC = DP / 16;
  __shared__ __align__(16) T Ks[CH * DP];
  __shared__ __align__(16) T Vs[CH * DP];
  __shared__ __align__(16) T KTs[DP * TS];
  __shared__ __align__(16) float kb[CH + 32];
  __shared__ float s_pw[68];
  __shared__ float s_dpw[68];
  const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE, g = lane >> 4;
  const int bh = blockIdx.y, b = bh / a.H, h = bh % a.H;
  const int Mq = a.Mq, Nk = a.Nk;
  const int q0 = blockIdx.x * AT_RB;
  const int qt = q0 + 16 * wave;
  const int qi = qt + (lane & 15);
  const T* Qg = reinterpret_cast<const T*>(a.q) + (size_t)b * a.qsb + (size_t)h * a.qsh;
  const T* Kg = reinterpret_cast<const T*>(a.k) + (size_t)b * a.ksb + (size_t)h * a.ksh;
  const T* Vg = reinterpret_cast<const T*>(a.v) + (size_t)b * a.ksb + (size_t)h * a.ksh;
  const T* dOw = reinterpret_cast<const T*>(a.do_w) + (size_t)bh * Mq * DP;
  const float sc = a.scale * LOG2E;

  int k_lo = 0, k_hi = Nk, wk_lo = 0, wk_hi = Nk;
  if (a.window) {
    int l1, h1, l2, h2;
    window_keys(q0, Nk, l1, h1);
    window_keys(min(q0 + AT_RB, Mq) - 1, Nk, l2, h2);
    k_lo = l1;
    k_hi = h2;
    window_keys(qt, Nk, wk_lo, wk_hi);
  }
  if (BIAS == ATTN_BIAS_BINS)
    for (int k = threadIdx.x; k < 68; k += AT_NT) {
      s_pw[k] = LOG2E * a.pos_w[h * 68 + k];
      s_dpw[k] = 0.f;
    }
  ScoreBias<T, BIAS> bias;
  bias.bins = a.bins ? a.bins + (size_t)b * Mq * Nk : nullptr;
  bias.pw2 = s_pw;
  bias.bias = nullptr;
  if (BIAS == ATTN_BIAS_DENSE) bias.bias = reinterpret_cast<const T*>(a.bias) + (size_t)bh * Mq * Nk;
  if (BIAS == ATTN_BIAS_WINDOW) bias.bias = reinterpret_cast<const T*>(a.bias);
  bias.Nk = Nk;
  bias.H = a.H;
  bias.h = h;
  T* dbias = nullptr;
  if (a.dbias && BIAS == ATTN_BIAS_DENSE) dbias = reinterpret_cast<T*>(a.dbias) + (size_t)bh * Mq * Nk;
  if (a.dbias && BIAS == ATTN_BIAS_WINDOW) dbias = reinterpret_cast<T*>(a.dbias);

  typename M::Frag qf, df;
  frag_rows<T, DP>(qf, Qg, a.qsn, qi, Mq, a.d, lane);
  frag_rows<T, DP>(df, dOw, DP, qi, Mq, DP, lane);
  const bool active = qt < Mq;
  const bool qrow = qi < Mq;
  const bool qok = qrow && (!a.qmask || a.qmask[(size_t)b * Mq + qi] > 0.5f);
  const float l2 = qok ? a.lse[(size_t)bh * Mq + qi] * LOG2E : POS_BIG;
  const float Di = qok ? a.dcoef[(size_t)bh * Mq + qi] : 0.f;
  f32x4 dq[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) dq[c] = f32x4{0.f, 0.f, 0.f, 0.f};
  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};

  for (int c0 = k_lo; c0 < k_hi; c0 += CH) {
    __syncthreads();
    stage_rm<T, DP>(Ks, Kg, a.ksn, c0, Nk, a.d);
    stage_rm<T, DP>(Vs, Vg, a.ksn, c0, Nk, a.d);
    stage_tr<T, DP>(KTs, Kg, a.ksn, c0, Nk, a.d);
    for (int j = threadIdx.x; j < CH + 32; j += AT_NT) {
      const int key = c0 + j;
      const bool ok = j < CH && key < k_hi && (!a.kmask || a.kmask[(size_t)b * Nk + key] > 0.5f);
      kb[j] = ok ? 0.f : NEG_BIG;
    }
    __syncthreads();
    if (!active) continue;
    const int t_lo = max(c0, wk_lo), t_hi = min(c0 + CH, wk_hi);
    for (int kp = t_lo; kp < t_hi; kp += 32) {
      f32x4 ds[2];
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        const int kt2 = kp + 16 * hf;
        ds[hf] = zero;
        if (kt2 < t_hi) {
          typename M::Frag ka, va;
          M::load(ka, Ks + (size_t)(kt2 - c0 + (lane & 15)) * DP, lane);
          M::load(va, Vs + (size_t)(kt2 - c0 + (lane & 15)) * DP, lane);
          const f32x4 s = M::qk(ka, qf, zero);
          const f32x4 dp = M::qk(va, df, zero);
          const f32x4 kbv = *reinterpret_cast<const f32x4*>(kb + kt2 - c0 + 4 * g);
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int key = kt2 + 4 * g + r;
            float dsv = 0.f;
            if (qok && kbv[r] == 0.f && key < t_hi) {
              float xv = s[r] * sc;
              if (BIAS != ATTN_BIAS_NONE) xv += bias(qi, key);
              const float pv = fast_exp2(xv - l2);
              dsv = pv * (dp[r] - Di);
            }
            ds[hf][r] = dsv;
            if (BIAS == ATTN_BIAS_BINS && dsv != 0.f) {
              const unsigned bk = (unsigned)bias.bins[(size_t)qi * Nk + key];
              if (bk < 68u) atomicAdd(&s_dpw[bk], dsv);
            }
            if (dbias && qrow && key < t_hi) {
              if (BIAS == ATTN_BIAS_DENSE) dbias[(size_t)qi * Nk + key] = from_f32<T>(dsv);
              if (BIAS == ATTN_BIAS_WINDOW) {
                const int w = qi / ATTN_WQ;
                dbias[(((size_t)w * a.H + h) * ATTN_WQ + (qi - ATTN_WQ * w)) * ATTN_WK +
                      (key - (ATTN_WQ * w - ATTN_WOFF))] = from_f32<T>(dsv);
              }
            }
          }
        }
      }
#pragma unroll
      for (int c = 0; c < NC; ++c)
        dq[c] = M::pvt(ds[0], ds[1], KTs + (size_t)(c * 16 + (lane & 15)) * TS + (kp - c0), lane, dq[c]);
    }
  }
  if (BIAS == ATTN_BIAS_BINS) {
    __syncthreads();
    for (int k = threadIdx.x; k < 68; k += AT_NT)
      a.dpw_part[((size_t)bh * gridDim.x + blockIdx.x) * 68 + k] = s_dpw[k];
  }
  if (!active || !qrow) return;
  T* dQ = reinterpret_cast<T*>(a.dq) + ((size_t)bh * Mq + qi) * a.d;
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int col = c * 16 + 4 * g + r;
      if (col < a.d) dQ[col] = from_f32<T>(a.scale * dq[c][r]);
    }
}

// dK / dV from query-split partials; d pos_weight from per-workgroup partials (fixed order).
template <typename T, int DP>
__global__ void __launch_bounds__(256) attn_bwd_finalize_kernel(AttnArgs a, int n_qblocks) {
  const size_t e = (size_t)blockIdx.x * 256 + threadIdx.x;
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
template <typename T, int DP, int BIAS>
static hipError_t attn_fwd_t(const AttnArgs& a, hipStream_t s) {
  dim3 grid((a.Mq + AT_RB - 1) / AT_RB, a.B * a.H);
  hipLaunchKernelGGL((attn_fwd_kernel<T, DP, BIAS>), grid, dim3(AT_NT), 0, s, a);
  return hipGetLastError();
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

template <typename T, int DP, int BIAS>
static hipError_t attn_bwd_t(const AttnArgs& a, hipStream_t s) {
  const size_t rows = (size_t)a.B * a.H * a.Mq;
  hipLaunchKernelGGL((attn_bwd_prep_kernel<T, DP>), dim3((unsigned)((rows * DP + 255) / 256)), dim3(256), 0, s, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  dim3 gkv((a.Nk + AT_RB - 1) / AT_RB, a.B * a.H, a.qsplit);
  hipLaunchKernelGGL((attn_bwd_kv_kernel<T, DP, BIAS>), gkv, dim3(AT_NT), 0, s, a);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  const int nqb = (a.Mq + AT_RB - 1) / AT_RB;
  dim3 gq(nqb, a.B * a.H);
  hipLaunchKernelGGL((attn_bwd_q_kernel<T, DP, BIAS>), gq, dim3(AT_NT), 0, s, a);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  if (a.qsplit > 1 || (BIAS == ATTN_BIAS_BINS && a.dpos_w)) {
    const size_t n = std::max((size_t)a.B * a.H * a.Nk * a.d, (size_t)a.H * 68);
    hipLaunchKernelGGL((attn_bwd_finalize_kernel<T, DP>), dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, a,
                       nqb);
    e = hipGetLastError();
  }
  return e;
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
