// Sweep engine shared by the Sinkhorn forward and backward kernels.
//
// A "sweep" visits, for every resident 16-row tile owned by this workgroup, all
// streamed 16-row tiles of the same (b,h): the cost tile QK^T is recomputed on
// MFMA from LDS-resident operands and reduced on the fly.  In a row sweep the
// resident rows are Q (plan rows i) and the streamed rows are K (plan columns
// j); in a column sweep the roles swap.
#pragma once
#include "common.h"

namespace dfl {

constexpr int SK_NT = 256;
constexpr int SK_NW = SK_NT / WAVE;
constexpr int SK_RT = 4;  // resident tiles per register chunk

// Position-bin / geometry bias of the cost, in log2 units of the logit:
//   bias(i, j) = -(log2 e / eps) * (pw[bins_ij] + w * d_ij / (r0 + d_ij)).
struct Bias {
  const int* bins;    // (N, N) of this batch row, or null
  const float* posw;  // LDS: 68 pre-scaled weights of this head
  const float* xs;    // LDS: coordinates [Np][3], or null (no geometry term)
  float geo_scale;    // -log2e * w / eps
  float r0;
  int N;
  __device__ __forceinline__ float operator()(int i, int j) const {
    float b = 0.f;
    if (bins) b += posw[bins[(size_t)i * N + j]];
    if (xs) {
      const float dx = xs[3 * i] - xs[3 * j], dy = xs[3 * i + 1] - xs[3 * j + 1], dz = xs[3 * i + 2] - xs[3 * j + 2];
      const float dist = sqrtf(dx * dx + dy * dy + dz * dz);
      b += geo_scale * dist / (r0 + dist);
    }
    return b;
  }
};

// Stage rows [0, n) of a row-strided slice into LDS row-major [Np][DP]
// (zero-filling columns >= d and rows >= n).
template <typename T, int DP>
__device__ void stage_rows(T* dst, const T* __restrict__ src, long long sn, int n, int d, int Np) {
  for (int e = threadIdx.x; e < Np * DP; e += blockDim.x) {
    const int row = e / DP, col = e - row * DP;
    T v = from_f32<T>(0.f);
    if (row < n && col < d) v = src[(size_t)row * sn + col];
    dst[e] = v;
  }
}
// Transposed: dst[col][row], row stride Np.
template <typename T, int DP>
__device__ void stage_rows_t(T* dst, const T* __restrict__ src, long long sn, int n, int d, int Np) {
  for (int e = threadIdx.x; e < Np * DP; e += blockDim.x) {
    const int col = e / Np, row = e - col * Np;
    T v = from_f32<T>(0.f);
    if (row < n && col < d) v = src[(size_t)row * sn + col];
    dst[e] = v;
  }
}

// QK-type fragment of row `row` read straight from global memory (zero outside
// rows [0, n) and columns [0, d)).
template <typename T, int DP>
__device__ __forceinline__ void load_frag_global(typename Mfma<T, DP>::Frag& f, const T* __restrict__ src,
                                                 long long sn, int row, int n, int d, int lane) {
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

// Valid-token bookkeeping: n_hi = 1 + last valid index; valid[] bytes in LDS.
__device__ __forceinline__ int mask_setup(const float* mask, int N, unsigned char* valid, int* s_tmp) {
  if (threadIdx.x == 0) *s_tmp = 0;
  __syncthreads();
  int hi = 0;
  for (int i = threadIdx.x; i < N; i += blockDim.x) {
    const bool ok = mask ? (mask[i] > 0.5f) : true;
    valid[i] = ok ? 1 : 0;
    if (ok) hi = i + 1;
  }
  atomicMax(s_tmp, hi);
  __syncthreads();
  const int n = *s_tmp;
  __syncthreads();
  return n;
}

// Gather a published vector and convert it into log2-unit LDS form, pinning
// invalid entries (and the tail [n, Np)) to NEG_BIG.
__device__ __forceinline__ bool gather_potential(const uint64_t* buf, int n, int Np, uint32_t tag, float* dst,
                                                 const unsigned char* valid, uint32_t* err, int* s_flag) {
  if (!xch_gather<SK_NT>(buf, n, tag, dst, LOG2E, err, s_flag)) return false;
  for (int i = threadIdx.x; i < Np; i += SK_NT)
    if (i >= n || !valid[i]) dst[i] = NEG_BIG;
  __syncthreads();
  return true;
}

// Online log2-sum-exp of x_ij = sc * <res_i, str_j> + w2_j (+ bias) over all
// streamed rows j, for each resident row of tiles [rt0, rt0 + nr).  TRANS: the
// streamed index is the plan's row index (column sweep), which matters only
// for the bias.  lse2[q] (and mx2[q] if non-null) receive the result for local
// resident row q in [0, nr*16).  Called by the whole block.
template <typename T, int DP, bool GENERAL, bool TRANS>
__device__ void lse_sweep(const T* __restrict__ res_lds, const T* __restrict__ str_lds,
                          const float* __restrict__ w2, int n_str_tiles, int rt0, int nr, float sc,
                          const Bias& bias, float* lse2, float* mx2, float* scratch) {
  using M = Mfma<T, DP>;
  const int lane = threadIdx.x & (WAVE - 1);
  const int wave = threadIdx.x / WAVE;
  const int g = lane >> 4;
  for (int c0 = 0; c0 < nr; c0 += SK_RT) {
    const int nc = min(SK_RT, nr - c0);
    typename M::Frag bf[SK_RT];
#pragma unroll
    for (int r = 0; r < SK_RT; ++r)
      if (r < nc) M::load(bf[r], res_lds + (size_t)((rt0 + c0 + r) * 16 + (lane & 15)) * DP, lane);
    float m[SK_RT], s[SK_RT];
#pragma unroll
    for (int r = 0; r < SK_RT; ++r) { m[r] = NEG_BIG; s[r] = 0.f; }
    for (int st = wave; st < n_str_tiles; st += SK_NW) {
      typename M::Frag af;
      M::load(af, str_lds + (size_t)(st * 16 + (lane & 15)) * DP, lane);
      const f32x4 w = *reinterpret_cast<const f32x4*>(w2 + st * 16 + 4 * g);
#pragma unroll
      for (int r = 0; r < SK_RT; ++r) {
        if (r < nc) {
          const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
          const f32x4 acc = M::qk(af, bf[r], zero);
          float x[4];
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            x[k] = __builtin_fmaf(acc[k], sc, w[k]);
            if (GENERAL) {
              const int ires = (rt0 + c0 + r) * 16 + (lane & 15);
              const int jstr = st * 16 + 4 * g + k;
              if (w[k] > 0.5f * NEG_BIG) x[k] += TRANS ? bias(jstr, ires) : bias(ires, jstr);
            }
          }
          const float tm = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
          const float mn = fmaxf(m[r], tm);
          float acc_s = s[r] * fast_exp2(m[r] - mn);
#pragma unroll
          for (int k = 0; k < 4; ++k) acc_s += fast_exp2(x[k] - mn);
          s[r] = acc_s;
          m[r] = mn;
        }
      }
    }
#pragma unroll
    for (int r = 0; r < SK_RT; ++r) {
      if (r < nc) {
        const float mm = max_groups(m[r]);
        const float ss = sum_groups(s[r] * fast_exp2(m[r] - mm));
        if (lane < 16) {
          scratch[(wave * SK_RT + r) * 16 + lane] = mm;
          scratch[SK_NW * SK_RT * 16 + (wave * SK_RT + r) * 16 + lane] = ss;
        }
      }
    }
    __syncthreads();
    if ((int)threadIdx.x < nc * 16) {
      const int q = threadIdx.x;
      const int r = q >> 4, l = q & 15;
      float mm = NEG_BIG;
#pragma unroll
      for (int w = 0; w < SK_NW; ++w) mm = fmaxf(mm, scratch[(w * SK_RT + r) * 16 + l]);
      float ss = 0.f;
#pragma unroll
      for (int w = 0; w < SK_NW; ++w)
        ss += scratch[SK_NW * SK_RT * 16 + (w * SK_RT + r) * 16 + l] * fast_exp2(scratch[(w * SK_RT + r) * 16 + l] - mm);
      lse2[c0 * 16 + q] = mm + fast_log2(ss);
      if (mx2) mx2[c0 * 16 + q] = mm;
    }
    __syncthreads();
  }
}

// Scratch floats needed by lse_sweep.
constexpr int LSE_SCRATCH = 2 * SK_NW * SK_RT * 16;

// Stripe of 16-row tiles owned by `member` out of G.
__device__ __forceinline__ void stripe(int n_tiles, int member, int G, int& t0, int& t1) {
  t0 = (int)((long long)n_tiles * member / G);
  t1 = (int)((long long)n_tiles * (member + 1) / G);
}

}  // namespace dfl
