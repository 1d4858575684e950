// Flash-Sinkhorn IFT backward on gfx950 (persistent per-(b,h) workgroup groups).
//
// Restates FlashSinkhornAttn.backward of vv137/deepfold-linear
// (src/deepfold/model/kernels/flash_sinkhorn_attn.py:246-667) per (b,h), on the
// valid tokens only (the reference ignores the mask; per-sample evaluation on the
// unpadded slice is the consistent definition):
//
//   gO = sigma(G) dO,  dG = sigma(1-sigma) O_avg dO,  D_i = gO_i.O_i + dxc_i.xc_i
//   T_ij = exp(u_i + L_ij + v_j - logZ_i)      (= S_row_ij)
//   S_col_ij = exp(L_ij + u_i - col_lse_j)      (= T_ij r_i / c_j)
//   gls = T (dT - D_i),  dT_ij = gO_i.V_j + dxc_i.x_j,  g_v = sum_i gls
//   (I - kappa^2 S_row^T S_col) z_v = g_v,  z_u = kappa S_col z_v
//   dC = -(1/eps) gls - (kappa/eps) z_u_i S_row + sgn (kappa/eps) z_v_j S_col
//        (sgn = -1 reference, +1 analytic adjoint)
//   dQ = -(1/sqrt d) dC K,  dK = -(1/sqrt d) dC^T Q,  dV = T^T gO, ...
//
// Phases inside one launch:
//   P0  prologue: D_i for all rows, dG for my rows
//   C1  column pass (resident j): g_v, dV, dx transport term      -> exchange g_v
//   S   solve: reference Gauss-Seidel sweeps, or CG on
//       (I - kappa^2 W^T W) y = D_c^{-1/2} g_v,  W = D_r^{-1/2} T D_c^{-1/2},
//       one exchange per half-step; CG vectors are kept redundantly (and
//       bit-identically) in every member
//   R2  row pass (resident i): dQ, dx_i cost term, d w_dist, d pos_weight
//   C2  column pass (resident j): dK, dx_j cost term
// The heavy passes (C1, R2, C2) stream their operands through LDS in chunks.
// Two storage modes (template flag STREAM):
//   resident: the solve keeps Q and K of the whole (b,h) in LDS, and every
//             length-N vector (potentials, D, g_v, z, CG vectors) lives in LDS;
//   stream  : for long sequences the solve keeps only the member's Q and K
//             stripes in LDS and streams the other operand from zero-padded
//             global copies; the length-N vectors live in a per-workgroup region
//             of the workspace (L1/L2-resident).
#pragma once
#include "sinkhorn_args.h"
#include "sinkhorn_engine.h"

#include <algorithm>
#include <type_traits>

namespace dfl {

constexpr int BWD_NT = 512;             // 8 waves: two per SIMD
constexpr int BWD_NW = BWD_NT / WAVE;
// Resident tiles per wave in the heavy passes: two at d <= 32; one at d = 64,
// where two tiles' fragments and accumulators exceed the register file.
template <int DP> constexpr int bwd_maxt() { return DP <= 32 ? 2 : 1; }
constexpr int BWD_SCRATCH = sweep_scratch<BWD_NT>();
constexpr int BWD_STREAM_SCRATCH = stream_scratch<BWD_NT>();
// Length-Np float vectors of one workgroup: 13 vectors + coordinates and
// grad x_centroid ([Np][3] each).  Stream mode keeps them in the workspace.
constexpr int BWD_STREAM_VECS = 13 + 6;

// ---------------------------------------------------------------------------
// Weighted sum of resident storage: out[q] = sum_j exp2(sc*<res_q, str_j> + cres[q]
// + w2_j (+bias)) * z_j over the streamed tiles.  Every exponent is <= 0 here (S_col,
// T and W are bounded by 1), so no shift.  NR resident tiles known at compile time
// (the CG and fixed-point matvecs): resident fragments and row constants
// are loaded once, all NR * SCH MFMAs of a slot group are issued before the
// exponentials, and each resident tile keeps four independent accumulators (one per
// accumulator row of a lane) instead of one dependent chain.  Slots past the wave's
// last streamed tile re-read tile `wave` with w = NEG_BIG and z = 0.
template <typename T, int DP, int NR, bool GENERAL, bool TRANS>
__device__ __forceinline__ void lean_wsum_chunk(const T* __restrict__ res_lds, const T* __restrict__ str_lds,
                                                const float* __restrict__ w2, const float* __restrict__ zv,
                                                int n_str_tiles, int rt0, int q0, float sc,
                                                const float* __restrict__ cres, const Bias& bias, float* out,
                                                float* scratch) {
  using M = Mfma<T, DP>;
  constexpr int SCH = sweep_sch<T, DP>();
  const int lane = threadIdx.x & (WAVE - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE);
  const int g = lane >> 4;
  const float isc = 1.f / sc;
  const int ks = wave < n_str_tiles ? (n_str_tiles - wave + BWD_NW - 1) / BWD_NW : 0;
  typename M::Frag bf[NR];
  f32x4 ci[NR];
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    M::load(bf[r], res_lds + (size_t)((rt0 + r) * 16 + (lane & 15)) * DP, lane);
    const float c = cres[q0 + r * 16 + (lane & 15)] * isc;
    ci[r] = f32x4{c, c, c, c};
  }
  float s[NR][4];
#pragma unroll
  for (int r = 0; r < NR; ++r)
#pragma unroll
    for (int e = 0; e < 4; ++e) s[r][e] = 0.f;
  for (int k0 = 0; k0 < ks; k0 += SCH) {
    typename M::Frag af[SCH];
    f32x4 w[SCH], z[SCH];
#pragma unroll
    for (int k = 0; k < SCH; ++k) {
      const bool live = k0 + k < ks;
      const int st = live ? wave + BWD_NW * (k0 + k) : wave;
      M::load(af[k], str_lds + (size_t)(st * 16 + (lane & 15)) * DP, lane);
      w[k] = *reinterpret_cast<const f32x4*>(w2 + st * 16 + 4 * g);
      z[k] = *reinterpret_cast<const f32x4*>(zv + st * 16 + 4 * g);
      if (!live) {
        w[k] = f32x4{NEG_BIG, NEG_BIG, NEG_BIG, NEG_BIG};
        z[k] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
    }
    f32x4 x[NR][SCH];
#pragma unroll
    for (int r = 0; r < NR; ++r)
#pragma unroll
      for (int k = 0; k < SCH; ++k) x[r][k] = M::qk(af[k], bf[r], ci[r]);  // independent MFMAs
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      f32x4 bv[SCH];
      if (GENERAL) {  // dead slots repeat tile `wave` (their w is NEG_BIG)
        int s0[SCH];
#pragma unroll
        for (int k = 0; k < SCH; ++k) s0[k] = (k0 + k < ks ? wave + BWD_NW * (k0 + k) : wave) * 16 + 4 * g;
        bias.template quads<TRANS>((rt0 + r) * 16 + (lane & 15), s0, bv);
      }
#pragma unroll
      for (int k = 0; k < SCH; ++k)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float xv = __builtin_fmaf(x[r][k][e], sc, w[k][e]);
          if (GENERAL) xv += bv[k][e];
          s[r][e] = __builtin_fmaf(fast_exp2(xv), z[k][e], s[r][e]);
        }
    }
  }
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    const float ss = sum_groups((s[r][0] + s[r][1]) + (s[r][2] + s[r][3]));
    if (lane < 16) scratch[(wave * NR + r) * 16 + lane] = ss;
  }
  __syncthreads();
  if ((int)threadIdx.x < NR * 16) {
    const int q = threadIdx.x, r = q >> 4, l = q & 15;
    float ss = 0.f;
#pragma unroll
    for (int w_ = 0; w_ < BWD_NW; ++w_) ss += scratch[(w_ * NR + r) * 16 + l];
    out[q0 + q] = ss;
  }
  __syncthreads();
}

// The weighted sum with a bias (position bins or geometry): out[q] = sum_j exp2(sc*<res_q,
// str_j> + cres[q] + w2_j + bias_qj) * z_j, one pass over a wave's streamed slots for up to
// SK_RT resident tiles, the tiles in a runtime loop that computes one tile's biases at a
// time (the compile-time chunks of lean_wsum_chunk hold two tiles' biases at most, and
// their second pass over the streamed slots made the full-cost backward 9% slower).
// Every exponent is <= 0 here (S_col, T and W are bounded by 1), so no shift.
template <typename T, int DP, bool GENERAL, bool TRANS>
__device__ __forceinline__ void bias_wsum(const T* __restrict__ res_lds, const T* __restrict__ str_lds,
                            const float* __restrict__ w2, const float* __restrict__ zv, int n_str_tiles, int rt0,
                            int nr, float sc, const float* __restrict__ cres, const Bias& bias, float* out,
                            float* scratch) {
  using M = Mfma<T, DP>;
  constexpr int SCH = sweep_sch<T, DP>();
  const int lane = threadIdx.x & (WAVE - 1);
  const int wave = threadIdx.x / WAVE;
  const int g = lane >> 4;
  const float isc = 1.f / sc;
  const int ks = wave < n_str_tiles ? (n_str_tiles - wave + BWD_NW - 1) / BWD_NW : 0;
  for (int c0 = 0; c0 < nr; c0 += SK_RT) {
    const int nc = min(SK_RT, nr - c0);
    float s[SK_RT];
#pragma unroll
    for (int r = 0; r < SK_RT; ++r) s[r] = 0.f;
    for (int k0 = 0; k0 < ks; k0 += SCH) {
      // streamed fragments, column terms and weights stay in registers for all
      // resident tiles; slots past the wave's last tile carry w = NEG_BIG (no
      // bias lookup, exp2 -> 0) and z = 0
      typename M::Frag af[SCH];
      f32x4 w[SCH], z[SCH];
#pragma unroll
      for (int k = 0; k < SCH; ++k) {
        const bool live = k0 + k < ks;
        const int st = live ? wave + BWD_NW * (k0 + k) : wave;
        M::load(af[k], str_lds + (size_t)(st * 16 + (lane & 15)) * DP, lane);
        w[k] = *reinterpret_cast<const f32x4*>(w2 + st * 16 + 4 * g);
        z[k] = *reinterpret_cast<const f32x4*>(zv + st * 16 + 4 * g);
        if (!live) {
          w[k] = f32x4{NEG_BIG, NEG_BIG, NEG_BIG, NEG_BIG};
          z[k] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
      }
#pragma unroll
      for (int r = 0; r < SK_RT; ++r) {
        if (r >= nc) continue;
        typename M::Frag bf;
        M::load(bf, res_lds + (size_t)((rt0 + c0 + r) * 16 + (lane & 15)) * DP, lane);
        const float ci = cres[(c0 + r) * 16 + (lane & 15)] * isc;
        const f32x4 cinit = f32x4{ci, ci, ci, ci};
        f32x4 bv[SCH];
        if (GENERAL) {  // dead slots repeat tile `wave` (their w is NEG_BIG)
          int s0[SCH];
#pragma unroll
          for (int k = 0; k < SCH; ++k) s0[k] = (k0 + k < ks ? wave + BWD_NW * (k0 + k) : wave) * 16 + 4 * g;
          bias.template quads<TRANS>((rt0 + c0 + r) * 16 + (lane & 15), s0, bv);
        }
        f32x4 x[SCH];
#pragma unroll
        for (int k = 0; k < SCH; ++k) x[k] = M::qk(af[k], bf, cinit);  // independent MFMAs
        float acc_s = 0.f;
#pragma unroll
        for (int k = 0; k < SCH; ++k) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            float xv = __builtin_fmaf(x[k][e], sc, w[k][e]);
            if (GENERAL) xv += bv[k][e];
            acc_s = __builtin_fmaf(fast_exp2(xv), z[k][e], acc_s);
          }
        }
        s[r] += acc_s;
      }
    }
#pragma unroll
    for (int r = 0; r < SK_RT; ++r)
      if (r < nc) {
        const float ss = sum_groups(s[r]);
        if (lane < 16) scratch[(wave * SK_RT + r) * 16 + lane] = ss;
      }
    __syncthreads();
    if ((int)threadIdx.x < nc * 16) {
      const int q = threadIdx.x, r = q >> 4, l = q & 15;
      float ss = 0.f;
#pragma unroll
      for (int w = 0; w < BWD_NW; ++w) ss += scratch[(w * SK_RT + r) * 16 + l];
      out[c0 * 16 + q] = ss;
    }
    __syncthreads();
  }
}

// lean_wsum_chunk over the nr resident tiles [rt0, rt0 + nr), chunks of at most 4
// tiles; with a bias, bias_wsum.
template <typename T, int DP, bool GENERAL, bool TRANS>
__device__ __forceinline__ void lean_wsum(const T* res_lds, const T* str_lds, const float* w2, const float* zv,
                                          int n_str_tiles, int rt0, int nr, float sc, const float* cres,
                                          const Bias& bias, float* out, float* scratch) {
  if constexpr (GENERAL) {
    bias_wsum<T, DP, GENERAL, TRANS>(res_lds, str_lds, w2, zv, n_str_tiles, rt0, nr, sc, cres, bias, out, scratch);
    return;
  }
  constexpr int CMAX = 4;
  for (int c0 = 0; c0 < nr; c0 += CMAX) {
    const int nc = min(CMAX, nr - c0);
    if (CMAX == 4 && nc == 4)
      lean_wsum_chunk<T, DP, CMAX, GENERAL, TRANS>(res_lds, str_lds, w2, zv, n_str_tiles, rt0 + c0, c0 * 16, sc,
                                                   cres, bias, out, scratch);
    else if (CMAX == 4 && nc == 3)
      lean_wsum_chunk<T, DP, CMAX - 1, GENERAL, TRANS>(res_lds, str_lds, w2, zv, n_str_tiles, rt0 + c0, c0 * 16,
                                                       sc, cres, bias, out, scratch);
    else if (nc == 2)
      lean_wsum_chunk<T, DP, 2, GENERAL, TRANS>(res_lds, str_lds, w2, zv, n_str_tiles, rt0 + c0, c0 * 16, sc, cres,
                                                bias, out, scratch);
    else
      lean_wsum_chunk<T, DP, 1, GENERAL, TRANS>(res_lds, str_lds, w2, zv, n_str_tiles, rt0 + c0, c0 * 16, sc, cres,
                                                bias, out, scratch);
  }
}

// ---------------------------------------------------------------------------
// Register storage of the CG matrix.  During the CG solve W_ij = exp2(sc q_i.k_j +
// alpha_i + beta_j (+ bias_ij)) does not change, so each wave computes its tiles once,
// in lean_wsum's work split (resident tile r < nr of the stripe against streamed tile
// wave + BWD_NW k, k < KS; tiles it lacks hold 0), for both orientations, and every
// matvec is one fma per element.  KS = bwd_reg_ks(n_tiles) (2, 4 or 6) and nr <=
// bwd_reg_nrm(KS), the limits of the forward's register mode.
__host__ __device__ constexpr int bwd_reg_ks(int n_tiles) {
  return (n_tiles + 7) / 8 <= 2 ? 2 : ((n_tiles + 7) / 8 <= 4 ? 4 : ((n_tiles + 7) / 8 <= 6 ? 6 : 0));
}
__host__ __device__ constexpr int bwd_reg_nrm(int ks) { return ks == 6 ? 3 : 4; }
constexpr int BWD_REG_SLOTS = 18;  // max over KS of bwd_reg_nrm(KS) * KS

// W tiles of one orientation: resident rows of res_lds (cres: their constant), streamed
// rows of str_lds (w2: their constant), the expression of lean_wsum_chunk / bias_wsum.
template <typename T, int DP, int KS, bool GENERAL, bool TRANS>
__device__ __forceinline__ void reg_wtiles(f32x4 (&W)[BWD_REG_SLOTS], const T* __restrict__ res_lds,
                                           const T* __restrict__ str_lds, const float* __restrict__ w2,
                                           int n_str_tiles, int rt0, int nr, float sc,
                                           const float* __restrict__ cres, const Bias& bias) {
  using M = Mfma<T, DP>;
  constexpr int NRM = bwd_reg_nrm(KS);
  const int lane = threadIdx.x & (WAVE - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE);
  const int g = lane >> 4;
  const float isc = 1.f / sc;
#pragma unroll
  for (int r = 0; r < NRM; ++r) {
#pragma unroll
    for (int k = 0; k < KS; ++k) {
      const int sl = r * KS + k, st = wave + BWD_NW * k;
      W[sl] = f32x4{0.f, 0.f, 0.f, 0.f};
      if (r < nr && st < n_str_tiles) {
        typename M::Frag af, bf;
        M::load(bf, res_lds + (size_t)((rt0 + r) * 16 + (lane & 15)) * DP, lane);
        M::load(af, str_lds + (size_t)(st * 16 + (lane & 15)) * DP, lane);
        const float c = cres[r * 16 + (lane & 15)] * isc;
        const f32x4 x = M::qk(af, bf, f32x4{c, c, c, c});
        const f32x4 w = *reinterpret_cast<const f32x4*>(w2 + st * 16 + 4 * g);
        f32x4 bv[1] = {f32x4{0.f, 0.f, 0.f, 0.f}};
        if (GENERAL) {
          const int s0[1] = {st * 16 + 4 * g};
          bias.template quads<TRANS, 1>((rt0 + r) * 16 + (lane & 15), s0, bv);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float xv = __builtin_fmaf(x[e], sc, w[e]);
          if (GENERAL) xv += bv[0][e];
          W[sl][e] = fast_exp2(xv);
        }
      }
    }
  }
}

// out[q] = sum_j W[q][j] z_j for the nr resident tiles: lean_wsum_chunk's order (four
// accumulators per resident tile over the slots in order, (s0 + s1) + (s2 + s3), the
// lane groups, then the waves in order).  Called by the whole block.  The vectors are
// given as float offsets into the kernel's dynamic LDS (so every access is a ds_
// instruction with a 32-bit address) and the counts are made wave-uniform: in the
// register-bound backward kernel, pointers and counts kept in VGPRs were spilled to
// scratch and reloaded before every matvec.
template <int KS>
__device__ __forceinline__ void reg_wsum(const f32x4 (&W)[BWD_REG_SLOTS], int n_str_tiles_in, int nr_in, int zv_off,
                                         int out_off, int scratch_off) {
  extern __shared__ __align__(16) unsigned char smem[];
  const float* zv = reinterpret_cast<const float*>(smem) + __builtin_amdgcn_readfirstlane(zv_off);
  float* out = reinterpret_cast<float*>(smem) + __builtin_amdgcn_readfirstlane(out_off);
  float* scratch = reinterpret_cast<float*>(smem) + __builtin_amdgcn_readfirstlane(scratch_off);
  const int n_str_tiles = __builtin_amdgcn_readfirstlane(n_str_tiles_in);
  const int nr = __builtin_amdgcn_readfirstlane(nr_in);
  constexpr int NRM = bwd_reg_nrm(KS);
  const int lane = threadIdx.x & (WAVE - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE);
  const int g = lane >> 4;
  f32x4 z[KS];
#pragma unroll
  for (int k = 0; k < KS; ++k) {
    const int st = wave + BWD_NW * k;
    z[k] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (st < n_str_tiles) z[k] = *reinterpret_cast<const f32x4*>(zv + st * 16 + 4 * g);
  }
#pragma unroll
  for (int r = 0; r < NRM; ++r) {
    if (r < nr) {
      float s[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int k = 0; k < KS; ++k)
#pragma unroll
        for (int e = 0; e < 4; ++e) s[e] = __builtin_fmaf(W[r * KS + k][e], z[k][e], s[e]);
      const float ss = sum_groups((s[0] + s[1]) + (s[2] + s[3]));
      if (lane < 16) scratch[(wave * nr + r) * 16 + lane] = ss;
    }
  }
  __syncthreads();
  if ((int)threadIdx.x < nr * 16) {
    const int q = threadIdx.x, r = q >> 4, l = q & 15;
    float ss = 0.f;
#pragma unroll
    for (int w_ = 0; w_ < BWD_NW; ++w_) ss += scratch[(w_ * nr + r) * 16 + l];
    out[q] = ss;
  }
  __syncthreads();
}

// Deterministic block-wide sum of f(i) over i in [0, n) (same order in every block).
// red holds two slots of BWD_NW partials used alternately (flip), so one barrier
// suffices: a slot is rewritten only after the barrier of the call in between.
template <typename F>
__device__ __forceinline__ float block_sum(int n, F f, float* red, int& flip) {
  float acc = 0.f;
  for (int i = threadIdx.x; i < n; i += BWD_NT) acc += f(i);
  acc = wave_sum(acc);
  float* slot = red + flip * BWD_NW;
  flip ^= 1;
  if ((threadIdx.x & (WAVE - 1)) == 0) slot[threadIdx.x / WAVE] = acc;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int w = 0; w < BWD_NW; ++w) tot += slot[w];
  return tot;
}

// Gather a published vector into dst: values at valid indices < n, zero elsewhere
// (invalid entries and the tail [n, Np)); one barrier at the end.  Returns false
// (uniformly) if the error flag is raised or a wait expires.
__device__ __forceinline__ bool gather_vector(const uint64_t* buf, int n, int Np, uint32_t tag, float* dst,
                                              const unsigned char* valid, ErrRef err, int* s_flag) {
  const int t = threadIdx.x;
  for (int i = n + t; i < Np; i += BWD_NT) dst[i] = 0.f;
  const bool ok = poll_vector<BWD_NT>(buf, n, tag, err, [&](int off, uint64_t w) {
    const int i = off + t;
    dst[i] = valid[i] ? __uint_as_float((uint32_t)(w >> 32)) : 0.f;
  });
  if (!ok) *s_flag = 1;
  // dst may be global memory (stream storage keeps the vectors in the workspace)
  __syncthreads();
  return *s_flag == 0;
}

// Per-wave gather of the register-storage CG: the wave polls the words of its own
// streamed tiles (wave + BWD_NW k, the tiles its slots of reg_wsum read) and writes
// dst[i] (0 for a masked entry and for the last tile's entries i >= n), with no
// barrier: each tile has one owner wave.  Returns false, uniformly over the wave, if
// a wait expired (then the error has been raised).
__device__ __forceinline__ bool gather_own_tiles(const uint64_t* buf, int n, int n_tiles, uint32_t tag, float* dst,
                                                 const unsigned char* valid, ErrRef err) {
  const int lane = threadIdx.x & (WAVE - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE);
  const int nwords = wave < n_tiles ? ((n_tiles - 1 - wave) / BWD_NW + 1) * 16 : 0;
  bool ok = true;
  for (int base = 0; base < nwords && ok; base += 2 * WAVE) {
    int idx[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int e = base + k * WAVE + lane;
      const int i = (wave + BWD_NW * (e >> 4)) * 16 + (e & 15);
      idx[k] = (e < nwords && i < n) ? i : -1;
      if (e < nwords && i >= n) dst[i] = 0.f;
    }
    ok = poll_words<2>(buf, idx, tag, err, [&](int k, uint64_t w) {
      const int i = idx[k];
      dst[i] = valid[i] ? __uint_as_float((uint32_t)(w >> 32)) : 0.f;
    });
    ok = wave_max_u32(ok ? 0u : 1u) == 0u;
  }
  return ok;
}

// gather_vector followed by block_sum(Np, f) in one barrier: every thread gathers the
// entries i = t + k BWD_NT (the poll's assignment; the tail [n, Np) too), so after
// its polls it already holds what f reads of dst and can sum f over its entries; the
// wave partials then travel through the gather's own barrier.  The sum is the one
// block_sum gives (same entries, order and reduction).  *dot is uniform on return.
template <typename F>
__device__ __forceinline__ bool gather_vector_dot(const uint64_t* buf, int n, int Np, uint32_t tag, float* dst,
                                                  const unsigned char* valid, ErrRef err, int* s_flag, F f,
                                                  float* red, int& flip, float* dot) {
  const int t = threadIdx.x;
  for (int i = t; i < Np; i += BWD_NT)
    if (i >= n) dst[i] = 0.f;
  const bool ok = poll_vector<BWD_NT>(buf, n, tag, err, [&](int off, uint64_t w) {
    const int i = off + t;
    dst[i] = valid[i] ? __uint_as_float((uint32_t)(w >> 32)) : 0.f;
  });
  if (!ok) *s_flag = 1;
  float acc = 0.f;
  for (int i = t; i < Np; i += BWD_NT) acc += f(i);
  acc = wave_sum(acc);
  float* slot = red + flip * BWD_NW;
  flip ^= 1;
  if ((t & (WAVE - 1)) == 0) slot[t / WAVE] = acc;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int w = 0; w < BWD_NW; ++w) tot += slot[w];
  *dot = tot;
  return *s_flag == 0;
}

// Resident-tile assignment of the heavy passes.  With nr <= BWD_NW resident tiles,
// each tile gets wpt = BWD_NW / nr waves that take interleaved 32-row pairs of
// every streamed chunk (all waves busy); the part > 0 waves hand their partial
// sums to part 0 through LDS.  With more tiles, waves own whole tiles (up to
// MAXT each) as before.
struct PassSplit {
  bool split;
  int wpt, part;
  bool active;  // this wave has a tile in split mode
  __device__ __forceinline__ PassSplit(int nr, int wave) {
    split = nr <= BWD_NW;
    wpt = split ? BWD_NW / nr : 1;
    part = split ? wave / nr : 0;
    active = !split || part < wpt;
  }
  // resident tile of slot k in batch rt0 (nr if none)
  __device__ __forceinline__ int tile(int rt0, int k, int nr, int wave) const {
    if (split) return (k == 0 && active) ? wave % nr : nr;
    return rt0 + wave + BWD_NW * k;
  }
};
// Floats per lane of the partial sums handed over in split mode.
template <int DP> constexpr int pass_partial_floats() { return 4 + 4 * (DP / 16); }

__device__ __forceinline__ float sigm(float x) { return 1.f / (1.f + __expf(-x)); }

constexpr int STAGE_BATCH = 4;  // 16-byte loads each thread keeps in flight while staging

// Rows [r0, r0 + CH) of a row-major [.][DP] operand into LDS dst[CH][DP]
// (zero outside rows [0, n) and columns [0, d)).  `src` rows are `sn` elements
// apart; 16-byte vector copies when d == DP and the rows are 16-byte aligned.
template <typename T, int DP>
__device__ __forceinline__ void stage_chunk(T* dst, const T* __restrict__ src, long long sn, int r0, int CH, int n,
                                            int d) {
  constexpr int VE = 16 / sizeof(T);
  typedef __attribute__((__vector_size__(16))) int i32x4;
  if (d == DP && sn % VE == 0 && (reinterpret_cast<uintptr_t>(src) & 15) == 0) {
    constexpr int CPR = DP / VE;
    const int total = CH * CPR;
    // STAGE_BATCH loads in flight per thread before the first store
    for (int c0 = threadIdx.x; c0 < total; c0 += STAGE_BATCH * BWD_NT) {
      i32x4 v[STAGE_BATCH];
#pragma unroll
      for (int u = 0; u < STAGE_BATCH; ++u) {
        const int c = c0 + u * BWD_NT;
        const int row = c / CPR, k = c - row * CPR;
        v[u] = i32x4{0, 0, 0, 0};
        if (c < total && r0 + row < n) v[u] = *reinterpret_cast<const i32x4*>(src + (size_t)(r0 + row) * sn + k * VE);
      }
#pragma unroll
      for (int u = 0; u < STAGE_BATCH; ++u) {
        const int c = c0 + u * BWD_NT;
        const int row = c / CPR, k = c - row * CPR;
        if (c < total) *reinterpret_cast<i32x4*>(dst + (size_t)row * DP + k * VE) = v[u];
      }
    }
    return;
  }
  for (int e = threadIdx.x; e < CH * DP; e += BWD_NT) {
    const int row = e / DP, col = e - row * DP;
    const int i = r0 + row;
    T v = from_f32<T>(0.f);
    if (i < n && col < d) v = src[(size_t)i * sn + col];
    dst[e] = v;
  }
}

// Transposed: dst[DP][CH + VE] with dst[c][row] = src[r0 + row][c].  The 16-byte
// row padding keeps the 16 lanes that read one MFMA operand column run (rows c0..c0+15)
// in different LDS banks; an unpadded 256-row stride put all of them in one bank.
template <typename T, int DP>
__device__ __forceinline__ void stage_chunk_t(T* dst, const T* __restrict__ src, long long sn, int r0, int CH, int n,
                                              int d) {
  constexpr int VE = 16 / sizeof(T);
  if (d == DP && sn % VE == 0 && (reinterpret_cast<uintptr_t>(src) & 15) == 0) {
    typedef __attribute__((__vector_size__(16))) int i32x4;
    constexpr int CPR = DP / VE;
    const int total = CH * CPR;
    for (int c0 = threadIdx.x; c0 < total; c0 += STAGE_BATCH * BWD_NT) {
      i32x4 w[STAGE_BATCH];
#pragma unroll
      for (int u = 0; u < STAGE_BATCH; ++u) {
        const int c = c0 + u * BWD_NT;
        const int row = c % CH, k = c / CH;  // consecutive threads -> consecutive rows
        w[u] = i32x4{0, 0, 0, 0};
        if (c < total && r0 + row < n) w[u] = *reinterpret_cast<const i32x4*>(src + (size_t)(r0 + row) * sn + k * VE);
      }
#pragma unroll
      for (int u = 0; u < STAGE_BATCH; ++u) {
        const int c = c0 + u * BWD_NT;
        const int row = c % CH, k = c / CH;
        if (c < total) {
          T v[VE];
          __builtin_memcpy(v, &w[u], 16);
#pragma unroll
          for (int e = 0; e < VE; ++e) dst[(size_t)(k * VE + e) * (CH + VE) + row] = v[e];
        }
      }
    }
    return;
  }
  for (int e = threadIdx.x; e < CH * DP; e += BWD_NT) {
    const int col = e / CH, row = e - col * CH;
    const int i = r0 + row;
    T v = from_f32<T>(0.f);
    if (i < n && col < d) v = src[(size_t)i * sn + col];
    dst[(size_t)col * (CH + VE) + row] = v;
  }
}

// Columns [r0, r0 + CH) of a prepared transposed operand src[DP][Np] into dst[DP][CH + VE]
// (Np and r0 are multiples of 32 and CH of 32, so rows are 16-byte aligned).
template <typename T, int DP>
__device__ __forceinline__ void stage_chunk_tt(T* dst, const T* __restrict__ src, int Np, int r0, int CH) {
  constexpr int VE = 16 / sizeof(T);
  typedef __attribute__((__vector_size__(16))) int i32x4;
  const int per = CH / VE;
  const int total = DP * per;
  for (int c0 = threadIdx.x; c0 < total; c0 += STAGE_BATCH * BWD_NT) {
    i32x4 v[STAGE_BATCH];
#pragma unroll
    for (int u = 0; u < STAGE_BATCH; ++u) {
      const int c = c0 + u * BWD_NT;
      const int k = c / per, e = c - k * per;
      v[u] = i32x4{0, 0, 0, 0};
      if (c < total && r0 + e * VE < Np) v[u] = *reinterpret_cast<const i32x4*>(src + (size_t)k * Np + r0 + e * VE);
    }
#pragma unroll
    for (int u = 0; u < STAGE_BATCH; ++u) {
      const int c = c0 + u * BWD_NT;
      const int k = c / per, e = c - k * per;
      if (c < total) *reinterpret_cast<i32x4*>(dst + (size_t)k * (CH + VE) + e * VE) = v[u];
    }
  }
}

// Several operands of one chunk staged together, with the loads of every job in
// flight at once (one L2 round trip per chunk instead of one per operand).
//   kind 0: rows [r0, r0 + CH) of src (row stride sn, rows < n, columns < d) -> dst[CH][DP]
//   kind 1: the same rows transposed -> dst[DP][CH + VE]
//   kind 2: columns [r0, r0 + CH) of a prepared transposed src[DP][n] -> dst[DP][CH + VE]
// Jobs without 16-byte aligned full rows fall back to the element-wise stagers.
struct StageJob {
  const void* src;
  void* dst;
  long long sn;
  int n, d, kind;
};

template <typename T, int DP, int NJ>
__device__ __forceinline__ void stage_jobs(const StageJob (&J)[NJ], int r0, int CH) {
  constexpr int VE = 16 / sizeof(T);
  constexpr int CPR = DP / VE;
  constexpr int KPT = 2;  // blocks per thread and job in flight
  typedef __attribute__((__vector_size__(16))) int i32x4;
  bool vec[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const T* src = static_cast<const T*>(J[j].src);
    vec[j] = J[j].kind == 2 ||
             (J[j].d == DP && J[j].sn % VE == 0 && (reinterpret_cast<uintptr_t>(src) & 15) == 0);
    if (!vec[j]) {
      if (J[j].kind == 0) stage_chunk<T, DP>(static_cast<T*>(J[j].dst), src, J[j].sn, r0, CH, J[j].n, J[j].d);
      else stage_chunk_t<T, DP>(static_cast<T*>(J[j].dst), src, J[j].sn, r0, CH, J[j].n, J[j].d);
    }
  }
  const int total = CH * CPR;  // 16-byte blocks per job (kind 2: DP rows of CH / VE)
  for (int c0 = threadIdx.x; c0 < total; c0 += KPT * BWD_NT) {
    i32x4 v[NJ][KPT];
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int u = 0; u < KPT; ++u) {
        const int c = c0 + u * BWD_NT;
        const T* src = static_cast<const T*>(J[j].src);
        v[j][u] = i32x4{0, 0, 0, 0};
        if (!vec[j] || c >= total) continue;
        if (J[j].kind == 2) {
          const int per = CH / VE, k = c / per, e = c - k * per;
          if (r0 + e * VE < J[j].n) v[j][u] = *reinterpret_cast<const i32x4*>(src + (size_t)k * J[j].n + r0 + e * VE);
        } else {
          const int row = J[j].kind == 0 ? c / CPR : c % CH;
          const int k = J[j].kind == 0 ? c - row * CPR : c / CH;
          if (r0 + row < J[j].n) v[j][u] = *reinterpret_cast<const i32x4*>(src + (size_t)(r0 + row) * J[j].sn + k * VE);
        }
      }
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int u = 0; u < KPT; ++u) {
        const int c = c0 + u * BWD_NT;
        if (!vec[j] || c >= total) continue;
        T* dst = static_cast<T*>(J[j].dst);
        if (J[j].kind == 2) {
          const int per = CH / VE, k = c / per, e = c - k * per;
          *reinterpret_cast<i32x4*>(dst + (size_t)k * (CH + VE) + e * VE) = v[j][u];
        } else if (J[j].kind == 0) {
          const int row = c / CPR, k = c - row * CPR;
          *reinterpret_cast<i32x4*>(dst + (size_t)row * DP + k * VE) = v[j][u];
        } else {
          const int row = c % CH, k = c / CH;
          T e8[VE];
          __builtin_memcpy(e8, &v[j][u], 16);
#pragma unroll
          for (int e = 0; e < VE; ++e) dst[(size_t)(k * VE + e) * (CH + VE) + row] = e8[e];
        }
      }
  }
}

// Gradients of q, k, v, g are stored in the input type (one rounding of the fp32 sums).
template <typename T>
__device__ __forceinline__ void put_grad(void* p, size_t i, float v) {
  static_cast<T*>(p)[i] = from_f32<T>(v);
}

struct BwdShared {
  int flag, tmp, local;
  float posw[BIN_NONE + 1];
  float red[2 * BWD_NW];
};

// Streamed rows per LDS chunk in resident mode (stream mode sizes it on the host).
__host__ __device__ inline int bwd_chunk(int N) {
  const int Np = ((N + 31) / 32) * 32;
  return Np < 256 ? Np : 256;
}
__host__ __device__ inline int bwd_local_rows(int N, int G) { return 16 * (((N + 15) / 16 + G - 1) / G); }

// GEN: the cost may carry position bins or geometry (set by the host when either is
// passed); GEN = false compiles no bias code.
template <typename T, int DP, bool STREAM, bool GEN>
__global__ void __launch_bounds__(BWD_NT) sinkhorn_bwd_kernel(SinkBwdArgs a) {
  using M = Mfma<T, DP>;
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ BwdShared sh;
  int grp, member;
  if (!group_of(a.B * a.H, a.G, grp, member)) return;  // surplus workgroup of the XCD-aligned grid
  const int b = grp / a.H, h = grp % a.H;
  const int N = a.N, d = a.d;
  const int Np = ((N + 31) / 32) * 32;
  const int CH = a.ch;
  constexpr int TPAD = 16 / (int)sizeof(T);  // row padding of the transposed chunk buffers
  const int loc = bwd_local_rows(N, a.G);
  const int lane = threadIdx.x & (WAVE - 1);
  const int wave = threadIdx.x / WAVE;
  const int g = lane >> 4;
  if (threadIdx.x == 0) { sh.flag = 0; sh.local = 1; }
  if (blockIdx.x == 0 && threadIdx.x == 0)
    __hip_atomic_store(a.err.ws + 1, a.salt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

  const size_t bh = (size_t)b * a.H + h;
  const size_t wg_id = bh * a.G + member;
  // ---- LDS carve-up (must match sinkhorn_bwd_lds_bytes)
  unsigned char* valid = smem;
  const int res_rows = STREAM ? loc : Np;  // rows of Q and K kept in LDS by the solve
  const size_t region = max(max((size_t)2 * res_rows * DP * sizeof(T), (size_t)(4 * CH + TPAD) * DP * sizeof(T)),
                            (size_t)BWD_NW * WAVE * pass_partial_floats<DP>() * 4);
  T* R0 = reinterpret_cast<T*>(smem + ((Np + 15) / 16) * 16);
  float* after_region = reinterpret_cast<float*>(reinterpret_cast<unsigned char*>(R0) + region);
  float* fv = STREAM ? a.vec_ws + wg_id * (size_t)BWD_STREAM_VECS * Np : after_region;
  float* uu = fv;            // u (log2), rows
  float* vv = uu + Np;       // v (log2), cols
  float* lz = vv + Np;       // log Z (log2), rows
  float* cl = lz + Np;       // col_lse (log2), cols
  float* Dv = cl + Np;       // D_i, rows
  float* gv = Dv + Np;       // g_v, cols
  float* zu = gv + Np;       // z_u, rows
  float* zvv = zu + Np;      // z_v, cols
  float* cy = zvv + Np;      // CG y / scratch vector (cols)
  float* cr = cy + Np;       // CG r (cols)
  float* cp = cr + Np;       // CG p (cols)
  float* ct = cp + Np;       // CG t (rows)
  float* ctw = ct + Np;      // CG W x (rows)
  float* xs = ctw + Np;      // x coordinates [Np][3]
  float* dxc = xs + 3 * Np;  // grad x_centroid rows [Np][3]
  float* lres = STREAM ? after_region : dxc + 3 * Np;  // per-local-row constants [loc] (stream mode)
  float* lout = lres + loc;      // per-local-row results [loc]
  float* dxs = lout + loc;       // dx accumulator for my stripe [loc][3]
  float* dpw = dxs + 3 * loc;    // d pos_weight histogram [68]
  float* scratch = dpw + 68;     // BWD_SCRATCH (resident) or BWD_STREAM_SCRATCH (stream) floats
  // block-uniform counts, made scalar: held in VGPRs they were among the values this
  // register-bound kernel spills to scratch and reloads in its loops
  const int n = __builtin_amdgcn_readfirstlane(mask_setup(a.mask ? a.mask + (size_t)b * N : nullptr, N, valid, &sh.tmp));
  const int n_tiles = (n + 15) / 16;
  int t0, t1;
  stripe(n_tiles, member, a.G, t0, t1);
  t0 = __builtin_amdgcn_readfirstlane(t0);
  t1 = __builtin_amdgcn_readfirstlane(t1);
  const int nr = t1 - t0;
  // Every output position is written: rows past the last valid tile (owned by no
  // stripe) are zeroed here, row i by member i % G; invalid stripe rows get zeros
  // where the stripe's outputs are written.
  for (int i = n_tiles * 16 + member; i < N; i += a.G) {
    for (int c = threadIdx.x; c < d; c += BWD_NT) {
      put_grad<T>(a.dq, (bh * N + i) * d + c, 0.f);
      put_grad<T>(a.dk, (bh * N + i) * d + c, 0.f);
      put_grad<T>(a.dv, (bh * N + i) * d + c, 0.f);
    }
    if (threadIdx.x == 0) {
      a.dlog_mu[bh * N + i] = 0.f;
      a.dlog_nu[bh * N + i] = 0.f;
    }
  }
  if (n == 0 || nr <= 0) {
    // owns nothing: publish empty partials so the finaliser can sum every slot
    for (int k = threadIdx.x; k < 68; k += BWD_NT) a.dpw_part[wg_id * 68 + k] = 0.f;
    if (threadIdx.x == 0) a.dw_part[wg_id] = 0.f;
    return;
  }
  const int r_lo = t0 * 16, r_hi = min(t1 * 16, n);

  const size_t qoff = (size_t)b * a.sb + (size_t)h * a.sh;
  const T* Qg = reinterpret_cast<const T*>(a.q) + qoff;
  const T* Kg = reinterpret_cast<const T*>(a.k) + qoff;
  const T* Vg = reinterpret_cast<const T*>(a.v) + qoff;
  const T* gOh = reinterpret_cast<const T*>(a.go_hi) + bh * Np * DP;  // [Np][DP]
  const T* gOlo = reinterpret_cast<const T*>(a.go_lo) + bh * Np * DP;  // [Np][DP]
  const T* gOt = reinterpret_cast<const T*>(a.go_t) + bh * DP * Np;    // [DP][Np]
  const float eps = a.eps[h];
  const float kappa = a.lam / (a.lam + eps);
  const float sc = LOG2E / (sqrtf((float)d) * eps);
  const float inv_eps = 1.f / eps;
  const float kape = kappa / eps;
  const float sgn_col = a.mode == 1 ? 1.f : -1.f;
  const float inv_sqrt_d = 1.f / sqrtf((float)d);
  const bool has_dxc = a.grad_xc != nullptr;

  // ---- per-(b,h) vectors (log2 units; invalid -> NEG_BIG / 0)
  for (int i = threadIdx.x; i < Np; i += BWD_NT) {
    const bool ok = i < n && valid[i];
    uu[i] = ok ? a.log_u[bh * N + i] * LOG2E : NEG_BIG;
    vv[i] = ok ? a.log_v[bh * N + i] * LOG2E : NEG_BIG;
    lz[i] = ok ? a.log_z[bh * N + i] * LOG2E : 0.f;
    cl[i] = ok ? a.col_lse[bh * N + i] * LOG2E : 0.f;
    for (int c = 0; c < 3; ++c) {
      xs[3 * i + c] = (a.x && i < n) ? a.x[((size_t)b * N + i) * 3 + c] : 0.f;
      dxc[3 * i + c] = (has_dxc && ok) ? a.grad_xc[(bh * N + i) * 3 + c] : 0.f;
    }
  }
  for (int q = threadIdx.x; q < 3 * loc; q += BWD_NT) dxs[q] = 0.f;
  for (int k = threadIdx.x; k < 68; k += BWD_NT) dpw[k] = 0.f;
  const float w_h = a.w_dist ? a.w_dist[h] : 0.f;
  const bool use_geo = GEN && (a.x != nullptr) && (w_h != 0.f);
  const bool use_pos = GEN && (a.bins8 != nullptr) && (a.pos_w != nullptr);
  if (use_pos)
    for (int k = threadIdx.x; k <= (int)BIN_NONE; k += BWD_NT)
      sh.posw[k] = k < (int)BIN_NONE ? -LOG2E * a.pos_w[h * 68 + k] / eps : 0.f;
  __syncthreads();
  Bias bias;
  bias.b8 = use_pos ? a.bins8 + (size_t)b * Np * Np : nullptr;
  bias.b8t = use_pos ? a.bins8t + (size_t)b * Np * Np : nullptr;
  bias.posw = sh.posw;
  bias.xs = use_geo ? xs : nullptr;
  bias.geo_scale = -LOG2E * w_h / eps;
  bias.r0 = a.r0;
  bias.Np = Np;
  const bool general = use_pos || use_geo;
  if (general && a.bias_mat) {
    bias.mat = a.bias_mat + bh * Np * Np;
    bias.matT = a.bias_matT + bh * Np * Np;
  }
  const bool geo_grad = GEN && a.geo_grad != 0 && a.x != nullptr;

  // ---- D_i (prep kernel) for all rows
  const float* Dg = a.dcoef + bh * Np;
  for (int i = threadIdx.x; i < Np; i += BWD_NT) Dv[i] = Dg[i];
  __syncthreads();

  uint64_t* xbase = a.xch + bh * 4 * (size_t)Np;
  const uint32_t salt = a.salt << 12;
  uint32_t phase = 0;
  // placement words of the group (after all (b,h)'s four vector slots); plain-store
  // publishing from the second exchange on if every member is on its XCD
  uint64_t* xpl = a.xch + (size_t)a.B * a.H * 4 * Np + bh * 32;
  publish_placement(xpl, member, a.salt);
  bool local = false;
  constexpr int NC = DP / 16;

  // =========================================================================
  // C1: column pass, resident j (my tiles), streamed i in chunks.
  //   T = exp2(sc qk + (u-logZ)_i + v_j);  gls = T (dT - D_i);  g_v_j = sum_i gls
  //   dV_j = sum_i T gO_i;  dx_tr_j = sum_i T dxc_i
  {
    T* Qc = R0;
    T* gOc = Qc + (size_t)CH * DP;
    T* gOl = gOc + (size_t)CH * DP;  // low halves of gO (bf16 only)
    T* gOT = gOl + (size_t)CH * DP;  // [DP][CH + TPAD]
    float* a2 = ct;                  // (u - logZ) in log2, rows (ct is free until the solve)
    for (int i = threadIdx.x; i < Np; i += BWD_NT) a2[i] = (i < n && valid[i]) ? uu[i] - lz[i] : NEG_BIG;
    __syncthreads();
    const PassSplit ps(nr, wave);
    for (int rt0 = 0; rt0 < nr; rt0 += ps.split ? nr : bwd_maxt<DP>() * BWD_NW) {
      constexpr int MAXT = bwd_maxt<DP>();
      typename M::Frag kf[MAXT], vf[MAXT];
      f32x4 cinit[MAXT], dvacc[MAXT][NC];
      float gva[MAXT], dxa[MAXT][3], xj[MAXT][3];
      int tl[MAXT];
      int ntile = 0;
#pragma unroll
      for (int k = 0; k < MAXT; ++k) {
        const int rt = ps.tile(rt0, k, nr, wave);
        tl[k] = rt;
        gva[k] = 0.f;
        dxa[k][0] = dxa[k][1] = dxa[k][2] = 0.f;
#pragma unroll
        for (int c = 0; c < NC; ++c) dvacc[k][c] = f32x4{0.f, 0.f, 0.f, 0.f};
        if (rt < nr) {
          ++ntile;
          const int j = (t0 + rt) * 16 + (lane & 15);
          load_frag_global<T, DP>(kf[k], Kg, a.sn, j, n, d, lane);
          load_frag_global<T, DP>(vf[k], Vg, a.sn, j, n, d, lane);
          const float ci = vv[j] / sc;
          cinit[k] = f32x4{ci, ci, ci, ci};
          xj[k][0] = xs[3 * j]; xj[k][1] = xs[3 * j + 1]; xj[k][2] = xs[3 * j + 2];
        }
      }
      for (int c0 = 0; c0 < n; c0 += CH) {
        __syncthreads();
        if constexpr (M::SPLIT) {
          const StageJob jobs[4] = {{Qg, Qc, a.sn, n, d, 0}, {gOh, gOc, DP, Np, DP, 0}, {gOlo, gOl, DP, Np, DP, 0},
                                    {gOt, gOT, Np, Np, DP, 2}};
          stage_jobs<T, DP, 4>(jobs, c0, CH);
        } else {
          const StageJob jobs[3] = {{Qg, Qc, a.sn, n, d, 0}, {gOh, gOc, DP, Np, DP, 0}, {gOt, gOT, Np, Np, DP, 2}};
          stage_jobs<T, DP, 3>(jobs, c0, CH);
        }
        __syncthreads();
        const int npair = (min(CH, n - c0) + 31) / 32;
        for (int pr = ps.part; pr < npair; pr += ps.wpt) {
          typename M::Frag qa[2], ga[2], gl[2];
          f32x4 wa[2], Dq[2];
#pragma unroll
          for (int hf = 0; hf < 2; ++hf) {
            const int sl = pr * 32 + hf * 16;  // chunk-local streamed tile base
            M::load(qa[hf], Qc + (size_t)(sl + (lane & 15)) * DP, lane);
            M::load(ga[hf], gOc + (size_t)(sl + (lane & 15)) * DP, lane);
            if (M::SPLIT) M::load(gl[hf], gOl + (size_t)(sl + (lane & 15)) * DP, lane);
            wa[hf] = *reinterpret_cast<const f32x4*>(a2 + c0 + sl + 4 * g);
            Dq[hf] = *reinterpret_cast<const f32x4*>(Dv + c0 + sl + 4 * g);
          }
#pragma unroll
          for (int k = 0; k < MAXT; ++k) {
            if (k < ntile) {
              const int j = (t0 + tl[k]) * 16 + (lane & 15);
              f32x4 tv[2];
#pragma unroll
              for (int hf = 0; hf < 2; ++hf) {
                const f32x4 acc = M::qk(qa[hf], kf[k], cinit[k]);
                const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
                f32x4 dt = M::qk(ga[hf], vf[k], zero);
                if (M::SPLIT) dt = M::qk(gl[hf], vf[k], dt);
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                  const int i = c0 + pr * 32 + hf * 16 + 4 * g + r;
                  float x = __builtin_fmaf(acc[r], sc, wa[hf][r]);
                  if (general && wa[hf][r] > 0.5f * NEG_BIG) x += bias(i, j);
                  const float tval = fast_exp2(x);
                  float dtv = dt[r];
                  if (has_dxc) {
                    const float* dc = dxc + 3 * i;
                    dtv += dc[0] * xj[k][0] + dc[1] * xj[k][1] + dc[2] * xj[k][2];
                    dxa[k][0] = __builtin_fmaf(tval, dc[0], dxa[k][0]);
                    dxa[k][1] = __builtin_fmaf(tval, dc[1], dxa[k][1]);
                    dxa[k][2] = __builtin_fmaf(tval, dc[2], dxa[k][2]);
                  }
                  gva[k] = __builtin_fmaf(tval, dtv - Dq[hf][r], gva[k]);
                  tv[hf][r] = tval;
                }
              }
#pragma unroll
              for (int c = 0; c < NC; ++c)
                dvacc[k][c] = M::pv(tv[0], tv[1], gOT + (size_t)(c * 16 + (lane & 15)) * (CH + TPAD) + pr * 32, lane,
                                    dvacc[k][c]);
            }
          }
        }
      }
      // split mode: part > 0 waves hand their partials to part 0 (staging buffer is free)
      if (ps.split && ps.wpt > 1) {
        constexpr int PF = pass_partial_floats<DP>();
        float* pp = reinterpret_cast<float*>(R0);
        __syncthreads();
        if (ntile > 0 && ps.part > 0) {
          float* dst = pp + ((size_t)wave * WAVE + lane) * PF;
          dst[0] = gva[0]; dst[1] = dxa[0][0]; dst[2] = dxa[0][1]; dst[3] = dxa[0][2];
#pragma unroll
          for (int c = 0; c < NC; ++c) *reinterpret_cast<f32x4*>(dst + 4 + 4 * c) = dvacc[0][c];
        }
        __syncthreads();
        if (ntile > 0 && ps.part == 0) {
          for (int q = 1; q < ps.wpt; ++q) {
            const float* src = pp + ((size_t)(wave + q * nr) * WAVE + lane) * PF;
            gva[0] += src[0]; dxa[0][0] += src[1]; dxa[0][1] += src[2]; dxa[0][2] += src[3];
#pragma unroll
            for (int c = 0; c < NC; ++c) {
              const f32x4 o = *reinterpret_cast<const f32x4*>(src + 4 + 4 * c);
#pragma unroll
              for (int r = 0; r < 4; ++r) dvacc[0][c][r] += o[r];
            }
          }
        }
        if (ps.part > 0) ntile = 0;
      }
      // epilogue for this batch of resident tiles
#pragma unroll
      for (int k = 0; k < MAXT; ++k) {
        if (k < ntile) {
          const int tile = t0 + tl[k];
          const int jl = tile * 16 + (lane & 15);
          const float gsum = sum_groups(gva[k]);
          const float d0 = sum_groups(dxa[k][0]), d1 = sum_groups(dxa[k][1]), d2 = sum_groups(dxa[k][2]);
          if (lane < 16 && jl < n) {
            lout[jl - r_lo] = gsum;
            dxs[3 * (jl - r_lo) + 0] += d0;
            dxs[3 * (jl - r_lo) + 1] += d1;
            dxs[3 * (jl - r_lo) + 2] += d2;
          }
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int j = tile * 16 + 4 * g + r;
            if (j < N) {
              const bool jv = j < n && valid[j];
#pragma unroll
              for (int c = 0; c < NC; ++c) {
                const int col = c * 16 + (lane & 15);
                if (col < d) put_grad<T>(a.dv, (bh * N + j) * d + col, jv ? dvacc[k][c][r] : 0.f);
              }
            }
          }
        }
      }
    }
    __syncthreads();
    ++phase;
    uint64_t* xg = xbase;  // slot 0: g_v
    for (int j = r_lo + (int)threadIdx.x; j < r_hi; j += BWD_NT) xch_put(xg + j, lout[j - r_lo], salt | phase);
    if (!gather_vector(xg, n, Np, salt | phase, gv, valid, a.err, &sh.flag)) return;
    if (!read_placement(xpl, a.G, n_tiles, a.salt, a.err, &sh.flag, &sh.local)) return;
    local = sh.local != 0;
  }

  // =========================================================================
  // S: solve (I - kappa^2 S_row^T S_col) z_v = g_v.
  // resident: all rows of Q and K (global tile index); stream: my stripes (local tile index)
  T* QS = R0;
  T* KS = R0 + (size_t)res_rows * DP;
  const T* Qp = STREAM ? reinterpret_cast<const T*>(a.qp) + bh * Np * DP : nullptr;
  const T* Kp = STREAM ? reinterpret_cast<const T*>(a.kp) + bh * Np * DP : nullptr;
  __syncthreads();
  if constexpr (STREAM) {
    stage_rows<T, DP>(QS, Qp + (size_t)r_lo * DP, DP, nr * 16, DP, loc);
    stage_rows<T, DP>(KS, Kp + (size_t)r_lo * DP, DP, nr * 16, DP, loc);
  } else {
    stage_rows<T, DP>(QS, Qg, a.sn, n, d, Np);
    stage_rows<T, DP>(KS, Kg, a.sn, n, d, Np);
  }
  __syncthreads();
  // lout[q] = sum_j exp2(sc <res_q, str_j> + cres[q] + w2_j (+bias)) z_j over all
  // streamed j; row = true: resident plan rows (Q) against streamed K.
  // cres: per-resident-row constants, local index (X + r_lo for an Np-vector X).
  // Resident mode reads them in place (LDS); stream mode keeps its vectors in the
  // workspace, so they are first copied to LDS (lres).
  auto wsum = [&](bool row, const float* w2, const float* z, const float* cres_in) {
    const float* cres = cres_in;
    if constexpr (STREAM) {
      for (int q = threadIdx.x; q < nr * 16; q += BWD_NT) lres[q] = cres_in[q];
      __syncthreads();
      cres = lres;
      if (row) {
        if (general) stream_sweep<BWD_NT, T, DP, SW_WSUM, true, false>(QS, Kp, w2, z, n_tiles, t0, nr, sc, cres, bias, lout, nullptr, scratch, nullptr, NoPublish());
        else stream_sweep<BWD_NT, T, DP, SW_WSUM, false, false>(QS, Kp, w2, z, n_tiles, t0, nr, sc, cres, bias, lout, nullptr, scratch, nullptr, NoPublish());
      } else {
        if (general) stream_sweep<BWD_NT, T, DP, SW_WSUM, true, true>(KS, Qp, w2, z, n_tiles, t0, nr, sc, cres, bias, lout, nullptr, scratch, nullptr, NoPublish());
        else stream_sweep<BWD_NT, T, DP, SW_WSUM, false, true>(KS, Qp, w2, z, n_tiles, t0, nr, sc, cres, bias, lout, nullptr, scratch, nullptr, NoPublish());
      }
    } else {
      if (row) {
        if (general) lean_wsum<T, DP, true, false>(QS, KS, w2, z, n_tiles, t0, nr, sc, cres, bias, lout, scratch);
        else lean_wsum<T, DP, false, false>(QS, KS, w2, z, n_tiles, t0, nr, sc, cres, bias, lout, scratch);
      } else {
        if (general) lean_wsum<T, DP, true, true>(KS, QS, w2, z, n_tiles, t0, nr, sc, cres, bias, lout, scratch);
        else lean_wsum<T, DP, false, true>(KS, QS, w2, z, n_tiles, t0, nr, sc, cres, bias, lout, scratch);
      }
    }
  };
  uint64_t* xA = xbase + Np;      // slot 1
  uint64_t* xB = xbase + 2 * Np;  // slot 2
  if (a.solver == 0) {
    // reference Gauss-Seidel (flash_sinkhorn_attn.py:471-542): z_u = 0, z_v = g_v
    for (int i = threadIdx.x; i < Np; i += BWD_NT) { zu[i] = 0.f; zvv[i] = gv[i]; }
    float* mcl = cy;  // -col_lse (log2) on valid columns
    float* a2 = cr;   // u - logZ (log2) on valid rows
    for (int i = threadIdx.x; i < Np; i += BWD_NT) {
      const bool ok = i < n && valid[i];
      mcl[i] = ok ? -cl[i] : NEG_BIG;
      a2[i] = ok ? uu[i] - lz[i] : NEG_BIG;
    }
    __syncthreads();
    for (int it = 0; it < a.iters; ++it) {
      // z_u_i = kappa sum_j S_col_ij z_v_j   (resident rows: cres = u_i)
      wsum(true, mcl, zvv, uu + r_lo);
      ++phase;
      for (int i = r_lo + (int)threadIdx.x; i < r_hi; i += BWD_NT) xch_put(xA + i, kappa * lout[i - r_lo], salt | phase, local);
      if (!gather_vector(xA, n, Np, salt | phase, zu, valid, a.err, &sh.flag)) return;
      // z_v_j = g_v_j + kappa sum_i T_ij z_u_i   (resident cols: cres = v_j)
      wsum(false, a2, zu, vv + r_lo);
      ++phase;
      for (int j = r_lo + (int)threadIdx.x; j < r_hi; j += BWD_NT)
        xch_put(xB + j, gv[j] + kappa * lout[j - r_lo], salt | phase, local);
      if (!gather_vector(xB, n, Np, salt | phase, zvv, valid, a.err, &sh.flag)) return;
    }
  } else {
    // CG on (I - kappa^2 W^T W) y = D_c^{-1/2} g_v, W_ij = exp2(sc qk + alpha_i + beta_j)
    float* al = zu;   // alpha_i = u - logZ/2 (rows); zu is rebuilt after the solve
    float* be = zvv;  // beta_j = (v - col_lse)/2 (cols)
    float* cs = gv;   // s = W^T t; g_v is not read again once r and p are set
    for (int i = threadIdx.x; i < Np; i += BWD_NT) {
      const bool ok = i < n && valid[i];
      al[i] = ok ? uu[i] - 0.5f * lz[i] : NEG_BIG;
      be[i] = ok ? 0.5f * (vv[i] - cl[i]) : NEG_BIG;
      const float bj = ok ? gv[i] * fast_exp2(-0.5f * (vv[i] + cl[i])) : 0.f;
      cy[i] = 0.f;
      cr[i] = bj;
      cp[i] = bj;
      ctw[i] = 0.f;
      ct[i] = 0.f;  // entries past the last tile are never gathered
    }
    __syncthreads();
    int flip = 0;
    float rr = block_sum(Np, [&](int i) { return cr[i] * cr[i]; }, sh.red, flip);
    // cg_rtol > 0: stop once ||r|| <= rtol ||b|| (utils/cg.py:63-80).  cg_rtol == 0:
    // exactly `iters` iterations; a residual that reaches zero stays zero (alpha = beta = 0).
    // rr, pAp and rr_new are bit-identical in every member, so the exit is uniform.
    const bool early_exit = a.cg_rtol > 0.f;
    const float stop2 = a.cg_rtol * a.cg_rtol * rr;
    const float k2 = kappa * kappa;
    // mv(true): lout = W p (my rows); mv(false): lout = W^T t (my columns).  own_t: mv(false)
    // reads t only on the wave's own streamed tiles (register storage), so each wave
    // gathers just those; a failed wait sets the flag that the next gather's barrier
    // turns into a uniform exit.
    auto cg_run = [&](auto&& mv, bool own_t) __attribute__((always_inline)) -> bool {
    for (int it = 0; it < a.iters; ++it) {
      if (early_exit && (rr <= stop2 || rr == 0.f)) break;
      // t_i = sum_j W_ij p_j (my rows)
      mv(true);
      ++phase;
      for (int i = r_lo + (int)threadIdx.x; i < r_hi; i += BWD_NT) xch_put(xA + i, lout[i - r_lo], salt | phase, local);
      if (own_t) {
        if (!gather_own_tiles(xA, n, n_tiles, salt | phase, ct, valid, a.err)) sh.flag = 1;
      } else if (!gather_vector(xA, n, Np, salt | phase, ct, valid, a.err, &sh.flag)) {
        return false;
      }
      // s_j = sum_i W_ij t_i (my cols)
      mv(false);
      ++phase;
      for (int j = r_lo + (int)threadIdx.x; j < r_hi; j += BWD_NT) xch_put(xB + j, lout[j - r_lo], salt | phase, local);
      // CG update, identical in every member (utils/cg.py:70-92 with x0 = 0); p^T A p
      // rides on the gather's barrier
      float pAp;
      if (!gather_vector_dot(xB, n, Np, salt | phase, cs, valid, a.err, &sh.flag,
                             [&](int i) { return cp[i] * (cp[i] - k2 * cs[i]); }, sh.red, flip, &pAp))
        return false;
      if (early_exit && pAp == 0.f) break;
      const float alpha = (pAp != 0.f && rr != 0.f) ? rr / pAp : 0.f;
      // the update and ||r_new||^2 in one pass: each thread squares the entries it wrote
      const float rr_new = block_sum(Np, [&](int i) {
        cy[i] += alpha * cp[i];
        const float ri = cr[i] - alpha * (cp[i] - k2 * cs[i]);
        cr[i] = ri;
        ctw[i] += alpha * ct[i];
        return ri * ri;
      }, sh.red, flip);
      const float beta = rr != 0.f ? rr_new / rr : 0.f;
      rr = rr_new;
      if constexpr (STREAM) {
        for (int i = threadIdx.x; i < Np; i += BWD_NT) cp[i] = cr[i] + beta * cp[i];
        __syncthreads();
      } else {
        // each wave updates the entries of p that its own slots of the next row sweep
        // read (streamed tiles wave + BWD_NW k, lean_wsum's assignment), so no barrier;
        // the rest of p ([n_tiles * 16, Np), and r = p = 0 there) stays zero
        const int wv = threadIdx.x / WAVE, ln = threadIdx.x & (WAVE - 1);
        for (int e = ln; e < ((n_tiles - wv + BWD_NW - 1) / BWD_NW) * 16; e += WAVE) {
          const int i = (wv + BWD_NW * (e >> 4)) * 16 + (e & 15);
          cp[i] = cr[i] + beta * cp[i];
        }
      }
    }
    return true;
    };
    bool cg_ok = false, reg_done = false;
    if constexpr (!STREAM) {
      const int ksg = bwd_reg_ks(n_tiles);
      if (ksg > 0 && nr <= bwd_reg_nrm(ksg)) {
        // register storage of W for the whole solve
        auto reg_cg = [&](auto ksc) __attribute__((always_inline)) -> bool {
          constexpr int KSL = decltype(ksc)::value;
          f32x4 WR[BWD_REG_SLOTS], WC[BWD_REG_SLOTS];
          if (general) {
            reg_wtiles<T, DP, KSL, true, false>(WR, QS, KS, be, n_tiles, t0, nr, sc, al + r_lo, bias);
            reg_wtiles<T, DP, KSL, true, true>(WC, KS, QS, al, n_tiles, t0, nr, sc, be + r_lo, bias);
          } else {
            reg_wtiles<T, DP, KSL, false, false>(WR, QS, KS, be, n_tiles, t0, nr, sc, al + r_lo, bias);
            reg_wtiles<T, DP, KSL, false, true>(WC, KS, QS, al, n_tiles, t0, nr, sc, be + r_lo, bias);
          }
          // float offsets of the vectors in the dynamic LDS (reg_wsum)
          const float* lds0 = reinterpret_cast<const float*>(smem);
          const int o_cp = (int)(cp - lds0), o_ct = (int)(ct - lds0), o_out = (int)(lout - lds0),
                    o_scr = (int)(scratch - lds0);
          return cg_run([&](bool row) __attribute__((always_inline)) {
            if (row) reg_wsum<KSL>(WR, n_tiles, nr, o_cp, o_out, o_scr);
            else reg_wsum<KSL>(WC, n_tiles, nr, o_ct, o_out, o_scr);
          }, true);
        };
        if (ksg == 2) cg_ok = reg_cg(std::integral_constant<int, 2>{});
        else if (ksg == 4) cg_ok = reg_cg(std::integral_constant<int, 4>{});
        else cg_ok = reg_cg(std::integral_constant<int, 6>{});
        reg_done = true;
      }
    }
    if (!reg_done)
      cg_ok = cg_run([&](bool row) __attribute__((always_inline)) {
        if (row) wsum(true, be, cp, al + r_lo);
        else wsum(false, al, ct, be + r_lo);
      }, false);
    if (!cg_ok) return;
    // z_v = D_c^{1/2} y, z_u = kappa D_r^{1/2} (W y)
    for (int i = threadIdx.x; i < Np; i += BWD_NT) {
      const bool ok = i < n && valid[i];
      zvv[i] = ok ? cy[i] * fast_exp2(0.5f * (vv[i] + cl[i])) : 0.f;
      zu[i] = ok ? kappa * ctw[i] * fast_exp2(0.5f * lz[i]) : 0.f;
    }
    __syncthreads();
  }
  // marginal gradients (flash_sinkhorn_attn.py:645-646; analytic: d log_mu = kappa lambda_u = -kappa z_u)
  for (int i = r_lo + (int)threadIdx.x; i < min(t1 * 16, N); i += BWD_NT) {
    const bool iv = i < n && valid[i];
    a.dlog_mu[bh * N + i] = iv ? (a.mode == 1 ? -kappa : kappa) * zu[i] : 0.f;
    a.dlog_nu[bh * N + i] = iv ? kappa * zvv[i] : 0.f;
  }

  // per-row helper vectors for R2 / C2
  float* a2 = cy;   // u - logZ (log2), rows
  float* lc = cr;   // v + col_lse (log2) = log c_j, cols
  for (int i = threadIdx.x; i < Np; i += BWD_NT) {
    const bool ok = i < n && valid[i];
    a2[i] = ok ? uu[i] - lz[i] : NEG_BIG;
    lc[i] = ok ? vv[i] + cl[i] : 0.f;
  }
  __syncthreads();

  float dw_acc = 0.f;  // thread-local part of d w_dist (R2 lanes)

  // =========================================================================
  // R2: row pass, resident i, streamed j in chunks: dQ, dx_i (cost), dw, dpw
  {
    T* Kc = R0;
    T* Vc = Kc + (size_t)CH * DP;
    T* KT = Vc + (size_t)CH * DP;  // [DP][CH + TPAD]
    const PassSplit ps(nr, wave);
    for (int rt0 = 0; rt0 < nr; rt0 += ps.split ? nr : bwd_maxt<DP>() * BWD_NW) {
      constexpr int MAXT = bwd_maxt<DP>();
      typename M::Frag qf[MAXT], gf[MAXT], gfl[MAXT];
      f32x4 cinit[MAXT], dqacc[MAXT][NC];
      float lzi[MAXT], zui[MAXT], Di[MAXT], xi[MAXT][3], dci[MAXT][3], dxa[MAXT][3];
      int tl[MAXT];
      int ntile = 0;
#pragma unroll
      for (int k = 0; k < MAXT; ++k) {
        const int rt = ps.tile(rt0, k, nr, wave);
        tl[k] = rt;
        dxa[k][0] = dxa[k][1] = dxa[k][2] = 0.f;
#pragma unroll
        for (int c = 0; c < NC; ++c) dqacc[k][c] = f32x4{0.f, 0.f, 0.f, 0.f};
        if (rt < nr) {
          ++ntile;
          const int i = (t0 + rt) * 16 + (lane & 15);
          load_frag_global<T, DP>(qf[k], Qg, a.sn, i, n, d, lane);
          load_frag_global<T, DP>(gf[k], gOh, DP, i, Np, DP, lane);
          if (M::SPLIT) load_frag_global<T, DP>(gfl[k], gOlo, DP, i, Np, DP, lane);
          const float ci = a2[i] / sc;
          cinit[k] = f32x4{ci, ci, ci, ci};
          lzi[k] = lz[i];
          zui[k] = zu[i];
          Di[k] = Dv[i];
          xi[k][0] = xs[3 * i]; xi[k][1] = xs[3 * i + 1]; xi[k][2] = xs[3 * i + 2];
          dci[k][0] = dxc[3 * i]; dci[k][1] = dxc[3 * i + 1]; dci[k][2] = dxc[3 * i + 2];
        }
      }
      for (int c0 = 0; c0 < n; c0 += CH) {
        __syncthreads();
        {
          const StageJob jobs[3] = {{Kg, Kc, a.sn, n, d, 0}, {Vg, Vc, a.sn, n, d, 0}, {Kg, KT, a.sn, n, d, 1}};
          stage_jobs<T, DP, 3>(jobs, c0, CH);
        }
        __syncthreads();
        const int npair = (min(CH, n - c0) + 31) / 32;
        for (int pr = ps.part; pr < npair; pr += ps.wpt) {
          typename M::Frag ka[2], va[2];
          f32x4 wv[2], wl[2], wz[2];
#pragma unroll
          for (int hf = 0; hf < 2; ++hf) {
            const int sl = pr * 32 + hf * 16;
            M::load(ka[hf], Kc + (size_t)(sl + (lane & 15)) * DP, lane);
            M::load(va[hf], Vc + (size_t)(sl + (lane & 15)) * DP, lane);
            wv[hf] = *reinterpret_cast<const f32x4*>(vv + c0 + sl + 4 * g);
            wl[hf] = *reinterpret_cast<const f32x4*>(lc + c0 + sl + 4 * g);
            wz[hf] = *reinterpret_cast<const f32x4*>(zvv + c0 + sl + 4 * g);
          }
#pragma unroll
          for (int k = 0; k < MAXT; ++k) {
            if (k < ntile) {
              const int i = (t0 + tl[k]) * 16 + (lane & 15);
              f32x4 dcv[2];
#pragma unroll
              for (int hf = 0; hf < 2; ++hf) {
                const f32x4 acc = M::qk(ka[hf], qf[k], cinit[k]);
                const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
                f32x4 dt = M::qk(va[hf], gf[k], zero);
                if (M::SPLIT) dt = M::qk(va[hf], gfl[k], dt);
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                  const int j = c0 + pr * 32 + hf * 16 + 4 * g + r;
                  const bool jok = wv[hf][r] > 0.5f * NEG_BIG;
                  float x = __builtin_fmaf(acc[r], sc, wv[hf][r]);
                  if (general && jok) x += bias(i, j);
                  const float tval = fast_exp2(x);
                  const float scol = jok ? fast_exp2(x + lzi[k] - wl[hf][r]) : 0.f;
                  float dtv = dt[r];
                  if (has_dxc) dtv += dci[k][0] * xs[3 * j] + dci[k][1] * xs[3 * j + 1] + dci[k][2] * xs[3 * j + 2];
                  const float gls = tval * (dtv - Di[k]);
                  float dC = -inv_eps * gls - kape * zui[k] * tval + sgn_col * kape * wz[hf][r] * scol;
                  if (!jok) dC = 0.f;
                  dcv[hf][r] = dC;
                  if ((geo_grad || use_pos) && jok && i < n && valid[i]) {
                    if (geo_grad) {
                      // backward tiles clamp the distance at 1e-8 (flash_sinkhorn_attn.py:45, 624-634);
                      // d w_dist is non-zero even where w_dist == 0
                      const float dx0 = xi[k][0] - xs[3 * j], dx1 = xi[k][1] - xs[3 * j + 1], dx2 = xi[k][2] - xs[3 * j + 2];
                      const float dist = fmaxf(sqrtf(dx0 * dx0 + dx1 * dx1 + dx2 * dx2), 1e-8f);
                      const float rd = a.r0 + dist;
                      const float om = dC * w_h * a.r0 / (rd * rd * dist);
                      dxa[k][0] = __builtin_fmaf(om, dx0, dxa[k][0]);
                      dxa[k][1] = __builtin_fmaf(om, dx1, dxa[k][1]);
                      dxa[k][2] = __builtin_fmaf(om, dx2, dxa[k][2]);
                      dw_acc = __builtin_fmaf(dC, dist / rd, dw_acc);
                    }
                    if (use_pos) {
                      const unsigned bk = bias.b8[(size_t)i * Np + j];
                      if (bk < 68u) atomicAdd(&dpw[bk], dC);
                    }
                  }
                }
              }
#pragma unroll
              for (int c = 0; c < NC; ++c)
                dqacc[k][c] = M::pv(dcv[0], dcv[1], KT + (size_t)(c * 16 + (lane & 15)) * (CH + TPAD) + pr * 32, lane,
                                    dqacc[k][c]);
            }
          }
        }
      }
      if (ps.split && ps.wpt > 1) {
        constexpr int PF = pass_partial_floats<DP>();
        float* pp = reinterpret_cast<float*>(R0);
        __syncthreads();
        if (ntile > 0 && ps.part > 0) {
          float* dst = pp + ((size_t)wave * WAVE + lane) * PF;
          dst[1] = dxa[0][0]; dst[2] = dxa[0][1]; dst[3] = dxa[0][2];
#pragma unroll
          for (int c = 0; c < NC; ++c) *reinterpret_cast<f32x4*>(dst + 4 + 4 * c) = dqacc[0][c];
        }
        __syncthreads();
        if (ntile > 0 && ps.part == 0) {
          for (int q = 1; q < ps.wpt; ++q) {
            const float* src = pp + ((size_t)(wave + q * nr) * WAVE + lane) * PF;
            dxa[0][0] += src[1]; dxa[0][1] += src[2]; dxa[0][2] += src[3];
#pragma unroll
            for (int c = 0; c < NC; ++c) {
              const f32x4 o = *reinterpret_cast<const f32x4*>(src + 4 + 4 * c);
#pragma unroll
              for (int r = 0; r < 4; ++r) dqacc[0][c][r] += o[r];
            }
          }
        }
        if (ps.part > 0) ntile = 0;
      }
#pragma unroll
      for (int k = 0; k < MAXT; ++k) {
        if (k < ntile) {
          const int tile = t0 + tl[k];
          const int il = tile * 16 + (lane & 15);
          const float d0 = sum_groups(dxa[k][0]), d1 = sum_groups(dxa[k][1]), d2 = sum_groups(dxa[k][2]);
          if (lane < 16 && il < n) {
            dxs[3 * (il - r_lo) + 0] += d0;
            dxs[3 * (il - r_lo) + 1] += d1;
            dxs[3 * (il - r_lo) + 2] += d2;
          }
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int i = tile * 16 + 4 * g + r;
            if (i < N) {
              const bool iv = i < n && valid[i];
#pragma unroll
              for (int c = 0; c < NC; ++c) {
                const int col = c * 16 + (lane & 15);
                if (col < d) put_grad<T>(a.dq, (bh * N + i) * d + col, iv ? -inv_sqrt_d * dqacc[k][c][r] : 0.f);
              }
            }
          }
        }
      }
    }
  }

  // =========================================================================
  // C2: column pass, resident j, streamed i in chunks: dK, dx_j (cost)
  {
    T* Qc = R0;
    T* gOc = Qc + (size_t)CH * DP;
    T* gOl = gOc + (size_t)CH * DP;  // low halves of gO (bf16 only)
    T* QT = gOl + (size_t)CH * DP;   // [DP][CH + TPAD]
    float* a2s = a2;
    float* zus = zu;
    const PassSplit ps(nr, wave);
    for (int rt0 = 0; rt0 < nr; rt0 += ps.split ? nr : bwd_maxt<DP>() * BWD_NW) {
      constexpr int MAXT = bwd_maxt<DP>();
      typename M::Frag kf[MAXT], vf[MAXT];
      f32x4 cinit[MAXT], dkacc[MAXT][NC];
      float lcj[MAXT], zvj[MAXT], xj[MAXT][3], dxa[MAXT][3];
      int tl[MAXT];
      int ntile = 0;
#pragma unroll
      for (int k = 0; k < MAXT; ++k) {
        const int rt = ps.tile(rt0, k, nr, wave);
        tl[k] = rt;
        dxa[k][0] = dxa[k][1] = dxa[k][2] = 0.f;
#pragma unroll
        for (int c = 0; c < NC; ++c) dkacc[k][c] = f32x4{0.f, 0.f, 0.f, 0.f};
        if (rt < nr) {
          ++ntile;
          const int j = (t0 + rt) * 16 + (lane & 15);
          load_frag_global<T, DP>(kf[k], Kg, a.sn, j, n, d, lane);
          load_frag_global<T, DP>(vf[k], Vg, a.sn, j, n, d, lane);
          const float ci = vv[j] / sc;
          cinit[k] = f32x4{ci, ci, ci, ci};
          lcj[k] = lc[j];
          zvj[k] = zvv[j];
          xj[k][0] = xs[3 * j]; xj[k][1] = xs[3 * j + 1]; xj[k][2] = xs[3 * j + 2];
        }
      }
      for (int c0 = 0; c0 < n; c0 += CH) {
        __syncthreads();
        if constexpr (M::SPLIT) {
          const StageJob jobs[4] = {{Qg, Qc, a.sn, n, d, 0}, {gOh, gOc, DP, Np, DP, 0}, {gOlo, gOl, DP, Np, DP, 0},
                                    {Qg, QT, a.sn, n, d, 1}};
          stage_jobs<T, DP, 4>(jobs, c0, CH);
        } else {
          const StageJob jobs[3] = {{Qg, Qc, a.sn, n, d, 0}, {gOh, gOc, DP, Np, DP, 0}, {Qg, QT, a.sn, n, d, 1}};
          stage_jobs<T, DP, 3>(jobs, c0, CH);
        }
        __syncthreads();
        const int npair = (min(CH, n - c0) + 31) / 32;
        for (int pr = ps.part; pr < npair; pr += ps.wpt) {
          typename M::Frag qa[2], ga[2], gl[2];
          f32x4 wa[2], wlz[2], wzu[2], wD[2];
#pragma unroll
          for (int hf = 0; hf < 2; ++hf) {
            const int sl = pr * 32 + hf * 16;
            M::load(qa[hf], Qc + (size_t)(sl + (lane & 15)) * DP, lane);
            M::load(ga[hf], gOc + (size_t)(sl + (lane & 15)) * DP, lane);
            if (M::SPLIT) M::load(gl[hf], gOl + (size_t)(sl + (lane & 15)) * DP, lane);
            wa[hf] = *reinterpret_cast<const f32x4*>(a2s + c0 + sl + 4 * g);
            wlz[hf] = *reinterpret_cast<const f32x4*>(lz + c0 + sl + 4 * g);
            wzu[hf] = *reinterpret_cast<const f32x4*>(zus + c0 + sl + 4 * g);
            wD[hf] = *reinterpret_cast<const f32x4*>(Dv + c0 + sl + 4 * g);
          }
#pragma unroll
          for (int k = 0; k < MAXT; ++k) {
            if (k < ntile) {
              const int j = (t0 + tl[k]) * 16 + (lane & 15);
              const bool jok = j < n && valid[j];
              f32x4 dcv[2];
#pragma unroll
              for (int hf = 0; hf < 2; ++hf) {
                const f32x4 acc = M::qk(qa[hf], kf[k], cinit[k]);
                const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
                f32x4 dt = M::qk(ga[hf], vf[k], zero);
                if (M::SPLIT) dt = M::qk(gl[hf], vf[k], dt);
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                  const int i = c0 + pr * 32 + hf * 16 + 4 * g + r;
                  const bool iok = wa[hf][r] > 0.5f * NEG_BIG;
                  float x = __builtin_fmaf(acc[r], sc, wa[hf][r]);
                  if (general && iok) x += bias(i, j);
                  const float tval = fast_exp2(x);
                  const float scol = (iok && jok) ? fast_exp2(x + wlz[hf][r] - lcj[k]) : 0.f;
                  float dtv = dt[r];
                  if (has_dxc) dtv += dxc[3 * i] * xj[k][0] + dxc[3 * i + 1] * xj[k][1] + dxc[3 * i + 2] * xj[k][2];
                  const float gls = tval * (dtv - wD[hf][r]);
                  float dC = -inv_eps * gls - kape * wzu[hf][r] * tval + sgn_col * kape * zvj[k] * scol;
                  if (!iok || !jok) dC = 0.f;
                  dcv[hf][r] = dC;
                  if (geo_grad && use_geo && iok && jok) {
                    const float dx0 = xs[3 * i] - xj[k][0], dx1 = xs[3 * i + 1] - xj[k][1], dx2 = xs[3 * i + 2] - xj[k][2];
                    const float dist = fmaxf(sqrtf(dx0 * dx0 + dx1 * dx1 + dx2 * dx2), 1e-8f);
                    const float rd = a.r0 + dist;
                    const float om = dC * w_h * a.r0 / (rd * rd * dist);
                    dxa[k][0] = __builtin_fmaf(-om, dx0, dxa[k][0]);
                    dxa[k][1] = __builtin_fmaf(-om, dx1, dxa[k][1]);
                    dxa[k][2] = __builtin_fmaf(-om, dx2, dxa[k][2]);
                  }
                }
              }
#pragma unroll
              for (int c = 0; c < NC; ++c)
                dkacc[k][c] = M::pv(dcv[0], dcv[1], QT + (size_t)(c * 16 + (lane & 15)) * (CH + TPAD) + pr * 32, lane,
                                    dkacc[k][c]);
            }
          }
        }
      }
      if (ps.split && ps.wpt > 1) {
        constexpr int PF = pass_partial_floats<DP>();
        float* pp = reinterpret_cast<float*>(R0);
        __syncthreads();
        if (ntile > 0 && ps.part > 0) {
          float* dst = pp + ((size_t)wave * WAVE + lane) * PF;
          dst[1] = dxa[0][0]; dst[2] = dxa[0][1]; dst[3] = dxa[0][2];
#pragma unroll
          for (int c = 0; c < NC; ++c) *reinterpret_cast<f32x4*>(dst + 4 + 4 * c) = dkacc[0][c];
        }
        __syncthreads();
        if (ntile > 0 && ps.part == 0) {
          for (int q = 1; q < ps.wpt; ++q) {
            const float* src = pp + ((size_t)(wave + q * nr) * WAVE + lane) * PF;
            dxa[0][0] += src[1]; dxa[0][1] += src[2]; dxa[0][2] += src[3];
#pragma unroll
            for (int c = 0; c < NC; ++c) {
              const f32x4 o = *reinterpret_cast<const f32x4*>(src + 4 + 4 * c);
#pragma unroll
              for (int r = 0; r < 4; ++r) dkacc[0][c][r] += o[r];
            }
          }
        }
        if (ps.part > 0) ntile = 0;
      }
#pragma unroll
      for (int k = 0; k < MAXT; ++k) {
        if (k < ntile) {
          const int tile = t0 + tl[k];
          const int jl = tile * 16 + (lane & 15);
          const float d0 = sum_groups(dxa[k][0]), d1 = sum_groups(dxa[k][1]), d2 = sum_groups(dxa[k][2]);
          if (lane < 16 && jl < n) {
            dxs[3 * (jl - r_lo) + 0] += d0;
            dxs[3 * (jl - r_lo) + 1] += d1;
            dxs[3 * (jl - r_lo) + 2] += d2;
          }
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int j = tile * 16 + 4 * g + r;
            if (j < N) {
              const bool jv = j < n && valid[j];
#pragma unroll
              for (int c = 0; c < NC; ++c) {
                const int col = c * 16 + (lane & 15);
                if (col < d) put_grad<T>(a.dk, (bh * N + j) * d + col, jv ? -inv_sqrt_d * dkacc[k][c][r] : 0.f);
              }
            }
          }
        }
      }
    }
  }
  __syncthreads();

  // ---- partials: dx for my stripe, dpw / dw of this workgroup
  for (int q = threadIdx.x; q < 3 * (r_hi - r_lo); q += BWD_NT)
    a.dx_part[(bh * N + r_lo) * 3 + q] = dxs[q];
  // d w_dist: per-thread partials summed in a fixed order
  {
    float acc = dw_acc;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) acc += __shfl_xor(acc, o, WAVE);
    if (lane == 0) sh.red[wave] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
      float tot = 0.f;
      for (int w = 0; w < BWD_NW; ++w) tot += sh.red[w];
      a.dw_part[wg_id] = tot;
    }
  }
  for (int k = threadIdx.x; k < 68; k += BWD_NT) a.dpw_part[wg_id * 68 + k] = dpw[k];
}

// ---------------------------------------------------------------------------
// LDS bytes of the main kernel for a chunk of CH streamed rows.
inline size_t sinkhorn_bwd_lds_bytes_t(int N, int DP, int elem, int G, int CH, bool stream) {
  const size_t Np = ((N + 31) / 32) * 32;
  const size_t loc = bwd_local_rows(N, G);
  const size_t res_rows = stream ? loc : Np;
  size_t bytes = ((Np + 15) / 16) * 16;                                   // valid
  // operand region: Q and K for the solve, or four chunk buffers (the transposed one
  // padded by 16 bytes a row), or the split-pass partials
  bytes += std::max(std::max(2 * res_rows * DP * elem, (size_t)(4 * CH + 16 / elem) * DP * elem),
                    (size_t)BWD_NW * WAVE * (4 + 4 * (DP / 16)) * 4);
  if (!stream) bytes += (size_t)BWD_STREAM_VECS * Np * 4;                 // vectors, xs, dxc
  bytes += (2 * loc + 3 * loc + 68) * 4;                                  // lres, lout, dxs, dpw
  bytes += (size_t)(stream ? BWD_STREAM_SCRATCH : BWD_SCRATCH) * 4;
  return bytes;
}

template <typename T, int DP, bool STREAM, bool GEN>
static hipError_t launch_bwd_t(const SinkBwdArgs& a, size_t lds, hipStream_t stream, bool coop) {
  auto kern = sinkhorn_bwd_kernel<T, DP, STREAM, GEN>;
  hipError_t e = set_lds_limit((const void*)kern, lds);
  if (e != hipSuccess) return e;
  dim3 grid(grid_blocks(a.B * a.H, a.G)), block(BWD_NT);
  SinkBwdArgs copy = a;
  if (coop) {
    void* args[] = {&copy};
    return hipLaunchCooperativeKernel((const void*)kern, grid, block, args, (unsigned)lds, stream);
  }
  hipLaunchKernelGGL(kern, grid, block, lds, stream, copy);
  return hipGetLastError();
}

template <bool STREAM, bool GEN>
hipError_t launch_bwd_dt(const SinkBwdArgs& a, bool bf16_in, int DP, size_t lds, hipStream_t stream, bool coop) {
  if (bf16_in) {
    if (DP == 32) return launch_bwd_t<bf16, 32, STREAM, GEN>(a, lds, stream, coop);
    if (DP == 64) return launch_bwd_t<bf16, 64, STREAM, GEN>(a, lds, stream, coop);
  } else {
    if (DP == 32) return launch_bwd_t<float, 32, STREAM, GEN>(a, lds, stream, coop);
    if (DP == 64) return launch_bwd_t<float, 64, STREAM, GEN>(a, lds, stream, coop);
  }
  return hipErrorInvalidValue;
}

template <bool STREAM>
hipError_t launch_bwd_mode(const SinkBwdArgs& a, bool bf16_in, int DP, size_t lds, hipStream_t stream, bool coop) {
  const bool gen = (a.bins8 && a.pos_w) || (a.x && a.w_dist);
  return gen ? launch_bwd_dt<STREAM, true>(a, bf16_in, DP, lds, stream, coop)
             : launch_bwd_dt<STREAM, false>(a, bf16_in, DP, lds, stream, coop);
}

}  // namespace dfl
