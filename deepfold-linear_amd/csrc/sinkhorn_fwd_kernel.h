// Flash-Sinkhorn forward: persistent per-(b,h) workgroup groups on gfx950.
//
// Restates the UOT log-domain Sinkhorn of vv137/deepfold-linear
// (src/deepfold/model/kernels/flash_sinkhorn_attn.py:144-218, same math as
// sinkhorn_kernel.py:1106-1492) without materialising the N x N plan:
//
//   u_i = kappa (log mu_i - LSE_j(L_ij + v_j))      (row update, valid j)
//   v_j = kappa (log nu_j - LSE_i(L_ij + u_i))      (column update, valid i)
//   L_ij = -C_ij / eps_h,  C_ij = -(q_i.k_j)/sqrt(d) + pw_h[bins_ij] + w_h d_ij/(r0 + d_ij)
//
// Work split: each (b,h) is served by a group of G workgroups.  Member m owns a
// contiguous stripe of 16-row tiles, used as plan rows in the row update and as
// plan columns in the column update.  The cost tile is recomputed on MFMA every
// sweep.  After each half-iteration the stripe's new potentials are published
// as tagged 64-bit words and every member gathers the full vector (common.h).
//
// Two storage modes (template flag STREAM):
//   resident: Q and K of the whole (b,h) stay in LDS for all iterations;
//   stream  : only the member's own Q and K stripes sit in LDS; the streamed
//             operand is read from zero-padded copies in global memory
//             (sinkhorn_pad_kernel), which stay L2-resident.  Used when the
//             resident layout does not fit in 160 KB of LDS (long sequences).
//
// Balanced mode (SinkFwdArgs::balanced) restates the balanced transport of
// flash_sinkhorn_transport.py:253-282 with the same machinery: column update
// first, kappa = 1, log marginals -log(n_valid) of the sample, logit
// (1 - w_h)(q.k)/eps - w_h d/(r + d)/eps (the constant (1 - w_h)/eps of the cost
// 1 - q.k shifts every column potential equally and leaves the plan unchanged),
// and the potentials of every half-iteration written to a history for the
// unrolled backward.  The last update is a row update, so the plan's rows sum to
// 1/n exactly and the output pass normalises by the row LSE of that update.
//
// All logits are handled in log2 units (x * log2 e) so that exp2 maps onto
// v_exp_f32 directly.
#pragma once
#include <type_traits>

#include "sinkhorn_args.h"
#include "sinkhorn_engine.h"

namespace dfl {

constexpr int FWD_NT = 512;  // 8 waves: two per SIMD for latency hiding
constexpr int FWD_NW = FWD_NT / WAVE;
// Largest |change| of a potential between two sweeps (log2 units) for which the
// previous LSE is used as the exponent shift: every term is then <= 2^delta and
// the sum >= 2^-delta, far inside fp32 range.
constexpr float FIXED_SHIFT_MAX_DELTA = 64.f;
// Stream mode: streamed rows per LDS chunk of the transport-output pass.
constexpr int FWD_OCH = 128;

__host__ __device__ inline int fwd_local_rows(int N, int G) { return 16 * (((N + 15) / 16 + G - 1) / G); }
// Stream mode: rows of the K region (the K stripe; the output pass reuses it for
// one K chunk and one transposed V chunk).
__host__ __device__ inline int fwd_kregion_rows(int N, int G) {
  const int l = fwd_local_rows(N, G);
  return l > 2 * FWD_OCH ? l : 2 * FWD_OCH;
}

template <typename T, int DP, bool GENERAL, bool TRANS, typename Pub>
__device__ __forceinline__ void fwd_sweep(bool online, const T* res, const T* str, const float* w2, int n_tiles,
                                          int t0, int nr, float sc, const Bias& bias, float* lse, float* mx,
                                          float* scratch, unsigned* s_reset, Pub pub) {
  if (online)
    lse_sweep<FWD_NT, T, DP, GENERAL, TRANS, true>(res, str, w2, n_tiles, t0, nr, sc, bias, lse, lse, mx, scratch,
                                                   s_reset, pub);
  else
    lse_sweep<FWD_NT, T, DP, GENERAL, TRANS, false>(res, str, w2, n_tiles, t0, nr, sc, bias, lse, lse, mx, scratch,
                                                    s_reset, pub);
}

// Stream mode: res is the member's stripe (local tiles), str the padded global copy.
template <typename T, int DP, bool GENERAL, bool TRANS, typename Pub>
__device__ __forceinline__ void fwd_sweep_stream(bool online, const T* res, const T* str, const float* w2,
                                                 int n_tiles, int t0, int nr, float sc, const Bias& bias, float* lse,
                                                 float* mx, float* scratch, unsigned* s_reset, Pub pub) {
  if (online)
    stream_sweep<FWD_NT, T, DP, SW_LSE_ONLINE, GENERAL, TRANS>(res, str, w2, nullptr, n_tiles, t0, nr, sc, lse, bias,
                                                               lse, mx, scratch, s_reset, pub);
  else
    stream_sweep<FWD_NT, T, DP, SW_LSE_FIXED, GENERAL, TRANS>(res, str, w2, nullptr, n_tiles, t0, nr, sc, lse, bias,
                                                              lse, mx, scratch, s_reset, pub);
}

// Outputs of one resident 16-row tile after the transport pass.  oacc holds
// sum_j p_ij V_j in the accumulator layout (lane: row 4g + r, column c*16 + l%16);
// xc0..2 the lane's partial sums of p_ij x_j for row tile*16 + l%16.  l2 is this
// lane's row LSE (log2) and lse2_t / mx2_t point at the tile's 16 row entries.
template <typename T, int DP>
__device__ __forceinline__ void fwd_write_tile(const SinkFwdArgs& a, int b, int h, int tile, int n,
                                               const unsigned char* valid, const float* lse2_t, const float* mx2_t,
                                               const float* vecU, const float* vecV, const f32x4* oacc, float xc0,
                                               float xc1, float xc2, const T* Gg, int lane, bool bal) {
  constexpr int NC = DP / 16;
  const int N = a.N, d = a.d;
  const int g = lane >> 4;
  const size_t bh = (size_t)b * a.H + h;
  const int irow = tile * 16 + (lane & 15);
  const float l2 = lse2_t[lane & 15];
  xc0 = sum_groups(xc0);
  xc1 = sum_groups(xc1);
  xc2 = sum_groups(xc2);
  // T_norm = p / (1 + 1e-6 * 2^(max - lse))  <=>  reference T / (sum T + 1e-6), T = e^(s - max)
  if (lane < 16 && irow < n && valid[irow]) {
    const float den = bal ? 1.f : 1.f + 1e-6f * fast_exp2(mx2_t[lane] - l2);
    const size_t o = (bh * N + irow) * 3;
    a.x_centroid[o + 0] = xc0 / den;
    a.x_centroid[o + 1] = xc1 / den;
    a.x_centroid[o + 2] = xc2 / den;
    const float u = vecU[irow] * LN2;
    a.log_u[bh * N + irow] = u;
    a.log_z[bh * N + irow] = u + l2 * LN2;
    a.log_v[bh * N + irow] = vecV[irow] * LN2;
  } else if (lane < 16 && irow < N) {  // invalid row of my stripe
    const size_t o = (bh * N + irow) * 3;
    a.x_centroid[o + 0] = a.x_centroid[o + 1] = a.x_centroid[o + 2] = 0.f;
    a.log_u[bh * N + irow] = a.log_z[bh * N + irow] = a.log_v[bh * N + irow] = 0.f;
    if (!bal) a.col_lse[bh * N + irow] = 0.f;
  }
  if (bal && !a.o_avg) return;  // balanced mode without V: coordinate centroid only
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int row = tile * 16 + 4 * g + r;
    if (row < N && !(row < n && valid[row])) {
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const int col = c * 16 + (lane & 15);
        if (col < d) {
          a.o_avg[(bh * N + row) * d + col] = 0.f;
          if (!bal) a.o_flat[((size_t)b * N + row) * (size_t)(a.H * d) + (size_t)h * d + col] = 0.f;
        }
      }
    }
    if (row < n && valid[row]) {
      const float den = bal ? 1.f : 1.f + 1e-6f * fast_exp2(mx2_t[4 * g + r] - lse2_t[4 * g + r]);
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const int col = c * 16 + (lane & 15);
        if (col < d) {
          const float o = oacc[c][r] / den;
          a.o_avg[(bh * N + row) * d + col] = o;
          if (!bal) {
            const float sg = Gg ? 1.f / (1.f + __expf(-to_f32(Gg[(size_t)row * a.sn + col]))) : 1.f;
            a.o_flat[((size_t)b * N + row) * (size_t)(a.H * d) + (size_t)h * d + col] = sg * o;
          }
        }
      }
    }
  }
}

// Resident-storage output pass for the row tiles [t0, t0 + nr): O_avg = T_norm V,
// x_c = T_norm x and the per-row outputs (fwd_write_tile), from the final row LSE
// lse2 and row maxima mx2 (local rows of the tile range) and the final potentials
// vecU (these rows) and vecV (all columns), log2 units.  K is read from KS (all
// rows); V^T is staged over QS; Q fragments come from global memory.  Called by
// the whole block.
// part / part_floats: free LDS for partial sums.  Where it holds them, the P =
// min(8 / nr, ...) waves of a tile take every P-th pair of streamed tiles each
// (nr < 8 leaves waves idle otherwise); the tile's first wave adds the others'
// partials in wave order and writes the tile.
template <typename T, int DP>
__device__ __forceinline__ void fwd_resident_output(const SinkFwdArgs& a, int b, int h, int n, int n_tiles, int Np,
                                                    int t0, int nr, const unsigned char* valid, T* QS, const T* KS,
                                                    const float* vecU, const float* vecV, const float* xs,
                                                    const float* lse2, const float* mx2, float sc, const Bias& bias,
                                                    bool general, bool bal, bool has_v, const T* Qg, const T* Vg,
                                                    const T* Gg, float* part = nullptr, int part_floats = 0) {
  using M = Mfma<T, DP>;
  const int N = a.N, d = a.d;
  const int lane = threadIdx.x & (WAVE - 1);
  const int wave = threadIdx.x / WAVE;
  const int g = lane >> 4;
  constexpr int NC = DP / 16;
  constexpr int PF = 4 * NC + 3;  // floats of one lane's partial: O accumulators, x_c sums
  // V^T replaces Q in LDS; resident Q fragments are read from global memory.
  T* VT = QS;  // [DP][Np]
  __syncthreads();
  if (has_v) stage_rows_t<T, DP>(VT, Vg, a.sn, n, d, Np);
  __syncthreads();
  const int n_pairs = (n_tiles + 1) / 2;
  int P = nr < FWD_NW ? FWD_NW / nr : 1;
  if (P > 1) P = min(P, 1 + part_floats / (nr * WAVE * PF));
  const int slots = P > 1 ? nr * P : nr;
  for (int wi = wave; wi < slots; wi += FWD_NW) {
    const int rt = wi % nr, pi = wi / nr;
    const int tile = t0 + rt;
    const int qloc = rt * 16;
    const int irow = tile * 16 + (lane & 15);  // this lane's row in the P layout
    typename M::Frag qf;
    load_frag_global<T, DP>(qf, Qg, a.sn, irow, n, d, lane);
    const float l2 = lse2[qloc + (lane & 15)];
    f32x4 oacc[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) oacc[c] = f32x4{0.f, 0.f, 0.f, 0.f};
    float xc0 = 0.f, xc1 = 0.f, xc2 = 0.f;
    for (int sp = pi; sp < n_pairs; sp += P) {
      f32x4 p[2];
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const int st = 2 * sp + half;
        p[half] = f32x4{0.f, 0.f, 0.f, 0.f};
        if (st < n_tiles) {
          typename M::Frag af;
          M::load(af, KS + (size_t)(st * 16 + (lane & 15)) * DP, lane);
          const f32x4 w = *reinterpret_cast<const f32x4*>(vecV + st * 16 + 4 * g);
          const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
          const f32x4 acc = M::qk(af, qf, zero);
#pragma unroll
          for (int kk = 0; kk < 4; ++kk) {
            const int j = st * 16 + 4 * g + kk;
            float x = __builtin_fmaf(acc[kk], sc, w[kk]);
            if (general && w[kk] > 0.5f * NEG_BIG) x += bias(irow, j);
            const float pv = fast_exp2(x - l2);
            p[half][kk] = pv;
            xc0 = __builtin_fmaf(pv, xs[3 * j], xc0);
            xc1 = __builtin_fmaf(pv, xs[3 * j + 1], xc1);
            xc2 = __builtin_fmaf(pv, xs[3 * j + 2], xc2);
          }
        }
      }
      if (has_v) {
#pragma unroll
        for (int c = 0; c < NC; ++c)
          oacc[c] = M::pv_split(p[0], p[1], VT + (size_t)(c * 16 + (lane & 15)) * Np + sp * 32, lane, oacc[c]);
      }
    }
    if (P == 1) {
      fwd_write_tile<T, DP>(a, b, h, tile, n, valid, lse2 + qloc, mx2 + qloc, vecU, vecV, oacc, xc0, xc1, xc2, Gg,
                            lane, bal);
      continue;
    }
    // slots <= FWD_NW: every wave holds at most one (tile, part)
    float* my = part + ((size_t)(pi > 0 ? pi - 1 : 0) * nr + rt) * WAVE * PF + lane;
    if (pi > 0) {
#pragma unroll
      for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int r = 0; r < 4; ++r) my[(4 * c + r) * WAVE] = oacc[c][r];
      my[(4 * NC) * WAVE] = xc0;
      my[(4 * NC + 1) * WAVE] = xc1;
      my[(4 * NC + 2) * WAVE] = xc2;
    }
    __syncthreads();
    if (pi == 0) {
      for (int q = 1; q < P; ++q) {
        const float* src = part + ((size_t)(q - 1) * nr + rt) * WAVE * PF + lane;
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
          for (int r = 0; r < 4; ++r) oacc[c][r] += src[(4 * c + r) * WAVE];
        xc0 += src[(4 * NC) * WAVE];
        xc1 += src[(4 * NC + 1) * WAVE];
        xc2 += src[(4 * NC + 2) * WAVE];
      }
      fwd_write_tile<T, DP>(a, b, h, tile, n, valid, lse2 + qloc, mx2 + qloc, vecU, vecV, oacc, xc0, xc1, xc2, Gg,
                            lane, bal);
    }
  }
  if (P > 1 && wave >= slots) __syncthreads();  // the idle waves' share of the merge barrier
}

// MODE (compile time, so the plain UOT instantiation carries none of the other
// modes' code): FWD_UOT, FWD_UOT_HIST (also records the potentials history for the
// unrolled backward) or FWD_BALANCED (balanced transport, history recorded).  The
// host picks FWD_BALANCED exactly when a.balanced != 0 and FWD_UOT_HIST when a.hist
// is given.
// GEN: the cost may carry position bins or geometry (the host sets it when either
// is passed); GEN = false compiles no bias code, which keeps the content-only
// sweeps at their register budget.
enum FwdMode : int { FWD_UOT = 0, FWD_UOT_HIST = 1, FWD_BALANCED = 2, FWD_UOT_REG = 3 };

// Register storage of the resident layout (FWD_UOT_REG): a wave holds the logits of
// its pairs (resident tile r < nr of the member's stripe, streamed tile wave + 8 k,
// k < KS) in VGPRs, KS = ceil(n_tiles / 8) rounded up to 2, 4 or 6 and nr at most
// reg_nrm(KS) (at most 18 pairs per direction, 144 VGPRs for both).
__host__ __device__ constexpr int reg_ks(int n_tiles) {
  return (n_tiles + 7) / 8 <= 2 ? 2 : ((n_tiles + 7) / 8 <= 4 ? 4 : ((n_tiles + 7) / 8 <= 6 ? 6 : 0));
}
__host__ __device__ constexpr int reg_nrm(int ks) { return ks == 6 ? 3 : 4; }
// Whether every member of every group fits when G members share up to N tokens (a
// group with fewer valid tokens has no more stripe tiles and no more slots).
__host__ __device__ inline bool reg_fits(int N, int G) {
  const int T = (N + 15) / 16, ks = reg_ks(T);
  return ks > 0 && G >= 1 && (T + G - 1) / G <= reg_nrm(ks);
}
// Entries of the split-potential arrays: every slot's streamed tile reads inside them.
__host__ __device__ inline int reg_cp_rows(int N, int rcap) {
  const int r = 8 * 16 * reg_ks((N + 15) / 16);
  return rcap > r ? rcap : r;
}
template <typename T, int DP, bool STREAM, int MODE, bool GEN>
__global__ void __launch_bounds__(FWD_NT) sinkhorn_fwd_kernel(SinkFwdArgs a) {
  constexpr bool BAL = MODE == FWD_BALANCED;
  constexpr bool HIST = MODE == FWD_UOT_HIST || MODE == FWD_BALANCED;
  constexpr bool REG = !STREAM && MODE == FWD_UOT_REG;
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ int s_flag, s_tmp, s_local;
  __shared__ unsigned s_du, s_dv;
  __shared__ int s_cnt;
  __shared__ int s_flagp[2];  // resident dataflow: expired waits of the half-iterations, by parity
  __shared__ float s_posw[BIN_NONE + 1];
  int grp, member;
  if (!group_of(a.B * a.H, a.G, grp, member)) return;  // surplus workgroup of the XCD-aligned grid
  const int b = grp / a.H, h = grp % a.H;
  const int N = a.N, d = a.d;
  const int Np = ((N + 31) / 32) * 32;
  constexpr bool bal = BAL;
  const bool has_v = !BAL || (a.v != nullptr && a.o_avg != nullptr);  // UOT mode always has V
  if (threadIdx.x == 0) { s_flag = 0; s_du = 0u; s_dv = 0u; s_cnt = 0; s_local = 1; s_flagp[0] = s_flagp[1] = 0; }
  if (blockIdx.x == 0 && threadIdx.x == 0)
    __hip_atomic_store(a.err.ws + 1, a.salt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

  // ---- LDS carve-up (must match sinkhorn_fwd_lds_bytes)
  const int loc = fwd_local_rows(N, a.G);
  // resident: Q, K and the potentials padded to the lean sweep's row groups
  // (zero operands, NEG_BIG potentials past the valid tokens)
  const int rcap = STREAM ? Np : lean_rows<FWD_NT>(Np, lean_sch<T, DP>());
  const int q_rows = STREAM ? loc : rcap;
  const int k_rows = STREAM ? fwd_kregion_rows(N, a.G) : rcap;
  unsigned char* valid = smem;
  T* QS = reinterpret_cast<T*>(smem + ((Np + 15) / 16) * 16);     // resident: all rows; stream: my stripe
  T* KS = QS + (size_t)q_rows * DP;
  float* vecU = reinterpret_cast<float*>(KS + (size_t)k_rows * DP);  // u of all rows (log2)
  float* vecV = vecU + rcap;                                        // v of all columns (log2)
  float* xs = vecV + rcap;                                          // resident only: [Np][3]
  float* lse_r = xs + (STREAM ? 0 : 3 * Np);  // row LSE of my rows (log2); shift of the next row sweep
  float* lse_c = lse_r + loc;   // column LSE of my columns (log2)
  float* mx2 = lse_c + loc;     // row maxima of the final sweep
  float* lmu_l = mx2 + loc;     // log mu of my rows
  float* lnu_l = lmu_l + loc;   // log nu of my columns
  float* scratch = lnu_l + loc;
  // register storage: split parts of u and v (by index) and of -shift of my rows / columns
  const int cpn = REG ? reg_cp_rows(N, rcap) : 0;
  bf16x4* cpU = reinterpret_cast<bf16x4*>(scratch + sweep_scratch<FWD_NT>());
  bf16x4* cpV = cpU + cpn;
  bf16x4* rpR = cpV + cpn;
  bf16x4* rpC = rpR + loc;

  const int n = mask_setup(a.mask ? a.mask + (size_t)b * N : nullptr, N, valid, &s_tmp);
  const int n_tiles = (n + 15) / 16;
  int t0, t1;
  stripe(n_tiles, member, a.G, t0, t1);
  const int nr = t1 - t0;
  {
    // Every output position is written: rows past the last valid tile, which no
    // stripe owns, are zeroed here (row i by member i % G); invalid rows inside
    // stripes are zeroed where the stripe's outputs are written.
    const size_t bh0 = (size_t)b * a.H + h;
    for (int i = n_tiles * 16 + member; i < N; i += a.G) {
      for (int c = threadIdx.x; c < d; c += FWD_NT) {
        if (has_v) a.o_avg[(bh0 * N + i) * d + c] = 0.f;
        if (!BAL) a.o_flat[((size_t)b * N + i) * (size_t)(a.H * d) + (size_t)h * d + c] = 0.f;
      }
      if (threadIdx.x < 3) a.x_centroid[(bh0 * N + i) * 3 + threadIdx.x] = 0.f;
      if (threadIdx.x == 0) {
        a.log_u[bh0 * N + i] = 0.f;
        a.log_v[bh0 * N + i] = 0.f;
        a.log_z[bh0 * N + i] = 0.f;
        if (!BAL) a.col_lse[bh0 * N + i] = 0.f;
      }
    }
  }
  if (n == 0 || nr <= 0) return;  // owns nothing; no other member waits on it

  const size_t bh = (size_t)b * a.H + h;
  const size_t qoff = (size_t)b * a.sb + (size_t)h * a.sh;
  const T* Qg = reinterpret_cast<const T*>(a.q) + qoff;
  const T* Kg = reinterpret_cast<const T*>(a.k) + qoff;
  const T* Vg = reinterpret_cast<const T*>(a.v) + qoff;
  const T* Gg = a.g ? reinterpret_cast<const T*>(a.g) + qoff : nullptr;
  // stream mode: padded copies of this (b,h)
  const T* Qp = STREAM ? reinterpret_cast<const T*>(a.qp) + bh * Np * DP : nullptr;
  const T* Kp = STREAM ? reinterpret_cast<const T*>(a.kp) + bh * Np * DP : nullptr;
  const int r_lo = t0 * 16;
  if constexpr (STREAM) {
    stage_rows<T, DP>(QS, Qp + (size_t)r_lo * DP, DP, nr * 16, DP, loc);
    stage_rows<T, DP>(KS, Kp + (size_t)r_lo * DP, DP, nr * 16, DP, loc);
  } else {
    stage_rows<T, DP>(QS, Qg, a.sn, n, d, rcap);
    stage_rows<T, DP>(KS, Kg, a.sn, n, d, rcap);
  }

  const float eps = a.eps[h];
  const float w_bal = bal ? 1.f / (1.f + __expf(-a.alpha[h])) : 0.f;
  const float kappa = bal ? 1.f : a.lam / (a.lam + eps);
  const float sc = bal ? LOG2E * (1.f - w_bal) / eps : LOG2E / (sqrtf((float)d) * eps);
  float lmarg = 0.f;  // balanced: log(1 / n_valid) of this sample
  if (bal) {
    int c = 0;
    for (int i = threadIdx.x; i < n; i += FWD_NT) c += valid[i];
    atomicAdd(&s_cnt, c);
    __syncthreads();
    lmarg = -logf((float)max(s_cnt, 1));
  }
  for (int q = threadIdx.x; q < nr * 16; q += FWD_NT) {
    const int i = r_lo + q;
    lmu_l[q] = i < n ? (bal ? lmarg : a.log_mu[bh * N + i]) : 0.f;
    lnu_l[q] = i < n ? (bal ? lmarg : a.log_nu[bh * N + i]) : 0.f;
  }
  for (int i = threadIdx.x; i < rcap; i += FWD_NT) {
    const bool ok = i < n && valid[i];
    vecU[i] = ok ? (a.u_init ? a.u_init[bh * N + i] * LOG2E : 0.f) : NEG_BIG;
    vecV[i] = ok ? (a.v_init ? a.v_init[bh * N + i] * LOG2E : 0.f) : NEG_BIG;
  }
  if constexpr (REG) {
    for (int i = threadIdx.x; i < cpn; i += FWD_NT) {  // the same thread wrote vecU[i], vecV[i]
      cpU[i] = split3(i < rcap ? vecU[i] : NEG_BIG);
      cpV[i] = split3(i < rcap ? vecV[i] : NEG_BIG);
    }
    for (int q = threadIdx.x; q < loc; q += FWD_NT) rpR[q] = rpC[q] = split3(0.f);
  }
  const float w_h = bal ? w_bal : (a.w_dist ? a.w_dist[h] : 0.f);
  const bool use_geo = GEN && (a.x != nullptr) && (w_h != 0.f);
  const bool use_pos = GEN && (a.bins8 != nullptr) && (a.pos_w != nullptr);
  if (use_pos)
    for (int k = threadIdx.x; k <= (int)BIN_NONE; k += FWD_NT)
      s_posw[k] = k < (int)BIN_NONE ? -LOG2E * a.pos_w[h * 68 + k] / eps : 0.f;
  // coordinates of this batch row: LDS (resident) or the padded global copy (stream)
  const float* xsrc = xs;
  if constexpr (STREAM) {
    xsrc = a.xs_p + (size_t)b * Np * 3;
  } else {
    for (int e = threadIdx.x; e < 3 * Np; e += FWD_NT) xs[e] = (a.x && e < 3 * n) ? a.x[(size_t)b * N * 3 + e] : 0.f;
  }
  __syncthreads();
  Bias bias;
  bias.b8 = use_pos ? a.bins8 + (size_t)b * Np * Np : nullptr;
  bias.b8t = use_pos ? a.bins8t + (size_t)b * Np * Np : nullptr;
  bias.posw = s_posw;
  bias.xs = use_geo ? xsrc : nullptr;
  bias.geo_scale = -LOG2E * w_h / eps;
  bias.r0 = bal ? fmaxf(fabsf(a.r_h[h]), 0.1f) : a.r0;
  bias.Np = Np;
  const bool general = use_pos || use_geo;

  // sweep dispatch: ROW = plan rows resident (Q), streamed K against v; else the transpose
  auto sweep = [&](bool row, bool online, float* lse, float* mx, unsigned* s_reset, auto pub)
                   __attribute__((always_inline)) {
    if constexpr (STREAM) {
      const T* res = row ? QS : KS;
      const T* str = row ? Kp : Qp;
      const float* w2 = row ? vecV : vecU;
      if (row) {
        if (general) fwd_sweep_stream<T, DP, true, false>(online, res, str, w2, n_tiles, t0, nr, sc, bias, lse, mx, scratch, s_reset, pub);
        else fwd_sweep_stream<T, DP, false, false>(online, res, str, w2, n_tiles, t0, nr, sc, bias, lse, mx, scratch, s_reset, pub);
      } else {
        if (general) fwd_sweep_stream<T, DP, true, true>(online, res, str, w2, n_tiles, t0, nr, sc, bias, lse, mx, scratch, s_reset, pub);
        else fwd_sweep_stream<T, DP, false, true>(online, res, str, w2, n_tiles, t0, nr, sc, bias, lse, mx, scratch, s_reset, pub);
      }
    } else {
      const T* res = row ? QS : KS;
      const T* str = row ? KS : QS;
      const float* w2 = row ? vecV : vecU;
      if (!online) {
        if (row) {
          if (general) lean_sweep<FWD_NT, T, DP, true, false>(res, str, w2, n_tiles, t0, nr, sc, bias, lse, scratch, s_reset, pub);
          else lean_sweep<FWD_NT, T, DP, false, false>(res, str, w2, n_tiles, t0, nr, sc, bias, lse, scratch, s_reset, pub);
        } else {
          if (general) lean_sweep<FWD_NT, T, DP, true, true>(res, str, w2, n_tiles, t0, nr, sc, bias, lse, scratch, s_reset, pub);
          else lean_sweep<FWD_NT, T, DP, false, true>(res, str, w2, n_tiles, t0, nr, sc, bias, lse, scratch, s_reset, pub);
        }
      } else if (row) {
        if (general) fwd_sweep<T, DP, true, false>(true, res, str, w2, n_tiles, t0, nr, sc, bias, lse, mx, scratch, s_reset, pub);
        else fwd_sweep<T, DP, false, false>(true, res, str, w2, n_tiles, t0, nr, sc, bias, lse, mx, scratch, s_reset, pub);
      } else {
        if (general) fwd_sweep<T, DP, true, true>(true, res, str, w2, n_tiles, t0, nr, sc, bias, lse, mx, scratch, s_reset, pub);
        else fwd_sweep<T, DP, false, true>(true, res, str, w2, n_tiles, t0, nr, sc, bias, lse, mx, scratch, s_reset, pub);
      }
    }
  };

  uint64_t* xu = a.xch + bh * 2 * (size_t)Np;  // u words
  uint64_t* xv = xu + Np;                       // v words
  const uint32_t salt = a.salt << 12;
  uint32_t phase = 0;
  // placement words of the group (after all (b,h)'s u/v words); plain-store
  // publishing from the second exchange on if every member is on its XCD
  uint64_t* xpl = a.xch + (size_t)a.B * a.H * 2 * Np + bh * 32;
  publish_placement(xpl, member, a.salt);
  bool local = false;
  auto agree_placement = [&]() __attribute__((always_inline)) -> bool {
    if (phase != 1) return true;
    if (!read_placement(xpl, a.G, n_tiles, a.salt, a.err, &s_flag, &s_local)) return false;
    local = s_local != 0;
    return true;
  };

  // History for the unrolled backward: this member's stripe of the vector just
  // exchanged, copied from its own words (exact published values), outside the sweep.
  auto record = [&](const uint64_t* words, int slot) __attribute__((always_inline)) {
    for (int q = threadIdx.x; q < nr * 16; q += FWD_NT) {
      const int i = r_lo + q;
      if (i < n) {
        const uint64_t w = __hip_atomic_load(const_cast<uint64_t*>(words + i), __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT);
        a.hist[((size_t)slot * a.B * a.H + bh) * N + i] = valid[i] ? __uint_as_float((uint32_t)(w >> 32)) : 0.f;
      }
    }
  };
  // Resident storage runs dataflow half-iterations (flow_sweep): each wave polls the
  // previous half-iteration's words of its own streamed tiles, chooses its shift from
  // their change, and the wave partials are combined after the chunk's barrier; no
  // block-wide gather.  The first sweep of each direction is online.  A wait that
  // expires sets the flag of its half-iteration's parity, read after that
  // half-iteration's last barrier (a wave can be at most one half-iteration ahead).
  int chunk = 0;
  auto flow_poll = [&](uint64_t* words, float* w2, int it) __attribute__((always_inline)) -> bool {
    if (phase == 1) return true;  // the first sweep reads the initial potentials
    float dm;
    if (!wave_gather<FWD_NW>(words, n, n_tiles, (salt | phase) - 1, w2, valid, a.err, dm)) s_flagp[phase & 1] = 1;
    return it == 0 || !(dm <= FIXED_SHIFT_MAX_DELTA);
  };
  // ---- row update: u_i = kappa (log mu_i - LSE_j(L_ij + v_j)) for my rows
  auto row_update = [&](int it) __attribute__((always_inline)) -> bool {
    ++phase;
    if constexpr (!STREAM) {
      const uint32_t tag = salt | phase;
      const bool online = flow_poll(xv, vecV, it) || it == 0;
      auto pub = [&](int q, float l2) {
        const int i = r_lo + q;
        if (i < n) {
          const float u = kappa * (lmu_l[q] - l2 * LN2);
          xch_put(xu + i, u, tag, local);
          if constexpr (HIST) a.hist[((size_t)(2 * it + 1) * a.B * a.H + bh) * N + i] = valid[i] ? u : 0.f;
        }
      };
      if (general) flow_sweep<FWD_NT, T, DP, true, false>(online, QS, KS, vecV, n_tiles, t0, nr, sc, bias, lse_r, scratch, chunk, pub);
      else flow_sweep<FWD_NT, T, DP, false, false>(online, QS, KS, vecV, n_tiles, t0, nr, sc, bias, lse_r, scratch, chunk, pub);
      if (s_flagp[phase & 1]) return false;
      return agree_placement();
    } else {
      const uint32_t tag = salt | phase;
      const bool online = it == 0 || __uint_as_float(s_dv) > FIXED_SHIFT_MAX_DELTA;
      auto pub = [&](int q, float l2) {
        const int i = r_lo + q;
        if (i < n) xch_put(xu + i, kappa * (lmu_l[q] - l2 * LN2), tag, local);
      };
      sweep(true, online, lse_r, nullptr, &s_du, pub);
      if (!gather_potential<FWD_NT>(xu, n, tag, vecU, valid, a.err, &s_flag, &s_du)) return false;
      if (!agree_placement()) return false;
      if constexpr (HIST) record(xu, 2 * it + 1);
    }
    return true;
  };
  // ---- column update: v_j = kappa (log nu_j - LSE_i(L_ij + u_i)) for my columns
  auto col_update = [&](int it) __attribute__((always_inline)) -> bool {
    ++phase;
    if constexpr (!STREAM) {
      const uint32_t tag = salt | phase;
      const bool online = flow_poll(xu, vecU, it) || it == 0;
      const bool last = it == a.K_iter - 1;
      auto pub = [&](int q, float l2) {
        const int j = r_lo + q;
        if (j < n) {
          const float v = kappa * (lnu_l[q] - l2 * LN2);
          xch_put(xv + j, v, tag, local);
          if (!BAL && last && valid[j]) a.col_lse[bh * N + j] = l2 * LN2;
          if constexpr (HIST) a.hist[((size_t)(2 * it) * a.B * a.H + bh) * N + j] = valid[j] ? v : 0.f;
        }
      };
      if (general) flow_sweep<FWD_NT, T, DP, true, true>(online, KS, QS, vecU, n_tiles, t0, nr, sc, bias, lse_c, scratch, chunk, pub);
      else flow_sweep<FWD_NT, T, DP, false, true>(online, KS, QS, vecU, n_tiles, t0, nr, sc, bias, lse_c, scratch, chunk, pub);
      if (s_flagp[phase & 1]) return false;
      return agree_placement();
    } else {
      const uint32_t tag = salt | phase;
      const bool online = it == 0 || __uint_as_float(s_du) > FIXED_SHIFT_MAX_DELTA;
      const bool last = it == a.K_iter - 1;
      auto pub = [&](int q, float l2) {
        const int j = r_lo + q;
        if (j < n) {
          xch_put(xv + j, kappa * (lnu_l[q] - l2 * LN2), tag, local);
          if (!BAL && last && valid[j]) a.col_lse[bh * N + j] = l2 * LN2;
        }
      };
      sweep(false, online, lse_c, nullptr, &s_dv, pub);
      if (!gather_potential<FWD_NT>(xv, n, tag, vecV, valid, a.err, &s_flag, &s_dv)) return false;
      if (!agree_placement()) return false;
      if constexpr (HIST) record(xv, 2 * it);
    }
    return true;
  };
  // The UOT order is row then column, the balanced order column then row.  One call
  // site per update in each instantiation: with two, the compiler outlines them
  // into calls with a stack frame.
  if constexpr (REG) {
    // ---- register storage: the logits of every wave's pairs stay in VGPRs
    bool reg_tail = false;  // the register tail wrote the outputs
    auto reg_loop = [&](auto ksc) __attribute__((always_inline)) -> bool {
      constexpr int KSL = decltype(ksc)::value;
      constexpr int NRM = reg_nrm(KSL);
      using M = Mfma<T, DP>;
      const int lane = threadIdx.x & (WAVE - 1);
      const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE);
      const int g = lane >> 4;
      if (nr > NRM) {  // the host's reg_fits rules this out
        if (threadIdx.x == 0) raise_error(a.err, a.salt, 3u);
        return false;
      }
      // S[r KSL + k]: row block (i resident, j streamed) and column block (j resident,
      // i streamed), sc q.k + bias, NEG_BIG where the wave has no tile
      f32x4 SR[NRM * KSL], SC[NRM * KSL];
#pragma unroll
      for (int r = 0; r < NRM; ++r) {
#pragma unroll
        for (int k = 0; k < KSL; ++k) {
          const int sl = r * KSL + k, st = wave + FWD_NW * k;
          SR[sl] = SC[sl] = f32x4{NEG_BIG, NEG_BIG, NEG_BIG, NEG_BIG};
          if (r < nr && st < n_tiles) {
            const int ri = (t0 + r) * 16 + (lane & 15), si = st * 16 + (lane & 15);
            typename M::Frag qr, kr, qs, ks;
            M::load(qr, QS + (size_t)ri * DP, lane);
            M::load(kr, KS + (size_t)ri * DP, lane);
            M::load(qs, QS + (size_t)si * DP, lane);
            M::load(ks, KS + (size_t)si * DP, lane);
            const f32x4 z = {0.f, 0.f, 0.f, 0.f};
            const f32x4 xr = M::qk(ks, qr, z);  // [m = j streamed][n = i resident]
            const f32x4 xc = M::qk(qs, kr, z);  // [m = i streamed][n = j resident]
            f32x4 br[1] = {z}, bc[1] = {z};
            if (general) {
              const int s0[1] = {st * 16 + 4 * g};
              bias.template quads<false, 1>(ri, s0, br);
              bias.template quads<true, 1>(ri, s0, bc);
            }
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              SR[sl][q] = __builtin_fmaf(xr[q], sc, br[0][q]);
              SC[sl][q] = __builtin_fmaf(xc[q], sc, bc[0][q]);
            }
          }
        }
      }
      // what the combining thread of local row / column q = threadIdx.x publishes with,
      // loaded once
      const int qc = threadIdx.x, ic = r_lo + qc;
      const bool in_c = qc < nr * 16 && ic < n, ok_c = in_c && valid[ic];
      const float lmu_c = in_c ? lmu_l[qc] : 0.f, lnu_c = in_c ? lnu_l[qc] : 0.f;
      for (int it = 0; it < a.K_iter; ++it) {
        // row update: u_i = kappa (log mu_i - LSE_j(L_ij + v_j))
        {
          ++phase;
          const uint32_t tag = salt | phase;
          bool online = it == 0;
          if (phase > 1) {
            float dm;
            if (!wave_gather<FWD_NW>(xv, n, n_tiles, tag - 1, vecV, valid, a.err, dm, cpV)) s_flagp[phase & 1] = 1;
            online = online || !(dm <= FIXED_SHIFT_MAX_DELTA);
          }
          float* part = scratch + (chunk & 1) * (FWD_NW * SK_RT * 16);
          ++chunk;
          reg_sweep<KSL, NRM, FWD_NW>(online, SR, nr, cpV, rpR, lse_r, part);
          lds_barrier();
          flow_combine<FWD_NW>(part, nr, lse_r, [&](int q, float l2) {
            if (in_c) xch_put(xu + ic, kappa * (lmu_c - l2 * LN2), tag, local);
            rpR[q] = split3(ok_c ? -l2 : 0.f);
          });
          // the other waves start polling once the combining threads have published:
          // earlier polls only load the L2 the publishing stores go through
          lds_barrier();
          if (s_flagp[phase & 1]) return false;
          if (!agree_placement()) return false;
        }
        // column update: v_j = kappa (log nu_j - LSE_i(L_ij + u_i))
        {
          ++phase;
          const uint32_t tag = salt | phase;
          const bool last = it == a.K_iter - 1;
          float dm;
          if (!wave_gather<FWD_NW>(xu, n, n_tiles, tag - 1, vecU, valid, a.err, dm, cpU)) s_flagp[phase & 1] = 1;
          const bool online = it == 0 || !(dm <= FIXED_SHIFT_MAX_DELTA);
          float* part = scratch + (chunk & 1) * (FWD_NW * SK_RT * 16);
          ++chunk;
          reg_sweep<KSL, NRM, FWD_NW>(online, SC, nr, cpU, rpC, lse_c, part);
          lds_barrier();
          flow_combine<FWD_NW>(part, nr, lse_c, [&](int q, float l2) {
            if (in_c) xch_put(xv + ic, kappa * (lnu_c - l2 * LN2), tag, local);
            rpC[q] = split3(ok_c ? -l2 : 0.f);
            if (last && ok_c) a.col_lse[bh * N + ic] = l2 * LN2;
          });
          lds_barrier();  // as after the row combine
          if (s_flagp[phase & 1]) return false;
        }
      }
      // ---- Tail from the register logits (where the merge of the output partials
      // fits the Q and K region, dead after the prologue): the final row sweep (exact
      // log Z and row maxima) and the output pass, with no QK^T or bias recompute.
      // (head dim 32: at 64 the output accumulators no longer fit beside the logits)
      if constexpr (DP == 32) {
      constexpr int NC = DP / 16;
      constexpr int PF = 4 * NC + 3;  // floats of one lane's output partial
      if ((size_t)FWD_NW * nr * PF * WAVE * sizeof(float) > (size_t)2 * rcap * DP * sizeof(T)) return true;
      T* VT = QS;  // [DP][Np]; its loads overlap the final sweep
      stage_rows_t<T, DP>(VT, Vg, a.sn, n, d, Np);
      {
        const int fp = (phase + 1) & 1;  // the flag parity of this extra half-iteration
        float dm;
        if (!wave_gather<FWD_NW>(xv, n, n_tiles, salt | phase, vecV, valid, a.err, dm, cpV)) s_flagp[fp] = 1;
        float* part = scratch + (chunk & 1) * (FWD_NW * SK_RT * 16);
        ++chunk;
        float* pmax = reinterpret_cast<float*>(cpU);  // u's parts are dead after the last column sweep
        reg_sweep<KSL, NRM, FWD_NW>(true, SR, nr, cpV, rpR, lse_r, part, pmax);
        lds_barrier();
        if (s_flagp[fp]) return false;
        if (qc < nr * 16) {
          float mm = NEG_BIG;
#pragma unroll
          for (int w_ = 0; w_ < FWD_NW; ++w_) mm = fmaxf(mm, pmax[qc * FWD_NW + w_]);
          mx2[qc] = mm;
        }
        flow_combine<FWD_NW>(part, nr, lse_r, [&](int q, float l2) { rpR[q] = split3(ok_c ? -l2 : 0.f); });
        __syncthreads();
      }
      // P_ij = exp2(S_ij + v_j - lse_i); each wave sums its streamed tiles, the
      // partials meet in LDS and the wave r writes resident tile r
      {
        bf16x4 A[KSL];
#pragma unroll
        for (int k = 0; k < KSL; ++k) A[k] = blk_col_operand(cpV, wave + FWD_NW * k, lane);
        f32x4 oacc[NRM][NC];
        float xc[NRM][3];
#pragma unroll
        for (int r = 0; r < NRM; ++r) {
#pragma unroll
          for (int c = 0; c < NC; ++c) oacc[r][c] = f32x4{0.f, 0.f, 0.f, 0.f};
          xc[r][0] = xc[r][1] = xc[r][2] = 0.f;
        }
#pragma unroll
        for (int r = 0; r < NRM; ++r) {
          if (r < nr) {
            const bf16x4 Bv = blk_row_operand(rpR, r, lane);
#pragma unroll
            for (int k = 0; k < KSL; ++k) {
              const int st = wave + FWD_NW * k;
              if (st < n_tiles) {
                const f32x4 x = mfma_rank(A[k], Bv, SR[r * KSL + k]);
                float pe[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) pe[e] = fast_exp2(x[e]);
                const f32x4* xj = reinterpret_cast<const f32x4*>(xs + 3 * (st * 16 + 4 * g));
                const f32x4 x0 = xj[0], x1 = xj[1], x2 = xj[2];
                const float xv[12] = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3],
                                      x2[0], x2[1], x2[2], x2[3]};
#pragma unroll
                for (int e = 0; e < 4; ++e)
#pragma unroll
                  for (int c = 0; c < 3; ++c) xc[r][c] = __builtin_fmaf(pe[e], xv[3 * e + c], xc[r][c]);
#pragma unroll
                for (int c = 0; c < NC; ++c)
                  oacc[r][c] = reg_pv<T>(pe, VT + (size_t)(c * 16 + (lane & 15)) * Np + st * 16 + 4 * g, oacc[r][c]);
              }
            }
          }
        }
        __syncthreads();  // V^T and the split parts are read
        float* mg = reinterpret_cast<float*>(QS);
#pragma unroll
        for (int r = 0; r < NRM; ++r) {
          if (r < nr) {
            float* dst = mg + (size_t)(wave * nr + r) * PF * WAVE + lane;
#pragma unroll
            for (int c = 0; c < NC; ++c)
#pragma unroll
              for (int e = 0; e < 4; ++e) dst[(4 * c + e) * WAVE] = oacc[r][c][e];
#pragma unroll
            for (int c = 0; c < 3; ++c) dst[(4 * NC + c) * WAVE] = xc[r][c];
          }
        }
        __syncthreads();
        if (wave < nr) {
          const int r = wave;
          f32x4 o[NC];
          float x3[3] = {0.f, 0.f, 0.f};
#pragma unroll
          for (int c = 0; c < NC; ++c) o[c] = f32x4{0.f, 0.f, 0.f, 0.f};
          for (int w_ = 0; w_ < FWD_NW; ++w_) {
            const float* src = mg + (size_t)(w_ * nr + r) * PF * WAVE + lane;
#pragma unroll
            for (int c = 0; c < NC; ++c)
#pragma unroll
              for (int e = 0; e < 4; ++e) o[c][e] += src[(4 * c + e) * WAVE];
#pragma unroll
            for (int c = 0; c < 3; ++c) x3[c] += src[(4 * NC + c) * WAVE];
          }
          fwd_write_tile<T, DP>(a, b, h, t0 + r, n, valid, lse_r + r * 16, mx2 + r * 16, vecU, vecV, o, x3[0], x3[1],
                                x3[2], Gg, lane, false);
        }
      }
      reg_tail = true;
      }
      return true;
    };
    const int ksg = reg_ks(n_tiles);
    bool ok;
    if (ksg == 2) ok = reg_loop(std::integral_constant<int, 2>{});
    else if (ksg == 4) ok = reg_loop(std::integral_constant<int, 4>{});
    else if (ksg == 6) ok = reg_loop(std::integral_constant<int, 6>{});
    else {
      if (threadIdx.x == 0) raise_error(a.err, a.salt, 3u);
      ok = false;
    }
    if (!ok || reg_tail) return;
  } else {
    for (int it = 0; it < a.K_iter; ++it) {
      if constexpr (BAL) {
        if (!col_update(it) || !row_update(it)) return;
      } else {
        if (!row_update(it) || !col_update(it)) return;
      }
    }
  }
  if (!STREAM && a.K_iter > 0) {
    // The output pass reads whole vectors.  The last half-iteration's is gathered by
    // the block; the other one is whole already (the last sweep's waves polled every
    // tile of it).
    if (!gather_potential<FWD_NT>(BAL ? xu : xv, n, salt | phase, BAL ? vecU : vecV, valid, a.err, &s_flag, &s_dv))
      return;
  }
  if (a.K_iter == 0 && !BAL) {
    auto pub = [&](int q, float l2) {
      const int j = r_lo + q;
      if (j < n && valid[j]) a.col_lse[bh * N + j] = l2 * LN2;
    };
    sweep(false, true, lse_c, nullptr, nullptr, pub);
  }

  // ---- final row LSE with the last v: exact log Z and the row maximum.  In
  // balanced mode the last update was a row update whose LSE is that value.
  if (!bal) sweep(true, true, lse_r, mx2, nullptr, NoPublish());
  const float* lse2 = lse_r;

  // ---- transport output for my rows: O_avg = T_norm V, x_c = T_norm x.
  using M = Mfma<T, DP>;
  const int lane = threadIdx.x & (WAVE - 1);
  const int wave = threadIdx.x / WAVE;
  const int g = lane >> 4;
  constexpr int NC = DP / 16;
  if constexpr (!STREAM) {
    // register storage: the sweep scratch and the split-potential arrays are free now
    const int free_floats = REG ? sweep_scratch<FWD_NT>() + (2 * cpn + 2 * loc) * 2 : 0;
    fwd_resident_output<T, DP>(a, b, h, n, n_tiles, Np, t0, nr, valid, QS, KS, vecU, vecV, xs, lse2, mx2, sc, bias,
                               general, bal, has_v, Qg, Vg, Gg, scratch, free_floats);
  } else {
    // Stream mode: K and V^T pass through LDS in chunks of FWD_OCH streamed rows
    // (the K stripe region is free now); resident Q fragments come from the Q stripe.
    T* KC = KS;                             // [FWD_OCH][DP]
    T* VC = KS + (size_t)FWD_OCH * DP;      // [DP][FWD_OCH]
    const T* Vt = reinterpret_cast<const T*>(a.vt) + bh * (size_t)DP * Np;
    constexpr int OB = 2;  // resident tiles per wave per batch
    constexpr int VE = 16 / sizeof(T);
    typedef __attribute__((__vector_size__(16))) int i32x4;
    for (int rb0 = 0; rb0 < nr; rb0 += OB * FWD_NW) {
      typename M::Frag qf[OB];
      f32x4 oacc[OB][NC];
      float xc[OB][3], l2v[OB];
#pragma unroll
      for (int k = 0; k < OB; ++k) {
        const int rt = rb0 + wave + FWD_NW * k;
        xc[k][0] = xc[k][1] = xc[k][2] = 0.f;
        l2v[k] = 0.f;
#pragma unroll
        for (int c = 0; c < NC; ++c) oacc[k][c] = f32x4{0.f, 0.f, 0.f, 0.f};
        if (rt < nr) {
          M::load(qf[k], QS + (size_t)(rt * 16 + (lane & 15)) * DP, lane);
          l2v[k] = lse2[rt * 16 + (lane & 15)];
        }
      }
      for (int c0 = 0; c0 < n_tiles * 16; c0 += FWD_OCH) {
        __syncthreads();
        stage_rows<T, DP>(KC, Kp + (size_t)c0 * DP, DP, min(FWD_OCH, Np - c0), DP, FWD_OCH);
        for (int e = threadIdx.x; has_v && e < DP * (FWD_OCH / VE); e += FWD_NT) {
          const int c = e / (FWD_OCH / VE), jv = e - c * (FWD_OCH / VE);
          i32x4 v = {0, 0, 0, 0};
          if (c0 + jv * VE < Np) v = *reinterpret_cast<const i32x4*>(Vt + (size_t)c * Np + c0 + jv * VE);
          *reinterpret_cast<i32x4*>(VC + (size_t)c * FWD_OCH + jv * VE) = v;
        }
        __syncthreads();
        const int npair = (min(FWD_OCH, n_tiles * 16 - c0) + 31) / 32;
        for (int sp = 0; sp < npair; ++sp) {
          typename M::Frag af[2];
          f32x4 w[2];
#pragma unroll
          for (int half = 0; half < 2; ++half) {
            const int st = c0 / 16 + 2 * sp + half;
            const int ls = st < n_tiles ? 2 * sp + half : 2 * sp;  // a dead half repeats a live tile
            M::load(af[half], KC + (size_t)(ls * 16 + (lane & 15)) * DP, lane);
            w[half] = *reinterpret_cast<const f32x4*>(vecV + (c0 / 16 + ls) * 16 + 4 * g);
            if (st >= n_tiles) w[half] = f32x4{NEG_BIG, NEG_BIG, NEG_BIG, NEG_BIG};
          }
#pragma unroll
          for (int k = 0; k < OB; ++k) {
            const int rt = rb0 + wave + FWD_NW * k;
            if (rt < nr) {
              const int irow = (t0 + rt) * 16 + (lane & 15);
              f32x4 p[2];
#pragma unroll
              for (int half = 0; half < 2; ++half) {
                const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
                const f32x4 acc = M::qk(af[half], qf[k], zero);
#pragma unroll
                for (int kk = 0; kk < 4; ++kk) {
                  const int j = c0 + (2 * sp + half) * 16 + 4 * g + kk;
                  float x = __builtin_fmaf(acc[kk], sc, w[half][kk]);
                  if (general && w[half][kk] > 0.5f * NEG_BIG) x += bias(irow, j);
                  const float pv = fast_exp2(x - l2v[k]);
                  p[half][kk] = pv;
                  const int jj = min(j, Np - 1);  // pv = 0 past the last tile
                  xc[k][0] = __builtin_fmaf(pv, xsrc[3 * jj], xc[k][0]);
                  xc[k][1] = __builtin_fmaf(pv, xsrc[3 * jj + 1], xc[k][1]);
                  xc[k][2] = __builtin_fmaf(pv, xsrc[3 * jj + 2], xc[k][2]);
                }
              }
              if (has_v) {
#pragma unroll
                for (int c = 0; c < NC; ++c)
                  oacc[k][c] = M::pv_split(p[0], p[1], VC + (size_t)(c * 16 + (lane & 15)) * FWD_OCH + sp * 32,
                                           lane, oacc[k][c]);
              }
            }
          }
        }
      }
#pragma unroll
      for (int k = 0; k < OB; ++k) {
        const int rt = rb0 + wave + FWD_NW * k;
        if (rt < nr)
          fwd_write_tile<T, DP>(a, b, h, t0 + rt, n, valid, lse2 + rt * 16, mx2 + rt * 16, vecU, vecV, oacc[k],
                                xc[k][0], xc[k][1], xc[k][2], Gg, lane, bal);
      }
    }
  }
}

// ---------------------------------------------------------------------------
inline size_t sinkhorn_fwd_lds_bytes_t(int N, int DP, int elem, int G, bool stream, bool reg = false) {
  const size_t Np = ((N + 31) / 32) * 32;
  const size_t loc = fwd_local_rows(N, G);
  size_t bytes = ((Np + 15) / 16) * 16;  // valid
  if (stream) {
    bytes += (loc + fwd_kregion_rows(N, G)) * DP * elem;  // Q stripe, K stripe / output chunks
    bytes += 2 * Np * 4;                                   // vecU, vecV
    bytes += 5 * loc * 4;                                  // lse_r, lse_c, mx2, lmu_l, lnu_l
    bytes += (size_t)stream_scratch<FWD_NT>() * 4;
  } else {
    const int sch = (elem == 2 && DP == 32) ? 6 : ((elem == 4 && DP == 64) ? 2 : 4);  // lean_sch<T, DP>()
    const size_t rcap = lean_rows<FWD_NT>((int)Np, sch);
    bytes += 2 * rcap * DP * elem;        // QS, KS (padded to the lean sweep's row groups)
    bytes += (2 * rcap + 3 * Np) * 4;     // vecU, vecV, xs
    bytes += 5 * loc * 4;                 // lse_r, lse_c, mx2, lmu_l, lnu_l
    bytes += (size_t)sweep_scratch<FWD_NT>() * 4;
    if (reg) bytes += (2 * (size_t)reg_cp_rows(N, (int)rcap) + 2 * loc) * 8;  // cpU, cpV, rpR, rpC
  }
  return bytes;
}

template <typename T, int DP, bool STREAM, int MODE, bool GEN>
static hipError_t launch_fwd_t(const SinkFwdArgs& a, size_t lds, hipStream_t stream, bool coop) {
  auto kern = sinkhorn_fwd_kernel<T, DP, STREAM, MODE, GEN>;
  hipError_t e = set_lds_limit((const void*)kern, lds);
  if (e != hipSuccess) return e;
  dim3 grid(grid_blocks(a.B * a.H, a.G)), block(FWD_NT);
  SinkFwdArgs copy = a;
  if (coop) {
    void* args[] = {&copy};
    return hipLaunchCooperativeKernel((const void*)kern, grid, block, args, (unsigned)lds, stream);
  }
  hipLaunchKernelGGL(kern, grid, block, lds, stream, copy);
  return hipGetLastError();
}

template <bool STREAM, int MODE, bool GEN>
hipError_t launch_fwd_dt(const SinkFwdArgs& a, bool bf16_in, int DP, size_t lds, hipStream_t stream, bool coop) {
  if (bf16_in) {
    if constexpr (MODE == FWD_BALANCED) return hipErrorInvalidValue;  // the balanced transport is fp32 only
    else {
      if (DP == 32) return launch_fwd_t<bf16, 32, STREAM, MODE, GEN>(a, lds, stream, coop);
      if (DP == 64) return launch_fwd_t<bf16, 64, STREAM, MODE, GEN>(a, lds, stream, coop);
    }
  } else {
    if (DP == 32) return launch_fwd_t<float, 32, STREAM, MODE, GEN>(a, lds, stream, coop);
    if (DP == 64) return launch_fwd_t<float, 64, STREAM, MODE, GEN>(a, lds, stream, coop);
  }
  return hipErrorInvalidValue;
}

template <bool GEN>
hipError_t launch_fwd_reg_dt(const SinkFwdArgs& a, bool bf16_in, int DP, size_t lds, hipStream_t stream, bool coop) {
  if (bf16_in) {
    if (DP == 32) return launch_fwd_t<bf16, 32, false, FWD_UOT_REG, GEN>(a, lds, stream, coop);
    if (DP == 64) return launch_fwd_t<bf16, 64, false, FWD_UOT_REG, GEN>(a, lds, stream, coop);
  } else {
    if (DP == 32) return launch_fwd_t<float, 32, false, FWD_UOT_REG, GEN>(a, lds, stream, coop);
    if (DP == 64) return launch_fwd_t<float, 64, false, FWD_UOT_REG, GEN>(a, lds, stream, coop);
  }
  return hipErrorInvalidValue;
}

template <bool STREAM>
hipError_t launch_fwd_mode(const SinkFwdArgs& a, bool bf16_in, int DP, size_t lds, hipStream_t stream, bool coop) {
  if (a.balanced) {
    if (!a.hist) return hipErrorInvalidValue;
    return launch_fwd_dt<STREAM, FWD_BALANCED, true>(a, bf16_in, DP, lds, stream, coop);
  }
  const bool gen = (a.bins8 && a.pos_w) || (a.x && a.w_dist);
  if (a.hist)
    return gen ? launch_fwd_dt<STREAM, FWD_UOT_HIST, true>(a, bf16_in, DP, lds, stream, coop)
               : launch_fwd_dt<STREAM, FWD_UOT_HIST, false>(a, bf16_in, DP, lds, stream, coop);
  return gen ? launch_fwd_dt<STREAM, FWD_UOT, true>(a, bf16_in, DP, lds, stream, coop)
             : launch_fwd_dt<STREAM, FWD_UOT, false>(a, bf16_in, DP, lds, stream, coop);
}

}  // namespace dfl
