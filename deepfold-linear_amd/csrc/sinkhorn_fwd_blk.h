// Flash-Sinkhorn forward with the logits held in registers for the whole launch.
//
// Same mathematics as sinkhorn_fwd_kernel (the UOT updates of
// flash_sinkhorn_attn.py:178-192 and the transport output :194-218); a different
// work split.  The G workgroups of a (b,h) group form an R x C grid of plan blocks:
// member (r, c) owns the plan rows I_r (a range of 16-row tiles) and the plan
// columns J_c, and computes the cost part of the logits of its block once,
//   S_ij = sc q_i.k_j + bias_ij      (log2 units, i in I_r, j in J_c),
// on MFMA into VGPRs, where it stays for all 2K half-iterations.  No sweep
// recomputes QK^T or the position / geometry terms.  A sweep adds the potentials
// with one bf16 MFMA per 16x16 tile, a rank-2 update whose operands carry
// three-part bf16 splits of the potentials (exact to fp32 rounding):
//   row sweep     x_ij = S_ij + v_j - s_i     (s_i: the row's previous LSE, the shift)
//   column sweep  x_ij = S_ij + u_i - t_j     (t_j: the column's previous LSE)
// then takes exp2 and sums.  Per element that is one exponential and one add.
//
// Exchange.  In a row update every member publishes, for each of its valid rows, the
// log2-sum-exp of its block's row segment as an absolute log2 value (tagged 64-bit
// words, common.h).  The C members of row block r each poll the C partials of their
// rows and combine them (max, sum of exp2, log2) in the same order, so all of them hold
// bit-identical u_i.  Column updates likewise over the R members of column block c.
// Each member decides per sweep whether the previous LSE is a safe exponent shift (the
// potentials its block reads moved by at most FIXED_SHIFT_MAX_DELTA) or takes an
// online maximum first; the published values do not depend on that choice.
//
// Members per group are chosen on the device from the valid lengths of the groups
// that share an XCD (blk_allocate): the 16 (b,h) of the headline workload (n = 501
// and 759 on each XCD) get 11 and 21 members, at most 16 x 7 tiles each, instead of 16 and 16
// with 2 x 32 and 3 x 48 tiles.
//
// Tail: members of row block 0 publish the final v; every member gathers it, stages Q
// and K into LDS and runs the resident output pass (fwd_resident_output) for its
// share of I_r (the final online row sweep, then O_avg = T_norm V and x_c = T_norm x).
#pragma once
#include "sinkhorn_blk_plan.h"
#include "sinkhorn_fwd_kernel.h"

namespace dfl {

// LDS that outlives the iterations (valid flags, final potentials, coordinates, the
// output pass's row LSE / maxima and sweep scratch); Q and K (resident layout of the
// output pass) share the rest with the iteration phase.
__host__ __device__ inline size_t blk_persist_lds(int Np) {
  size_t b = (size_t)((Np + 15) / 16) * 16;  // valid
  b += (size_t)2 * Np * 4;                   // vecU, vecV
  b += (size_t)3 * Np * 4;                   // xs
  b += (size_t)2 * Np * 4;                   // lse_r, mx2
  b += (size_t)sweep_scratch<FWD_NT>() * 4;
  return (b + 15) / 16 * 16;
}
inline size_t blk_lds_bytes(int N, int DP, int elem) {
  const int Np = ((N + 31) / 32) * 32;
  const size_t qk = (size_t)2 * Np * DP * elem;
  const size_t it = blk_iter_lds_bound((N + 15) / 16);
  return blk_persist_lds(Np) + (qk > it ? qk : it);
}

// One sweep of a wave's sub-block: row tiles wr0 .. wr0 + wr (wr <= BLK_WR, wave-uniform)
// against BLK_WC column tiles, of which the first wc are the wave's (wc0 .. wc0 + wc);
// the logits of the others are NEG_BIG, so they add exp2(-huge) = 0 and the inner loop
// over columns has no branch.  A[ic] are the column operands of the wave's columns.
//  ROW: per plan row, the lane's partial over the columns, sum of exp2(x) (MAX: maximum
//       of x) -> part[(slot * TR + tile) * 64 + lane].
//  column: per plan column (lane group g holds columns 4g .. 4g + 3 of a tile), partials
//       over the rows, stored so that the 16 row lanes of one column are consecutive:
//       part[(((slot * TC + tile) * 4 + g) * 4 + e) * 16 + lane % 16].
template <bool ROW, bool MAX>
__device__ __forceinline__ void blk_sweep(const f32x4 (&S)[BLK_WR][BLK_WC], const bf16x4 (&A)[BLK_WC], int wr, int wc,
                                          int wr0, int wc0, int slot, int TR, int TC, const bf16x4* rowp,
                                          float* part, int lane) {
  if constexpr (ROW) {
#pragma unroll
    for (int ir = 0; ir < BLK_WR; ++ir) {
      if (ir < wr) {
        const bf16x4 Bv = blk_row_operand(rowp, wr0 + ir, lane);
        float e[4 * BLK_WC];
#pragma unroll
        for (int ic = 0; ic < BLK_WC; ++ic) {
          const f32x4 x = mfma_rank(A[ic], Bv, S[ir][ic]);
#pragma unroll
          for (int q = 0; q < 4; ++q) e[4 * ic + q] = MAX ? x[q] : fast_exp2(x[q]);
        }
        float acc;
        if (MAX) {
#pragma unroll
          for (int w = 1; w < 4 * BLK_WC; w *= 2)
#pragma unroll
            for (int i = 0; i + w < 4 * BLK_WC; i += 2 * w) e[i] = fmaxf(e[i], e[i + w]);
          acc = e[0];
        } else {
          acc = tree_sum(e);
        }
        part[(slot * TR + wr0 + ir) * 64 + lane] = acc;
      }
    }
  } else {
    f32x4 acc[BLK_WC];
#pragma unroll
    for (int ic = 0; ic < BLK_WC; ++ic)
      acc[ic] = MAX ? f32x4{NEG_BIG, NEG_BIG, NEG_BIG, NEG_BIG} : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ir = 0; ir < BLK_WR; ++ir) {
      if (ir < wr) {
        const bf16x4 Bv = blk_row_operand(rowp, wr0 + ir, lane);
#pragma unroll
        for (int ic = 0; ic < BLK_WC; ++ic) {
          const f32x4 x = mfma_rank(A[ic], Bv, S[ir][ic]);
#pragma unroll
          for (int q = 0; q < 4; ++q) acc[ic][q] = MAX ? fmaxf(acc[ic][q], x[q]) : acc[ic][q] + fast_exp2(x[q]);
        }
      }
    }
    const int g = lane >> 4, i16 = lane & 15;
#pragma unroll
    for (int ic = 0; ic < BLK_WC; ++ic) {
      if (ic < wc) {
        float* p = part + ((size_t)((slot * TC + wc0 + ic) * 4 + g) * 4) * 16 + i16;
#pragma unroll
        for (int q = 0; q < 4; ++q) p[q * 16] = acc[ic][q];
      }
    }
  }
}

// Reduction of the wave partials of plan row q (local) of the block: over the sc column
// slots and the 4 lane groups.
template <bool MAX>
__device__ __forceinline__ float blk_row_reduce(const float* part, int q, int TR, int sc) {
  const int tile = q >> 4, i16 = q & 15;
  float r = MAX ? NEG_BIG : 0.f;
  for (int s = 0; s < sc; ++s) {
    const float* p = part + (s * TR + tile) * 64 + i16;
#pragma unroll
    for (int g = 0; g < 4; ++g) r = MAX ? fmaxf(r, p[16 * g]) : r + p[16 * g];
  }
  return r;
}
// Reduction for plan column jq (local) by the 4 threads 4 jq + quarter of a lane quad:
// each takes 4 of the 16 row lanes (one 16-byte read) over the sr row slots, then the
// quad combines (DPP).  Every lane of the wave must call it (live = false contributes
// nothing).
template <bool MAX>
__device__ __forceinline__ float blk_col_reduce(const float* part, int jq, int quarter, int TC, int sr, bool live) {
  float r = MAX ? NEG_BIG : 0.f;
  if (live) {
    const int tile = jq >> 4, j16 = jq & 15;  // j16 = 4 g + e
    for (int s = 0; s < sr; ++s) {
      const f32x4 v = *reinterpret_cast<const f32x4*>(part + ((size_t)(s * TC + tile) * 16 + j16) * 16 + 4 * quarter);
      r = MAX ? fmaxf(fmaxf(r, fmaxf(v[0], v[1])), fmaxf(v[2], v[3])) : r + ((v[0] + v[1]) + (v[2] + v[3]));
    }
  }
  const float a = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(r), 0xb1, 0xf, 0xf, false));
  r = MAX ? fmaxf(r, a) : r + a;
  const float b2 = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(r), 0x4e, 0xf, 0xf, false));
  return MAX ? fmaxf(r, b2) : r + b2;
}

// Polls the words base[k * stride], k < cnt <= W, until each carries `tag`; val[k]
// receives the float.  Two loads of each word in flight, checked alternately
// (poll_batch).  Returns false if the wait expires (then it raises the error).
template <int W>
__device__ __forceinline__ bool blk_poll(const uint64_t* base, size_t stride, int cnt, uint32_t tag, ErrRef err,
                                         float (&val)[W]) {
  if (cnt <= 0) return true;
  const uint32_t salt = tag >> 12;
  const uint64_t* addr[W];
  bool done[W];
#pragma unroll
  for (int k = 0; k < W; ++k) {
    done[k] = k >= cnt;
    addr[k] = base + (done[k] ? 0 : k * stride);
    val[k] = 0.f;
  }
  auto all = [&]() {
    bool r = true;
#pragma unroll
    for (int k = 0; k < W; ++k) r = r && done[k];
    return r;
  };
  auto ld = [&](int k) {
    return __hip_atomic_load(const_cast<uint64_t*>(addr[k]), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  };
  uint64_t wa[W], wb[W];
#pragma unroll
  for (int k = 0; k < W; ++k) wa[k] = ld(k);
  __builtin_amdgcn_s_sleep(1);
#pragma unroll
  for (int k = 0; k < W; ++k) wb[k] = ld(k);
  uint32_t spins = 0;
  while (true) {
#pragma unroll
    for (int k = 0; k < W; ++k)
      if (!done[k] && (uint32_t)wa[k] == tag) {
        val[k] = __uint_as_float((uint32_t)(wa[k] >> 32));
        done[k] = true;
      }
    if (all()) return true;
#pragma unroll
    for (int k = 0; k < W; ++k) wa[k] = ld(k);
    __builtin_amdgcn_s_sleep(1);
#pragma unroll
    for (int k = 0; k < W; ++k)
      if (!done[k] && (uint32_t)wb[k] == tag) {
        val[k] = __uint_as_float((uint32_t)(wb[k] >> 32));
        done[k] = true;
      }
    if (all()) return true;
#pragma unroll
    for (int k = 0; k < W; ++k) wb[k] = ld(k);
    __builtin_amdgcn_s_sleep(1);
    if (++spins > err.spin_limit / 2) {
      raise_error(err, salt, 2u);
      return false;
    }
  }
}

// log2 sum_k exp2(v_k), k < cnt (>= 1), in the order k = 0, 1, ...
template <int W>
__device__ __forceinline__ float blk_combine(const float (&v)[W], int cnt) {
  float m = v[0];
#pragma unroll
  for (int k = 1; k < W; ++k)
    if (k < cnt) m = fmaxf(m, v[k]);
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < W; ++k)
    if (k < cnt) s += fast_exp2(v[k] - m);
  return m + fast_log2(s);
}

template <typename T, int DP, bool HIST, bool GEN>
__global__ void __launch_bounds__(BLK_NT) sinkhorn_fwd_blk_kernel(SinkFwdArgs a) {
  using M = Mfma<T, DP>;
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ int s_flag, s_tmp, s_local;
  __shared__ unsigned s_du, s_dv;
  __shared__ float s_posw[BIN_NONE + 1];
  __shared__ int s_n[BLK_MAXS];
  __shared__ int s_G[BLK_MAXS];
  __shared__ int s_cost[BLK_MAXS * BLK_MAXL];

  const int t = threadIdx.x;
  const int lane = t & (WAVE - 1);
  const int L = (int)gridDim.x / 8;
  const int xcd = blockIdx.x & 7, l = blockIdx.x >> 3;
  const int BH = a.B * a.H;
  const int S = (BH - xcd + 7) / 8;  // groups xcd, xcd + 8, ... of this XCD
  if (t == 0) { s_flag = 0; s_du = 0u; s_dv = 0u; s_local = 1; }
  if (blockIdx.x == 0 && t == 0) __hip_atomic_store(a.err.ws + 1, a.salt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (S <= 0) return;
  const int N = a.N, d = a.d;
  const int Np = ((N + 31) / 32) * 32;

  // ---- members per group on this XCD, from the valid lengths of its groups
  for (int s = t; s < S; s += BLK_NT) s_n[s] = 0;
  __syncthreads();
  for (int s = 0; s < S; ++s) {
    const int bs = (xcd + 8 * s) / a.H;
    unsigned hi = 0;
    for (int i = t; i < N; i += BLK_NT)
      if (!a.mask || a.mask[(size_t)bs * N + i] > 0.5f) hi = i + 1;
    block_atomic_max_u32(reinterpret_cast<unsigned*>(&s_n[s]), hi);
  }
  __syncthreads();
  for (int e = t; e < S * L; e += BLK_NT) s_cost[e] = blk_grid(cdiv(s_n[e / L], 16), e % L + 1).pairs;
  __syncthreads();
  if (t == 0) blk_allocate(s_cost, S, L, s_G);
  __syncthreads();
  int my_s = -1, m = 0;
  {
    int off = 0;
    for (int s = 0; s < S; ++s) {
      if (l < off + s_G[s]) {
        my_s = s;
        m = l - off;
        break;
      }
      off += s_G[s];
    }
  }
  if (my_s < 0) return;  // surplus workgroup
  const int grp = xcd + 8 * my_s;
  const int b = grp / a.H, h = grp % a.H;
  const int G = s_G[my_s];
  const size_t bh = (size_t)b * a.H + h;

  unsigned char* valid = smem;
  float* vecU = reinterpret_cast<float*>(smem + ((Np + 15) / 16) * 16);
  float* vecV = vecU + Np;
  float* xs = vecV + Np;
  float* lse_r = xs + 3 * Np;
  float* mx2 = lse_r + Np;
  float* scratch = mx2 + Np;
  unsigned char* region = smem + blk_persist_lds(Np);  // iteration arrays, then Q and K
  T* QS = reinterpret_cast<T*>(region);
  T* KS = QS + (size_t)Np * DP;

  const int n = mask_setup(a.mask ? a.mask + (size_t)b * N : nullptr, N, valid, &s_tmp);
  const int n_tiles = (n + 15) / 16;
  // rows past the last valid tile belong to no block: zero their outputs
  for (int i = n_tiles * 16 + m; i < N; i += G) {
    for (int c = t; c < d; c += BLK_NT) {
      a.o_avg[(bh * N + i) * d + c] = 0.f;
      a.o_flat[((size_t)b * N + i) * (size_t)(a.H * d) + (size_t)h * d + c] = 0.f;
    }
    if (t < 3) a.x_centroid[(bh * N + i) * 3 + t] = 0.f;
    if (t == 0) a.log_u[bh * N + i] = a.log_v[bh * N + i] = a.log_z[bh * N + i] = a.col_lse[bh * N + i] = 0.f;
  }
  const BlkGrid gr = blk_grid(n_tiles, G);
  if (n > 0 && gr.pairs == BLK_NONE) {  // no grid fits (the host's check rules this out)
    if (t == 0) raise_error(a.err, a.salt, 3u);
    return;
  }
  if (n == 0 || m >= gr.R * gr.C) return;  // owns no block; no member waits on it
  const int R = gr.R, C = gr.C, sr = gr.sr, sc = gr.sc;
  const int r = m / C, c = m % C;
  const int rt0 = n_tiles * r / R, TR = n_tiles * (r + 1) / R - rt0;
  const int ct0 = n_tiles * c / C, TC = n_tiles * (c + 1) / C - ct0;

  // iteration arrays (their offsets follow blk_iter_lds)
  float* part_r = reinterpret_cast<float*>(region);
  float* part_c = part_r + (size_t)sc * TR * 64;
  bf16x4* rp_s = reinterpret_cast<bf16x4*>(part_c + (size_t)sr * TC * 256);  // -row shift
  bf16x4* rp_u = rp_s + TR * 16;                                             // u
  bf16x4* cp_v = rp_u + TR * 16;                                             // v
  bf16x4* cp_t = cp_v + TC * 16;                                             // -column shift
  float* u2 = reinterpret_cast<float*>(cp_t + TC * 16);
  float* sig = u2 + TR * 16;
  float* lmu = sig + TR * 16;
  float* v2 = lmu + TR * 16;
  float* tau = v2 + TC * 16;
  float* lnu = tau + TC * 16;

  const size_t qoff = (size_t)b * a.sb + (size_t)h * a.sh;
  const T* Qg = reinterpret_cast<const T*>(a.q) + qoff;
  const T* Kg = reinterpret_cast<const T*>(a.k) + qoff;
  const T* Vg = reinterpret_cast<const T*>(a.v) + qoff;
  const T* Gg = a.g ? reinterpret_cast<const T*>(a.g) + qoff : nullptr;
  const float eps = a.eps[h];
  const float kappa = a.lam / (a.lam + eps);
  const float sc_l = LOG2E / (sqrtf((float)d) * eps);
  const float w_h = a.w_dist ? a.w_dist[h] : 0.f;
  const bool use_geo = GEN && (a.x != nullptr) && (w_h != 0.f);
  const bool use_pos = GEN && (a.bins8 != nullptr) && (a.pos_w != nullptr);
  if (use_pos)
    for (int k = t; k <= (int)BIN_NONE; k += BLK_NT)
      s_posw[k] = k < (int)BIN_NONE ? -LOG2E * a.pos_w[h * 68 + k] / eps : 0.f;
  for (int e = t; e < 3 * Np; e += BLK_NT) xs[e] = (a.x && e < 3 * n) ? a.x[(size_t)b * N * 3 + e] : 0.f;
  for (int i = t; i < Np; i += BLK_NT) vecV[i] = NEG_BIG;
  for (int q = t; q < TR * 16; q += BLK_NT) {
    const int i = rt0 * 16 + q;
    const bool ok = i < n && valid[i];
    u2[q] = ok ? (a.u_init ? a.u_init[bh * N + i] * LOG2E : 0.f) : NEG_BIG;
    sig[q] = 0.f;
    lmu[q] = i < n ? a.log_mu[bh * N + i] : 0.f;
    rp_u[q] = split3(u2[q]);
    rp_s[q] = split3(0.f);
  }
  for (int q = t; q < TC * 16; q += BLK_NT) {
    const int j = ct0 * 16 + q;
    const bool ok = j < n && valid[j];
    v2[q] = ok ? (a.v_init ? a.v_init[bh * N + j] * LOG2E : 0.f) : NEG_BIG;
    tau[q] = 0.f;
    lnu[q] = j < n ? a.log_nu[bh * N + j] : 0.f;
    cp_v[q] = split3(v2[q]);
    cp_t[q] = split3(0.f);
  }
  __syncthreads();
  Bias bias;
  bias.b8 = use_pos ? a.bins8 + (size_t)b * Np * Np : nullptr;
  bias.b8t = use_pos ? a.bins8t + (size_t)b * Np * Np : nullptr;
  bias.posw = s_posw;
  bias.xs = use_geo ? xs : nullptr;
  bias.geo_scale = -LOG2E * w_h / eps;
  bias.r0 = a.r0;
  bias.Np = Np;
  const bool general = use_pos || use_geo;

  // ---- this wave's sub-block and its logits
  const int wave = __builtin_amdgcn_readfirstlane(t / WAVE);
  const int wi = wave / sc, wj = wave % sc;
  const int wr0 = TR * wi / sr, wr = TR * (wi + 1) / sr - wr0;
  const int wc0 = TC * wj / sc, wc = TC * (wj + 1) / sc - wc0;
  f32x4 Sl[BLK_WR][BLK_WC];  // columns past the wave's block: NEG_BIG (they add 0)
#pragma unroll
  for (int ir = 0; ir < BLK_WR; ++ir)
#pragma unroll
    for (int ic = 0; ic < BLK_WC; ++ic) Sl[ir][ic] = f32x4{NEG_BIG, NEG_BIG, NEG_BIG, NEG_BIG};
#pragma unroll
  for (int ir = 0; ir < BLK_WR; ++ir) {
    if (ir < wr) {
      const int irow = (rt0 + wr0 + ir) * 16 + (lane & 15);
      typename M::Frag qf;
      load_frag_global<T, DP>(qf, Qg, a.sn, irow, n, d, lane);
#pragma unroll
      for (int ic = 0; ic < BLK_WC; ++ic) {
        if (ic < wc) {
          const int jt = ct0 + wc0 + ic;
          typename M::Frag kf;
          load_frag_global<T, DP>(kf, Kg, a.sn, jt * 16 + (lane & 15), n, d, lane);
          const f32x4 acc = M::qk(kf, qf, f32x4{0.f, 0.f, 0.f, 0.f});
          f32x4 bv = {0.f, 0.f, 0.f, 0.f};
          if (general) {
            f32x4 o[1];
            const int s0[1] = {jt * 16 + 4 * (lane >> 4)};
            bias.template quads<false, 1>(irow, s0, o);
            bv = o[0];
          }
#pragma unroll
          for (int q = 0; q < 4; ++q) Sl[ir][ic][q] = general ? __builtin_fmaf(acc[q], sc_l, bv[q]) : acc[q] * sc_l;
        }
      }
    }
  }

  // ---- exchange words of this (b,h)
  uint64_t* xbase = a.xch + bh * (size_t)BLK_XCH_VECS * Np;
  // Row partials [2][C][Np] and column partials [2][R][Np], slot it & 1: a member can
  // write iteration it + 2's partials only after every member of its row (column) band
  // has published iteration it + 1's, which each does after reading iteration it's, so
  // no word is overwritten before all its readers have it.
  uint64_t* xrow = xbase;
  uint64_t* xcol = xbase + (size_t)2 * BLK_MAXRC * Np;
  uint64_t* xfin = xbase + (size_t)4 * BLK_MAXRC * Np;  // final v
  uint64_t* xpl = a.xch + (size_t)BH * BLK_XCH_VECS * Np + bh * BLK_MAXL;
  const uint32_t salt = a.salt << 12;
  uint32_t phase = 0;
  bool local = false;
  if (t == 0) xch_put(xpl + m, xcc_placed() ? 1.f : 0.f, salt);
  auto agree_placement = [&]() __attribute__((always_inline)) -> bool {
    if (phase != 1) return true;
    if (t < R * C) {
      uint32_t spins = 0;
      while (true) {
        const uint64_t w = __hip_atomic_load(xpl + t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if ((uint32_t)w == salt) {
          if (__uint_as_float((uint32_t)(w >> 32)) != 1.f) s_local = 0;
          break;
        }
        __builtin_amdgcn_s_sleep(1);
        if (++spins > a.err.spin_limit) { raise_error(a.err, a.salt, 2u); s_flag = 1; break; }
      }
    }
    __syncthreads();
    local = s_local != 0;
    return s_flag == 0;
  };

  // ---- row update: u_i = kappa (log mu_i - LSE_j(L_ij + v_j)), i in I_r
  auto row_update = [&](int it) __attribute__((always_inline)) -> bool {
    const uint32_t tag = salt | ++phase;
    const bool online = it == 0 || __uint_as_float(s_dv) > FIXED_SHIFT_MAX_DELTA;
    if (t == 0) s_du = 0u;
    bf16x4 A[BLK_WC];
#pragma unroll
    for (int ic = 0; ic < BLK_WC; ++ic) A[ic] = blk_col_operand(cp_v, min(wc0 + ic, TC - 1), lane);
    if (online) {
      blk_sweep<true, true>(Sl, A, wr, wc, wr0, wc0, wj, TR, TC, rp_s, part_r, lane);
      __syncthreads();
      for (int q = t; q < TR * 16; q += BLK_NT) {
        const float mq = blk_row_reduce<true>(part_r, q, TR, sc);
        sig[q] += mq > 0.5f * NEG_BIG ? mq : 0.f;  // no live column in J_c: keep the shift
        rp_s[q] = split3(-sig[q]);
      }
      __syncthreads();
    }
    blk_sweep<true, false>(Sl, A, wr, wc, wr0, wc0, wj, TR, TC, rp_s, part_r, lane);
    __syncthreads();
    float dmax = 0.f;
    for (int q = t; q < TR * 16; q += BLK_NT) {
      const int i = rt0 * 16 + q;
      const bool ok = i < n && valid[i];
      float lse = 0.f;
      if (ok) {
        const float part = sig[q] + fast_log2(blk_row_reduce<false>(part_r, q, TR, sc));
        uint64_t* xr = xrow + (size_t)(it & 1) * BLK_MAXRC * Np;
        xch_put(xr + (size_t)c * Np + i, part, tag, local);
        float val[BLK_MAXRC];
        if (!blk_poll<BLK_MAXRC>(xr + i, Np, C, tag, a.err, val)) s_flag = 1;
        lse = blk_combine<BLK_MAXRC>(val, C);
        const float u = kappa * (lmu[q] - lse * LN2);
        const float un = u * LOG2E;
        dmax = fmaxf(dmax, fabsf(un - u2[q]));
        u2[q] = un;
        if constexpr (HIST)
          if (c == 0) a.hist[((size_t)(2 * it + 1) * BH + bh) * N + i] = u;
      } else {
        u2[q] = NEG_BIG;
        if constexpr (HIST)
          if (c == 0 && i < n) a.hist[((size_t)(2 * it + 1) * BH + bh) * N + i] = 0.f;
      }
      sig[q] = lse;
      rp_s[q] = split3(-lse);
      rp_u[q] = split3(u2[q]);
    }
    block_atomic_max_u32(&s_du, dmax == dmax ? __float_as_uint(dmax) : 0x7f800000u);
    __syncthreads();
    if (s_flag) return false;
    return agree_placement();
  };

  // ---- column update: v_j = kappa (log nu_j - LSE_i(L_ij + u_i)), j in J_c
  auto col_update = [&](int it) __attribute__((always_inline)) -> bool {
    const uint32_t tag = salt | ++phase;
    const bool online = it == 0 || __uint_as_float(s_du) > FIXED_SHIFT_MAX_DELTA;
    const bool last = it == a.K_iter - 1;
    if (t == 0) s_dv = 0u;
    const int ncol = TC * 16;
    if (online) {
      bf16x4 A[BLK_WC];
#pragma unroll
      for (int ic = 0; ic < BLK_WC; ++ic) A[ic] = blk_col_operand(cp_t, min(wc0 + ic, TC - 1), lane);
      blk_sweep<false, true>(Sl, A, wr, wc, wr0, wc0, wi, TR, TC, rp_u, part_c, lane);
      __syncthreads();
      for (int q0 = 0; q0 < ncol; q0 += BLK_NT / 4) {
        const int q = q0 + t / 4;
        const float mq = blk_col_reduce<true>(part_c, q, t & 3, TC, sr, q < ncol);
        if (q < ncol && (t & 3) == 0) {
          tau[q] += mq > 0.5f * NEG_BIG ? mq : 0.f;
          cp_t[q] = split3(-tau[q]);
        }
      }
      __syncthreads();
    }
    {
      bf16x4 A[BLK_WC];
#pragma unroll
      for (int ic = 0; ic < BLK_WC; ++ic) A[ic] = blk_col_operand(cp_t, min(wc0 + ic, TC - 1), lane);
      blk_sweep<false, false>(Sl, A, wr, wc, wr0, wc0, wi, TR, TC, rp_u, part_c, lane);
    }
    __syncthreads();
    float dmax = 0.f;
    for (int q0 = 0; q0 < ncol; q0 += BLK_NT / 4) {
      const int q = q0 + t / 4;
      const float s = blk_col_reduce<false>(part_c, q, t & 3, TC, sr, q < ncol);
      if (q < ncol && (t & 3) == 0) {
        const int j = ct0 * 16 + q;
        const bool ok = j < n && valid[j];
        float lse = 0.f;
        if (ok) {
          uint64_t* xc = xcol + (size_t)(it & 1) * BLK_MAXRC * Np;
          xch_put(xc + (size_t)r * Np + j, tau[q] + fast_log2(s), tag, local);
          float val[BLK_MAXRC];
          if (!blk_poll<BLK_MAXRC>(xc + j, Np, R, tag, a.err, val)) s_flag = 1;
          lse = blk_combine<BLK_MAXRC>(val, R);
          const float v = kappa * (lnu[q] - lse * LN2);
          const float vn = v * LOG2E;
          dmax = fmaxf(dmax, fabsf(vn - v2[q]));
          v2[q] = vn;
          if (r == 0) {
            if (last) a.col_lse[bh * N + j] = lse * LN2;
            if constexpr (HIST) a.hist[((size_t)(2 * it) * BH + bh) * N + j] = v;
          }
        } else {
          v2[q] = NEG_BIG;
          if constexpr (HIST)
            if (r == 0 && j < n) a.hist[((size_t)(2 * it) * BH + bh) * N + j] = 0.f;
        }
        tau[q] = lse;
        cp_t[q] = split3(-lse);
        cp_v[q] = split3(v2[q]);
      }
    }
    block_atomic_max_u32(&s_dv, dmax == dmax ? __float_as_uint(dmax) : 0x7f800000u);
    __syncthreads();
    if (s_flag) return false;
    return agree_placement();
  };

  for (int it = 0; it < a.K_iter; ++it)
    if (!row_update(it) || !col_update(it)) return;

  // ---- final v to every member: row block 0 publishes its columns
  {
    const uint32_t tag = salt | ++phase;
    if (r == 0)
      for (int q = t; q < TC * 16; q += BLK_NT) {
        const int j = ct0 * 16 + q;
        if (j < n) xch_put(xfin + j, valid[j] ? v2[q] * LN2 : 0.f, tag, local);
      }
    // the tail's rows (a share of I_r) keep their u
    const int tt0 = rt0 + TR * c / C, tt1 = rt0 + TR * (c + 1) / C;
    for (int i = tt0 * 16 + t; i < tt1 * 16; i += BLK_NT) vecU[i] = u2[i - rt0 * 16];
    if (t == 0) s_dv = 0u;
    __syncthreads();
    if (!gather_potential<BLK_NT>(xfin, n, tag, vecV, valid, a.err, &s_flag, &s_dv)) return;
    const int nr_tail = tt1 - tt0;
    if (nr_tail <= 0) return;
    // the iteration arrays are dead: Q and K take the region (resident layout)
    stage_rows<T, DP>(QS, Qg, a.sn, n, d, Np);
    stage_rows<T, DP>(KS, Kg, a.sn, n, d, Np);
    __syncthreads();
    // final row LSE with the last v: exact log Z and the row maxima
    fwd_sweep<T, DP, GEN, false>(true, QS, KS, vecV, n_tiles, tt0, nr_tail, sc_l, bias, lse_r, mx2, scratch,
                                 nullptr, NoPublish());
    fwd_resident_output<T, DP>(a, b, h, n, n_tiles, Np, tt0, nr_tail, valid, QS, KS, vecU, vecV, xs, lse_r, mx2,
                               sc_l, bias, general, false, true, Qg, Vg, Gg);
  }
}

}  // namespace dfl
