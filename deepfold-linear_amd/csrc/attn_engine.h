// Streaming engine of the softmax-attention kernels (gfx950).
//
// A workgroup owns RQ resident rows (queries in the forward and dQ passes, keys in
// the dK/dV pass) as RT = RQ/16 MFMA tiles whose fragments stay in registers.
// The other operand streams through LDS in chunks of CH rows.  Each resident tile
// has KS = 2 waves that take alternate 32-row steps of every chunk (two waves per
// SIMD); their partial results merge through LDS at the end.
//
// Staging is software-pipelined: the 16-byte global loads of chunk c+1 are
// issued right after the barrier that publishes chunk c, so they complete while
// chunk c is computed; LDS is double-buffered, one barrier per chunk.
//
// Streamed rows enter the MFMAs in a permuted order: of a 32-row step, tile 0
// takes rows {8a + r} and tile 1 rows {8a + 4 + r} (a, r < 4).  The accumulator
// of a 16x16 tile gives lane group g rows 4g..4g+3, so after the permutation a
// lane holds 8 consecutive streamed rows 8g..8g+7 of its resident column.  That
// is exactly the k-slice a lane feeds to a 16x16x32 MFMA, so P and dS go into
// the PV-type products without any lane exchange, and the per-(row, column) bias
// of a lane is one contiguous 16-byte read.
#pragma once
#include "attn_args.h"
#include "common.h"

#include <type_traits>

namespace dfl {

template <typename T, int DP, bool WIN>
struct Eng {
  static constexpr int VEC = 16 / (int)sizeof(T);   // elements per 16-byte block
  static constexpr int RB = DP * (int)sizeof(T);    // bytes of one padded row
  static constexpr int RQ = WIN ? 32 : 64;           // resident rows per workgroup
  static constexpr int RT = RQ / 16;
  static constexpr int KS = 2;                       // waves per resident tile
  static constexpr int NW = RT * KS;
  static constexpr int NT = NW * WAVE;
  static constexpr int CH0 = RB <= 64 ? 256 : (RB <= 128 ? 128 : 64);
  static constexpr int CH = (WIN && CH0 > 128) ? 128 : CH0;  // streamed rows per chunk
  static constexpr int SPC = CH / 32;                // 32-row steps per chunk
  static constexpr int SPW = SPC / KS;               // steps per wave per chunk
  static constexpr int CB = DP / VEC;                // 16-byte blocks per row
  static constexpr int RS = DP + VEC;                // row stride of row-major LDS copies
  static constexpr int TS = CH + VEC;                // row stride of transposed LDS copies
  static constexpr int LD = CH * CB / NT;            // row blocks per thread per chunk and operand
  static_assert(SPW >= 1 && CH * CB % NT == 0 && LD >= 1, "engine geometry");
};

constexpr int lds_align(int x) { return (x + 15) / 16 * 16; }

__device__ __forceinline__ bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// 16-byte block [col, col + VEC) of row `row` of a row-strided operand; zero for
// rows >= nrows and columns >= d.  vec: base and row stride are 16-byte aligned.
template <typename T>
__device__ __forceinline__ uint4 ld_block(const T* __restrict__ base, long long sn, int row, int nrows, int col, int d,
                                          bool vec) {
  constexpr int VEC = 16 / (int)sizeof(T);
  union { uint4 u; T e[VEC]; } r;
  r.u = make_uint4(0u, 0u, 0u, 0u);
  if (row < nrows && col < d) {
    const T* p = base + (size_t)row * sn + col;
    if (vec && col + VEC <= d) {
      r.u = *reinterpret_cast<const uint4*>(p);
    } else {
#pragma unroll
      for (int e = 0; e < VEC; ++e)
        if (col + e < d) r.e[e] = p[e];
    }
  }
  return r.u;
}

// Element e of a 16-byte block, as float.
template <typename T> __device__ __forceinline__ float blk_elem(const uint4& u, int e);
template <> __device__ __forceinline__ float blk_elem<bf16>(const uint4& u, int e) {
  const unsigned w = e < 2 ? u.x : e < 4 ? u.y : e < 6 ? u.z : u.w;
  return __uint_as_float((e & 1) ? (w & 0xffff0000u) : (w << 16));
}
template <> __device__ __forceinline__ float blk_elem<float>(const uint4& u, int e) {
  return __uint_as_float(e == 0 ? u.x : e == 1 ? u.y : e == 2 ? u.z : u.w);
}

// Write the VEC elements of block u as column `row` of a transposed LDS array:
// dst[(col + e) * ts + row].
template <typename T>
__device__ __forceinline__ void st_transposed(T* dst, int ts, int row, int col, const uint4& u) {
  constexpr int VEC = 16 / (int)sizeof(T);
  union { uint4 u; T e[VEC]; } r;
  r.u = u;
#pragma unroll
  for (int e = 0; e < VEC; ++e) dst[(size_t)(col + e) * ts + row] = r.e[e];
}

// Local row of the permuted 32-row step that lane l feeds as MFMA row (l % 16) of tile hf.
__device__ __forceinline__ int perm_row(int lane, int hf) {
  return 8 * ((lane & 15) >> 2) + 4 * hf + (lane & 3);
}

// O^T[c][i] += sum_j VT[c][j] P[j][i] over the lane's 8 streamed rows j = 8g..8g+7.
// vt: LDS address of VT[c0 + l%16][j0 + 8g]; p: the lane's 8 values in row order.
template <typename T> struct PV8;
template <> struct PV8<bf16> {
  __device__ static __forceinline__ f32x4 mma(const bf16* vt, const float (&p)[8], f32x4 acc) {
    bf16x8 b;
#pragma unroll
    for (int e = 0; e < 8; ++e) b[e] = (bf16)p[e];
    const bf16x8 av = *reinterpret_cast<const bf16x8*>(vt);
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, b, acc, 0, 0, 0);
  }
};
template <> struct PV8<float> {
  __device__ static __forceinline__ f32x4 mma(const float* vt, const float (&p)[8], f32x4 acc) {
    const f32x4 lo = *reinterpret_cast<const f32x4*>(vt);
    const f32x4 hi = *reinterpret_cast<const f32x4*>(vt + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(lo[e], p[e], acc, 0, 0, 0);
#pragma unroll
    for (int e = 0; e < 4; ++e) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(hi[e], p[4 + e], acc, 0, 0, 0);
    return acc;
  }
};

// One thread's share of a streamed operand chunk in flight: LD row blocks of 16
// bytes.  Loads are unconditional, from clamped addresses, so no loaded register
// is ever merged with another definition at a branch join (that would force the
// wait right at the load); validity is applied when the block is written to LDS.
//   FAST (16-byte aligned rows, d a multiple of VEC): one 16-byte load per block.
//   otherwise: one clamped element load per element.
template <typename T, int LD, bool FAST> struct Flight;
template <typename T, int LD> struct Flight<T, LD, true> {
  uint4 r[LD];
  unsigned ok;
  __device__ __forceinline__ void load(int u, const T* __restrict__ base, long long sn, int row, int nrows, int col,
                                       int d) {
    if (u == 0) ok = 0u;
    ok |= (row < nrows && col < d) ? (1u << u) : 0u;
    r[u] = *reinterpret_cast<const uint4*>(base + (size_t)min(row, nrows - 1) * sn + (col < d ? col : 0));
  }
  __device__ __forceinline__ uint4 get(int u) const {
    const bool v = (ok >> u) & 1u;
    return make_uint4(v ? r[u].x : 0u, v ? r[u].y : 0u, v ? r[u].z : 0u, v ? r[u].w : 0u);
  }
};
template <typename T, int LD> struct Flight<T, LD, false> {
  static constexpr int VEC = 16 / (int)sizeof(T);
  T e[LD][VEC];
  unsigned ok[LD];
  __device__ __forceinline__ void load(int u, const T* __restrict__ base, long long sn, int row, int nrows, int col,
                                       int d) {
    unsigned m = 0u;
    const T* p = base + (size_t)min(row, nrows - 1) * sn;
#pragma unroll
    for (int k = 0; k < VEC; ++k) {
      m |= (row < nrows && col + k < d) ? (1u << k) : 0u;
      e[u][k] = p[min(col + k, d - 1)];
    }
    ok[u] = m;
  }
  __device__ __forceinline__ uint4 get(int u) const {
    union { uint4 u4; T v[VEC]; } r;
#pragma unroll
    for (int k = 0; k < VEC; ++k) r.v[k] = ((ok[u] >> k) & 1u) ? e[u][k] : from_f32<T>(0.f);
    return r.u4;
  }
};

// Per-(query, key) bias of one lane's query row, in log2 units.
//   DENSE / WINDOW: element type T, LOG2E * bias;  BINS: int32 bin -> pw2[bin] (pre-scaled).
// row: element of key 0 of the lane's (clamped) query row; keys start at the
// window offset for WINDOW.  FAST loads take 8 consecutive keys as 16-byte blocks
// from a start clamped to [.., k_hi - 8]: keys past k_hi read another key's value,
// which the -1e30 key mask of those keys swamps.
template <typename T, int BIAS>
struct BiasRow {
  using BT = typename std::conditional<BIAS == ATTN_BIAS_BINS, int, T>::type;
  static constexpr int BW = BIAS == ATTN_BIAS_NONE ? 1 : (8 * (int)sizeof(BT)) / 16;  // blocks per 8 keys
  const BT* row;
  __device__ __forceinline__ void load8(uint4 (&r)[BW], int key0, int k_hi) const {
    const int kc = min(key0, k_hi - 8);
#pragma unroll
    for (int w = 0; w < BW; ++w) r[w] = *reinterpret_cast<const uint4*>(row + kc + w * (16 / (int)sizeof(BT)));
  }
  __device__ __forceinline__ float elem(int key, int k_hi, const float* pw2) const {
    const BT v = row[min(key, k_hi - 1)];
    if constexpr (BIAS == ATTN_BIAS_BINS) {
      const unsigned k = (unsigned)v;
      return k < 68u ? pw2[k] : 0.f;
    } else {
      return LOG2E * to_f32(v);
    }
  }
};

template <typename T, int BIAS>
__device__ __forceinline__ float bias_value(const uint4* r, int e, const float* pw2) {
  if (BIAS == ATTN_BIAS_BINS) {
    const uint4 u = r[e >> 2];
    const unsigned k = (e & 3) == 0 ? u.x : (e & 3) == 1 ? u.y : (e & 3) == 2 ? u.z : u.w;
    return k < 68u ? pw2[k] : 0.f;  // bins outside [0, 68) carry no bias
  }
  if (sizeof(T) == 2) return LOG2E * blk_elem<bf16>(r[0], e);
  return LOG2E * blk_elem<float>(r[e >> 2], e & 3);
}

// Workgroup -> (block, unit).  A unit is a set of nblk workgroups that stream the
// same operand (one (b,h), or one (b,h) and query split in the dK/dV pass); units
// are numbered 0 .. U-1.  Hardware dispatches workgroups round-robin over the 8 XCDs
// (workgroup id % 8), each with its own L2, so the mapping keeps a unit's streamed
// operand inside as few L2s as it can:
//   U % 8 == 0:                 every unit on one XCD;
//   8 % U == 0, nblk U % 8 == 0: a unit on 8 / U XCDs, each taking a contiguous
//                               range of its blocks (windows that overlap stay on
//                               one XCD except at the range ends);
//   otherwise:                  unit-major order.
__device__ __forceinline__ void block_coords(int nblk, int U, int& blk, int& unit) {
  const int L = blockIdx.x, x = L & 7, s = L >> 3;
  if ((U & 7) == 0) {
    unit = x + 8 * (s / nblk);
    blk = s % nblk;
  } else if (8 % U == 0 && (nblk * U) % 8 == 0) {
    const int per = nblk * U / 8;
    unit = x % U;
    blk = (x / U) * per + s;
  } else {
    unit = L / nblk;
    blk = L % nblk;
  }
}

// Key range [lo, hi) of the query tile starting at q (windowed: its window).
__device__ __forceinline__ void window_keys2(int q, int Nk, int& lo, int& hi) {
  const int w = q / ATTN_WQ;
  lo = max(0, ATTN_WQ * w - ATTN_WOFF);
  hi = min(Nk, ATTN_WQ * w + ATTN_WQ + ATTN_WOFF);
}

// Query range [lo, hi) of the windows that contain any key of [k0, k1):
// key j is in window w  <=>  32w - 48 <= j < 32w + 80  <=>  floor((j - 80)/32) < w <= floor((j + 48)/32).
__device__ __forceinline__ int floordiv(int x, int y) { return x >= 0 ? x / y : -((-x + y - 1) / y); }
__device__ __forceinline__ void window_queries(int k0, int k1, int Mq, int& lo, int& hi) {
  const int wlo = max(0, floordiv(k0 - (ATTN_WQ + ATTN_WOFF), ATTN_WQ) + 1);
  const int whi = floordiv(k1 - 1 + ATTN_WOFF, ATTN_WQ);
  lo = min(Mq, ATTN_WQ * wlo);
  hi = min(Mq, ATTN_WQ * (whi + 1));
}

constexpr float POS_BIG = 1.0e30f;  // LSE of a masked query: every P becomes exp2(-huge) = 0
constexpr float LAZY_THR = 8.f;     // log2 units a score may exceed the running max before a rescale
constexpr float M_INIT = -1.0e29f;  // running max before any valid key (masked logits are -1e30)

// ===========================================================================
// Forward: O = softmax(scale Q K^T + bias) V, lse, optional gate.
template <typename T, int DP, bool WIN>
constexpr int attn_fwd_lds() {
  using E = Eng<T, DP, WIN>;
  return 2 * lds_align(E::CH * E::RS * (int)sizeof(T) + DP * E::TS * (int)sizeof(T) + E::CH * 4) + 68 * 4;
}
// LDS of the gate rows a gated forward parks after attn_fwd_lds (launched only with a gate,
// so that ungated launches keep their occupancy)
template <typename T, int DP, bool WIN>
constexpr int attn_fwd_gate_lds() {
  return Eng<T, DP, WIN>::RQ * DP * (int)sizeof(T);
}

template <typename T, int DP, int BIAS, bool WIN, bool FAST>
__global__ void __launch_bounds__((Eng<T, DP, WIN>::NT)) attn_fwd2_kernel(AttnArgs a) {
  using E = Eng<T, DP, WIN>;
  using M = Mfma<T, DP>;
  using BR = BiasRow<T, BIAS>;
  constexpr int NT = E::NT, CH = E::CH, RS = E::RS, TS = E::TS, VEC = E::VEC, CB = E::CB, LD = E::LD;
  constexpr int SPW = E::SPW, KS = E::KS, RT = E::RT;
  constexpr int NC = DP / 16;
  constexpr int BW = BR::BW;
  constexpr bool HASB = BIAS != ATTN_BIAS_NONE;
  constexpr int KOFF = 0, VOFF = CH * RS * (int)sizeof(T), BOFF = VOFF + DP * TS * (int)sizeof(T);
  constexpr int BUF = lds_align(BOFF + CH * 4);
  extern __shared__ __align__(16) unsigned char smem[];
  float* s_pw = reinterpret_cast<float*>(smem + 2 * BUF);
  T* s_g = reinterpret_cast<T*>(smem + 2 * BUF + 68 * 4);  // [RQ][DP] gate rows (gated launches only)

  const int t = threadIdx.x, lane = t & (WAVE - 1), wave = t / WAVE, g = lane >> 4;
  const int rt = wave % RT, ks = wave / RT;
  const int BH = a.B * a.H, Mq = a.Mq, Nk = a.Nk, d = a.d;
  const int nqb = (Mq + E::RQ - 1) / E::RQ;
  int qb, bh;
  block_coords(nqb, BH, qb, bh);
  const int b = bh / a.H, h = bh % a.H;
  const int q0 = qb * E::RQ;
  const int qt = q0 + 16 * rt;
  const int qi = qt + (lane & 15);
  const int qc = min(qi, Mq - 1);
  const bool active = qt < Mq, qrow = qi < Mq;
  const T* Qg = reinterpret_cast<const T*>(a.q) + (size_t)b * a.qsb + (size_t)h * a.qsh;
  const T* Kg = reinterpret_cast<const T*>(a.k) + (size_t)b * a.ksb + (size_t)h * a.ksh;
  const T* Vg = reinterpret_cast<const T*>(a.v) + (size_t)b * a.ksb + (size_t)h * a.ksh;
  const float* kmask = a.kmask ? a.kmask + (size_t)b * Nk : nullptr;
  const float sc = a.scale * LOG2E;
  int k_lo = 0, k_hi = Nk;
  if (WIN) window_keys2(q0, Nk, k_lo, k_hi);

  // The gate rows of the workgroup (gated launches) are loaded now, from clamped
  // addresses, and parked in LDS once chunk 0's prefetch is in flight, so the
  // epilogue reads them without a global round trip.
  constexpr int GPT = E::RQ * DP / NT;  // gate elements per thread
  static_assert(E::RQ * DP % NT == 0, "gate staging geometry");
  const bool hasg = a.g != nullptr;
  T gpre[GPT];
  if (hasg) {
    const T* Gb = reinterpret_cast<const T*>(a.g) + (size_t)b * a.qsb + (size_t)h * a.qsh;
#pragma unroll
    for (int u = 0; u < GPT; ++u) {
      const int e = t + NT * u;
      gpre[u] = Gb[(size_t)min(q0 + e / DP, Mq - 1) * a.qsn + min(e % DP, d - 1)];
    }
  }

  if (BIAS == ATTN_BIAS_BINS)
    for (int k = t; k < 68; k += NT) s_pw[k] = LOG2E * a.pos_w[h * 68 + k];
  BR br;
  br.row = nullptr;
  if (BIAS == ATTN_BIAS_DENSE) {
    br.row = reinterpret_cast<const typename BR::BT*>(reinterpret_cast<const T*>(a.bias) +
                                                       ((size_t)bh * Mq + qc) * Nk);
  } else if (BIAS == ATTN_BIAS_WINDOW) {
    const int w = q0 / ATTN_WQ;
    const T* row = reinterpret_cast<const T*>(a.bias) + (((size_t)w * a.H + h) * ATTN_WQ + (qc - ATTN_WQ * w)) * ATTN_WK;
    br.row = reinterpret_cast<const typename BR::BT*>(row - (ATTN_WQ * w - ATTN_WOFF));  // indexed by key
  } else if (BIAS == ATTN_BIAS_BINS) {
    br.row = reinterpret_cast<const typename BR::BT*>(a.bins + ((size_t)b * Mq + qc) * Nk);
  }

  typename M::Frag qf;
  {
    constexpr int RUN = M::RUN;
    T tmp[RUN];
    const int c0 = g * RUN;
    if constexpr (FAST) {
      // 16-byte blocks from a clamped row and block start; validity applied after
      static_assert(RUN % VEC == 0, "whole 16-byte blocks per lane");
#pragma unroll
      for (int k = 0; k < RUN / VEC; ++k)
        *reinterpret_cast<uint4*>(tmp + VEC * k) =
            *reinterpret_cast<const uint4*>(Qg + (size_t)qc * a.qsn + min(c0 + VEC * k, d - VEC));
#pragma unroll
      for (int e = 0; e < RUN; ++e) tmp[e] = (qrow && c0 + e < d) ? tmp[e] : from_f32<T>(0.f);
    } else {
#pragma unroll
      for (int e = 0; e < RUN; ++e)
        tmp[e] = (qrow && c0 + e < d) ? Qg[(size_t)qi * a.qsn + c0 + e] : from_f32<T>(0.f);
    }
    M::from_run(qf, tmp);
  }

  // chunk data in flight
  Flight<T, LD, FAST> kfl, vfl;
  float kmraw;
  uint4 bcur[SPW][BW], bnxt[SPW][BW];
  auto prefetch = [&](int c0) {
#pragma unroll
    for (int u = 0; u < LD; ++u) {
      const int idx = t + NT * u;
      kfl.load(u, Kg, a.ksn, c0 + idx / CB, k_hi, (idx % CB) * VEC, d);
      vfl.load(u, Vg, a.ksn, c0 + idx % CH, k_hi, (idx / CH) * VEC, d);
    }
    if (kmask) kmraw = kmask[min(c0 + t % CH, k_hi - 1)];
    if (HASB && FAST) {
#pragma unroll
      for (int j = 0; j < SPW; ++j) br.load8(bnxt[j], c0 + 32 * (ks + KS * j) + 8 * g, k_hi);
    }
  };

  float m = M_INIT, lsum = 0.f;
  f32x4 oacc[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) oacc[c] = f32x4{0.f, 0.f, 0.f, 0.f};
  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};

  prefetch(k_lo);
  if (hasg) {
#pragma unroll
    for (int u = 0; u < GPT; ++u) s_g[t + NT * u] = gpre[u];
  }
  int buf = 0;
  for (int c0 = k_lo; c0 < k_hi; c0 += CH, buf ^= 1) {
    unsigned char* base = smem + buf * BUF;
    T* Ks = reinterpret_cast<T*>(base + KOFF);
    T* VTs = reinterpret_cast<T*>(base + VOFF);
    float* kb = reinterpret_cast<float*>(base + BOFF);
#pragma unroll
    for (int u = 0; u < LD; ++u) {
      const int idx = t + NT * u;
      *reinterpret_cast<uint4*>(Ks + (size_t)(idx / CB) * RS + (idx % CB) * VEC) = kfl.get(u);
      st_transposed<T>(VTs, TS, idx % CH, (idx / CH) * VEC, vfl.get(u));
    }
    if (t < CH) kb[t] = (c0 + t < k_hi && (!kmask || kmraw > 0.5f)) ? 0.f : NEG_BIG;
    if (HASB && FAST) {
#pragma unroll
      for (int j = 0; j < SPW; ++j)
#pragma unroll
        for (int w = 0; w < BW; ++w) bcur[j][w] = bnxt[j][w];
    }
    __syncthreads();
    if (c0 + CH < k_hi) prefetch(c0 + CH);
    if (!active) continue;
#pragma unroll
    for (int j = 0; j < SPW; ++j) {
      const int kl = 32 * (ks + KS * j);  // local row of this step
      if (c0 + kl >= k_hi) break;
      typename M::Frag kf0, kf1;
      const int pr = kl + perm_row(lane, 0);
      M::load(kf0, Ks + (size_t)pr * RS, lane);
      M::load(kf1, Ks + (size_t)(pr + 4) * RS, lane);
      const f32x4 s0 = M::qk(kf0, qf, zero);
      const f32x4 s1 = M::qk(kf1, qf, zero);
      const f32x4 kb0 = *reinterpret_cast<const f32x4*>(kb + kl + 8 * g);
      const f32x4 kb1 = *reinterpret_cast<const f32x4*>(kb + kl + 8 * g + 4);
      float x[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float b0 = kb0[e], b1 = kb1[e];
        if (HASB) {
          if (FAST) {
            b0 += bias_value<T, BIAS>(bcur[j], e, s_pw);
            b1 += bias_value<T, BIAS>(bcur[j], 4 + e, s_pw);
          } else {
            const int key = c0 + kl + 8 * g + e;
            b0 += br.elem(key, k_hi, s_pw);
            b1 += br.elem(key + 4, k_hi, s_pw);
          }
        }
        x[e] = __builtin_fmaf(s0[e], sc, b0);
        x[4 + e] = __builtin_fmaf(s1[e], sc, b1);
      }
      float lm = fmaxf(fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3])), fmaxf(fmaxf(x[4], x[5]), fmaxf(x[6], x[7])));
      if (__builtin_amdgcn_ballot_w64(lm > m + LAZY_THR) != 0ull) {  // wave-uniform
        const float mn = fmaxf(m, max_groups(lm));
        const float alpha = fast_exp2(m - mn);
        lsum *= alpha;
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
          for (int r = 0; r < 4; ++r) oacc[c][r] *= alpha;
        m = mn;
      }
      float p[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        p[e] = fast_exp2(x[e] - m);
        lsum += p[e];
      }
#pragma unroll
      for (int c = 0; c < NC; ++c)
        oacc[c] = PV8<T>::mma(VTs + (size_t)(c * 16 + (lane & 15)) * TS + kl + 8 * g, p, oacc[c]);
    }
  }

  // merge the KS partials of each resident tile (waves ks > 0 hand theirs to ks = 0)
  __syncthreads();
  float* mg = reinterpret_cast<float*>(smem);
  constexpr int MGS = 2 + 4 * NC;  // floats per lane
  if (ks > 0 && active) {
    float* dst = mg + ((size_t)((ks - 1) * RT + rt) * WAVE + lane) * MGS;
    dst[0] = m;
    dst[1] = lsum;
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int r = 0; r < 4; ++r) dst[2 + 4 * c + r] = oacc[c][r];
  }
  __syncthreads();
  if (ks > 0 || !active) return;
#pragma unroll
  for (int s = 1; s < KS; ++s) {
    const float* src = mg + ((size_t)((s - 1) * RT + rt) * WAVE + lane) * MGS;
    const float m1 = src[0];
    const float mn = fmaxf(m, m1);
    const float a0 = fast_exp2(m - mn), a1 = fast_exp2(m1 - mn);
    lsum = lsum * a0 + src[1] * a1;
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int r = 0; r < 4; ++r) oacc[c][r] = oacc[c][r] * a0 + src[2 + 4 * c + r] * a1;
    m = mn;
  }
  lsum = sum_groups(lsum);
  const bool qok = qrow && (!a.qmask || a.qmask[(size_t)b * Mq + qi] > 0.5f) && lsum > 0.f;
  const float inv = qok ? 1.f / lsum : 0.f;
  if (!qrow) return;
  T* O = reinterpret_cast<T*>(a.o) + ((size_t)bh * Mq + qi) * d;
  const T* Gr = s_g + (size_t)(qi - q0) * DP;  // staged gate row (LDS)
  // lane holds O^T[col = c*16 + 4g + r][query qi]
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int col = c * 16 + 4 * g + r;
      if (col < d) {
        float o = oacc[c][r] * inv;
        if (hasg) o *= 1.f / (1.f + __expf(-to_f32(Gr[col])));
        O[col] = from_f32<T>(o);
      }
    }
  if (g == 0) a.lse[(size_t)bh * Mq + qi] = qok ? (m + fast_log2(lsum)) * LN2 : 0.f;
}

// ===========================================================================
// Backward, dQ pass: a wave pair owns 16 queries; keys stream.
//   P^T = exp2(sc K Q^T + bias - lse),  dP^T = V dO^T,  dS = P (dP - D)
//   dQ^T += K^T dS^T;  dense / window bias gradient = dS;  bins: d pos_weight partials.
template <typename T, int DP, bool WIN>
constexpr int attn_bwdq_lds() {
  using E = Eng<T, DP, WIN>;
  return 2 * lds_align(2 * E::CH * E::RS * (int)sizeof(T) + DP * E::TS * (int)sizeof(T) + E::CH * 4) + 2 * 68 * 4;
}

template <typename T, int DP, int BIAS, bool WIN, bool FAST>
__global__ void __launch_bounds__((Eng<T, DP, WIN>::NT)) attn_bwd_q2_kernel(AttnArgs a) {
  using E = Eng<T, DP, WIN>;
  using M = Mfma<T, DP>;
  using BR = BiasRow<T, BIAS>;
  constexpr int NT = E::NT, CH = E::CH, RS = E::RS, TS = E::TS, VEC = E::VEC, CB = E::CB, LD = E::LD;
  constexpr int SPW = E::SPW, KS = E::KS, RT = E::RT;
  constexpr int NC = DP / 16;
  constexpr int BW = BR::BW;
  constexpr bool HASB = BIAS != ATTN_BIAS_NONE;
  constexpr int KOFF = 0, VOFF = CH * RS * (int)sizeof(T), TOFF = 2 * CH * RS * (int)sizeof(T);
  constexpr int BOFF = TOFF + DP * TS * (int)sizeof(T);
  constexpr int BUF = lds_align(BOFF + CH * 4);
  extern __shared__ __align__(16) unsigned char smem[];
  float* s_pw = reinterpret_cast<float*>(smem + 2 * BUF);
  float* s_dpw = s_pw + 68;

  const int t = threadIdx.x, lane = t & (WAVE - 1), wave = t / WAVE, g = lane >> 4;
  const int rt = wave % RT, ks = wave / RT;
  const int BH = a.B * a.H, Mq = a.Mq, Nk = a.Nk, d = a.d;
  const int nqb = (Mq + E::RQ - 1) / E::RQ;
  int qb, bh;
  block_coords(nqb, BH, qb, bh);
  const int b = bh / a.H, h = bh % a.H;
  const int q0 = qb * E::RQ;
  const int qt = q0 + 16 * rt;
  const int qi = qt + (lane & 15);
  const int qc = min(qi, Mq - 1);
  const bool active = qt < Mq, qrow = qi < Mq;
  const bool qok = qrow && (!a.qmask || a.qmask[(size_t)b * Mq + qi] > 0.5f);
  const T* Qg = reinterpret_cast<const T*>(a.q) + (size_t)b * a.qsb + (size_t)h * a.qsh;
  const T* Kg = reinterpret_cast<const T*>(a.k) + (size_t)b * a.ksb + (size_t)h * a.ksh;
  const T* Vg = reinterpret_cast<const T*>(a.v) + (size_t)b * a.ksb + (size_t)h * a.ksh;
  const float* kmask = a.kmask ? a.kmask + (size_t)b * Nk : nullptr;
  const float sc = a.scale * LOG2E;
  int k_lo = 0, k_hi = Nk;
  if (WIN) window_keys2(q0, Nk, k_lo, k_hi);

  if (BIAS == ATTN_BIAS_BINS)
    for (int k = t; k < 68; k += NT) {
      s_pw[k] = LOG2E * a.pos_w[h * 68 + k];
      s_dpw[k] = 0.f;
    }
  BR br;
  br.row = nullptr;
  T* drow = nullptr;  // bias-gradient row of this lane's query, indexed by key
  if (BIAS == ATTN_BIAS_DENSE) {
    br.row = reinterpret_cast<const typename BR::BT*>(reinterpret_cast<const T*>(a.bias) +
                                                       ((size_t)bh * Mq + qc) * Nk);
    if (a.dbias) drow = reinterpret_cast<T*>(a.dbias) + ((size_t)bh * Mq + qc) * Nk;
  } else if (BIAS == ATTN_BIAS_WINDOW) {
    const int w = q0 / ATTN_WQ;
    const size_t off = (((size_t)w * a.H + h) * ATTN_WQ + (qc - ATTN_WQ * w)) * ATTN_WK;
    const int kofs = ATTN_WQ * w - ATTN_WOFF;
    br.row = reinterpret_cast<const typename BR::BT*>(reinterpret_cast<const T*>(a.bias) + off - kofs);
    if (a.dbias) {
      // The window bias has no batch dimension, so with B > 1 every batch row writes
      // its gradient to a slab set of its own and the finalize sums them in row order.
      T* dbase = a.dbias_rows
                     ? reinterpret_cast<T*>(a.dbias_rows) + (size_t)b * ((Mq + ATTN_WQ - 1) / ATTN_WQ) * a.H * ATTN_WQ * ATTN_WK
                     : reinterpret_cast<T*>(a.dbias);
      drow = dbase + off - kofs;
      // The main loop writes the window's keys [k_lo, k_hi) of its rows < Mq; the rest of
      // the (32, 128) slab (keys clipped at the sequence ends, rows past Mq) is zeroed
      // here, so the caller need not clear the gradient.
      // (only windows at the sequence ends have such entries: a uniform test)
      if (k_lo > kofs || k_hi < kofs + ATTN_WK || q0 + ATTN_WQ > Mq) {
        T* slab = dbase + ((size_t)w * a.H + h) * ATTN_WQ * ATTN_WK;
        for (int e = t; e < ATTN_WQ * ATTN_WK; e += NT) {
          const int key = kofs + (e % ATTN_WK);
          if (q0 + e / ATTN_WK >= Mq || key < k_lo || key >= k_hi) slab[e] = from_f32<T>(0.f);
        }
      }
    }
  } else if (BIAS == ATTN_BIAS_BINS) {
    br.row = reinterpret_cast<const typename BR::BT*>(a.bins + ((size_t)b * Mq + qc) * Nk);
  }

  Flight<T, LD, FAST> kfl, vfl;
  float kmraw;
  uint4 bcur[SPW][BW], bnxt[SPW][BW];
  auto prefetch = [&](int c0) {
#pragma unroll
    for (int u = 0; u < LD; ++u) {
      const int idx = t + NT * u;
      kfl.load(u, Kg, a.ksn, c0 + idx / CB, k_hi, (idx % CB) * VEC, d);
      vfl.load(u, Vg, a.ksn, c0 + idx / CB, k_hi, (idx % CB) * VEC, d);
    }
    if (kmask) kmraw = kmask[min(c0 + t % CH, k_hi - 1)];
    if (HASB && FAST) {
#pragma unroll
      for (int j = 0; j < SPW; ++j) br.load8(bnxt[j], c0 + 32 * (ks + KS * j) + 8 * g, k_hi);
    }
  };

  // Backward prep of the resident rows, for this pass and the dK/dV pass that runs
  // after it: do_w = sigma(G) dO (zero for masked rows and padded columns),
  // D_i = sum_c dO_ic O_ic, dG = (1 - sigma) O dO (O is the gated output).  The four
  // lanes of a row (g = 0..3) own RUN columns each; waves ks = 0 write.  The row's
  // operands are loaded from clamped addresses before chunk 0's prefetch is issued,
  // so both round trips overlap.
  constexpr int RUN = M::RUN;
  const int c0r = g * RUN;
  const size_t row = (size_t)bh * Mq + qc;
  T rq[RUN], rdo[RUN], ro[RUN], rg[RUN];
  {
    const T* Qr = Qg + (size_t)qc * a.qsn;
    const T* dO = reinterpret_cast<const T*>(a.dout) + row * d;
    const T* Or = reinterpret_cast<const T*>(a.o) + row * d;
    const T* Gr = a.g ? reinterpret_cast<const T*>(a.g) + (size_t)b * a.qsb + (size_t)h * a.qsh + (size_t)qc * a.qsn
                      : Or;
    if constexpr (FAST) {
      // 16-byte blocks; d is a multiple of VEC, so a block is wholly inside or
      // wholly outside the row (outside: a clamped block, zeroed below by c < d)
      static_assert(RUN % VEC == 0, "whole 16-byte blocks per lane");
#pragma unroll
      for (int k = 0; k < RUN / VEC; ++k) {
        const int cb = min(c0r + VEC * k, d - VEC);
        *reinterpret_cast<uint4*>(rq + VEC * k) = *reinterpret_cast<const uint4*>(Qr + cb);
        *reinterpret_cast<uint4*>(rdo + VEC * k) = *reinterpret_cast<const uint4*>(dO + cb);
        *reinterpret_cast<uint4*>(ro + VEC * k) = *reinterpret_cast<const uint4*>(Or + cb);
        *reinterpret_cast<uint4*>(rg + VEC * k) = *reinterpret_cast<const uint4*>(Gr + cb);
      }
    } else {
#pragma unroll
      for (int e = 0; e < RUN; ++e) {
        const int c = min(c0r + e, d - 1);
        rq[e] = Qr[c];
        rdo[e] = dO[c];
        ro[e] = Or[c];
        rg[e] = Gr[c];
      }
    }
  }
  prefetch(k_lo);

  typename M::Frag qf, df;
  float Di;
  {
    T tq[RUN], td[RUN];
    T* dGr = (a.g && a.dg && ks == 0 && qrow) ? reinterpret_cast<T*>(a.dg) + row * d : nullptr;
    float part = 0.f;
#pragma unroll
    for (int e = 0; e < RUN; ++e) {
      const int c = c0r + e;
      const bool in = c < d;
      tq[e] = (qrow && in) ? rq[e] : from_f32<T>(0.f);
      const float dov = (qok && in) ? to_f32(rdo[e]) : 0.f;
      const float ov = (qok && in) ? to_f32(ro[e]) : 0.f;
      const float s = (qok && in && a.g) ? 1.f / (1.f + __expf(-to_f32(rg[e]))) : 1.f;
      if (dGr && in) dGr[c] = from_f32<T>((1.f - s) * ov * dov);
      td[e] = from_f32<T>(s * dov);
      part += dov * ov;
    }
    part += __shfl_xor(part, 16, WAVE);
    part += __shfl_xor(part, 32, WAVE);
    Di = part;
    if (ks == 0 && qrow) {
      T* dst = reinterpret_cast<T*>(a.do_w) + row * DP + c0r;
#pragma unroll
      for (int e = 0; e < RUN; ++e) dst[e] = td[e];
      if (g == 0) a.dcoef[row] = part;
    }
    M::from_run(qf, tq);
    M::from_run(df, td);
  }
  // P = exp2(sc * (qk - l2 / sc) + bias): the -lse term rides in the MFMA accumulator
  const float l2 = qok ? a.lse[(size_t)bh * Mq + qi] * LOG2E : POS_BIG;
  const float ci = -l2 / sc;
  const f32x4 cinit = {ci, ci, ci, ci};
  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};

  f32x4 dq[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) dq[c] = zero;

  int buf = 0;
  for (int c0 = k_lo; c0 < k_hi; c0 += CH, buf ^= 1) {
    unsigned char* base = smem + buf * BUF;
    T* Ks = reinterpret_cast<T*>(base + KOFF);
    T* Vs = reinterpret_cast<T*>(base + VOFF);
    T* KTs = reinterpret_cast<T*>(base + TOFF);
    float* kb = reinterpret_cast<float*>(base + BOFF);
#pragma unroll
    for (int u = 0; u < LD; ++u) {
      const int idx = t + NT * u;
      const int row = idx / CB, col = (idx % CB) * VEC;
      const uint4 kv = kfl.get(u);
      *reinterpret_cast<uint4*>(Ks + (size_t)row * RS + col) = kv;
      *reinterpret_cast<uint4*>(Vs + (size_t)row * RS + col) = vfl.get(u);
      st_transposed<T>(KTs, TS, row, col, kv);
    }
    if (t < CH) kb[t] = (c0 + t < k_hi && (!kmask || kmraw > 0.5f)) ? 0.f : NEG_BIG;
    if (HASB && FAST) {
#pragma unroll
      for (int j = 0; j < SPW; ++j)
#pragma unroll
        for (int w = 0; w < BW; ++w) bcur[j][w] = bnxt[j][w];
    }
    __syncthreads();
    if (c0 + CH < k_hi) prefetch(c0 + CH);
    if (!active) continue;
#pragma unroll
    for (int j = 0; j < SPW; ++j) {
      const int kl = 32 * (ks + KS * j);
      if (c0 + kl >= k_hi) break;
      const int pr = kl + perm_row(lane, 0);
      typename M::Frag f0, f1;
      M::load(f0, Ks + (size_t)pr * RS, lane);
      M::load(f1, Ks + (size_t)(pr + 4) * RS, lane);
      const f32x4 s0 = M::qk(f0, qf, cinit);
      const f32x4 s1 = M::qk(f1, qf, cinit);
      M::load(f0, Vs + (size_t)pr * RS, lane);
      M::load(f1, Vs + (size_t)(pr + 4) * RS, lane);
      const f32x4 dp0 = M::qk(f0, df, zero);
      const f32x4 dp1 = M::qk(f1, df, zero);
      const f32x4 kb0 = *reinterpret_cast<const f32x4*>(kb + kl + 8 * g);
      const f32x4 kb1 = *reinterpret_cast<const f32x4*>(kb + kl + 8 * g + 4);
      const int key0 = c0 + kl + 8 * g;
      float ds[8];
      unsigned bins[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float b0 = kb0[e], b1 = kb1[e];
        if (HASB) {
          if (FAST) {
            b0 += bias_value<T, BIAS>(bcur[j], e, s_pw);
            b1 += bias_value<T, BIAS>(bcur[j], 4 + e, s_pw);
          } else {
            b0 += br.elem(key0 + e, k_hi, s_pw);
            b1 += br.elem(key0 + 4 + e, k_hi, s_pw);
          }
        }
        const float p0 = fast_exp2(__builtin_fmaf(s0[e], sc, b0));
        const float p1 = fast_exp2(__builtin_fmaf(s1[e], sc, b1));
        ds[e] = p0 * (dp0[e] - Di);
        ds[4 + e] = p1 * (dp1[e] - Di);
      }
#pragma unroll
      for (int c = 0; c < NC; ++c)
        dq[c] = PV8<T>::mma(KTs + (size_t)(c * 16 + (lane & 15)) * TS + kl + 8 * g, ds, dq[c]);
      if ((BIAS == ATTN_BIAS_DENSE || BIAS == ATTN_BIAS_WINDOW) && drow && qrow) {
        union { uint4 u[sizeof(T) == 2 ? 1 : 2]; T v[8]; } o;
#pragma unroll
        for (int e = 0; e < 8; ++e) o.v[e] = from_f32<T>(ds[e]);
        if (FAST && key0 + 8 <= k_hi) {
#pragma unroll
          for (int w = 0; w < (sizeof(T) == 2 ? 1 : 2); ++w)
            *reinterpret_cast<uint4*>(drow + key0 + w * (16 / (int)sizeof(T))) = o.u[w];
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (key0 + e < k_hi) drow[key0 + e] = o.v[e];
        }
      }
      if (BIAS == ATTN_BIAS_BINS) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          if (ds[e] != 0.f && key0 + e < k_hi) {
            unsigned k;
            if (FAST) {
              const uint4 u = bcur[j][e >> 2];
              k = (e & 3) == 0 ? u.x : (e & 3) == 1 ? u.y : (e & 3) == 2 ? u.z : u.w;
            } else {
              k = (unsigned)a.bins[((size_t)b * Mq + qc) * Nk + key0 + e];
            }
            if (k < 68u) atomicAdd(&s_dpw[k], ds[e]);
          }
        }
      }
    }
  }

  // merge the KS partial dQ of each resident tile
  __syncthreads();
  float* mg = reinterpret_cast<float*>(smem);
  if (ks > 0 && active) {
    float* dst = mg + ((size_t)((ks - 1) * RT + rt) * WAVE + lane) * 4 * NC;
#pragma unroll
    for (int c = 0; c < NC; ++c) *reinterpret_cast<f32x4*>(dst + 4 * c) = dq[c];
  }
  __syncthreads();
  if (BIAS == ATTN_BIAS_BINS)
    for (int k = t; k < 68; k += NT) a.dpw_part[((size_t)bh * nqb + qb) * 68 + k] = s_dpw[k];
  if (ks > 0 || !active || !qrow) return;
#pragma unroll
  for (int s = 1; s < KS; ++s) {
    const float* src = mg + ((size_t)((s - 1) * RT + rt) * WAVE + lane) * 4 * NC;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const f32x4 o = *reinterpret_cast<const f32x4*>(src + 4 * c);
#pragma unroll
      for (int r = 0; r < 4; ++r) dq[c][r] += o[r];
    }
  }
  T* dQ = reinterpret_cast<T*>(a.dq) + ((size_t)bh * Mq + qi) * d;
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int col = c * 16 + 4 * g + r;
      if (col < d) dQ[col] = from_f32<T>(a.scale * dq[c][r]);
    }
}

// ===========================================================================
// Backward, dK / dV pass: a wave pair owns 16 keys; queries stream.
//   P = exp2(sc Q K^T + bias - lse),  dP = dO V^T,  dS = P (dP - D)
//   dV^T += dO^T P,  dK^T += Q^T dS
// The lane holds key kj = l % 16 and queries 8g..8g+7 of a step.  The bias of those
// (query, key) pairs is read query-major (contiguous keys) as an MFMA A operand and
// transposed into the accumulator layout by a product with the identity.
template <typename T, int DP>
struct EngKV {
  using E = Eng<T, DP, false>;
  static constexpr int RK = 64, RT = 4, KS = 2, NT = 512;
  static constexpr int CH = E::CH, RS = E::RS, TS = E::TS, VEC = E::VEC, CB = E::CB;
  static constexpr int LD = CH * CB / NT, SPW = CH / 32 / KS;
  static_assert(SPW >= 1 && CH * CB % NT == 0 && LD >= 1, "dK/dV pass geometry");
};
template <typename T, int DP>
constexpr int attn_bwdkv_lds() {
  using K = EngKV<T, DP>;
  return 2 * lds_align(2 * K::CH * K::RS * (int)sizeof(T) + 2 * DP * K::TS * (int)sizeof(T) + 2 * K::CH * 4) + 68 * 4;
}

// bias(query m of the step's tile hf, key kt + n) for the 16x16 tile, in the accumulator layout.
template <typename T, int BIAS, bool FAST>
struct KVBias {
  using BT = typename std::conditional<BIAS == ATTN_BIAS_BINS, int, T>::type;
  static constexpr bool BF = BIAS != ATTN_BIAS_BINS && sizeof(T) == 2;  // bf16 values: one 16x16x16 MFMA
  static constexpr int NW = BF ? 2 : 4;                                 // 32-bit words per lane and tile
  struct Raw { unsigned w[NW]; };
  // lane: A row (l % 16) = query q, keys kt + 4g .. kt + 4g + 3 of row `row` (indexed by key)
  __device__ static __forceinline__ void load(Raw& r, const BT* row, int key, int k_hi) {
    if (FAST) {
      if (BF) {
        const uint2 v = *reinterpret_cast<const uint2*>(row + min(key, k_hi - 4));
        r.w[0] = v.x;
        r.w[1] = v.y;
      } else {
        const uint4 v = *reinterpret_cast<const uint4*>(row + min(key, k_hi - 4));
        r.w[0] = v.x; r.w[1] = v.y; r.w[2] = v.z; r.w[3] = v.w;
      }
    } else {
      union { unsigned w[NW]; BT e[4]; } u;
#pragma unroll
      for (int e = 0; e < 4; ++e) u.e[e] = row[min(key + e, k_hi - 1)];
#pragma unroll
      for (int i = 0; i < NW; ++i) r.w[i] = u.w[i];
    }
  }
  // D[m][n] = value(query m, key n) in log2 units (bins: pre-scaled table; dense: times LOG2E later)
  __device__ static __forceinline__ f32x4 transpose(const Raw& r, const float* pw2, int lane) {
    const int g = lane >> 4, n = lane & 15;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    if constexpr (BF) {
      typedef short s4 __attribute__((ext_vector_type(4)));
      s4 av, bv;
      av[0] = (short)(r.w[0] & 0xffffu); av[1] = (short)(r.w[0] >> 16);
      av[2] = (short)(r.w[1] & 0xffffu); av[3] = (short)(r.w[1] >> 16);
#pragma unroll
      for (int e = 0; e < 4; ++e) bv[e] = (4 * g + e == n) ? (short)0x3f80 : (short)0;
      acc = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(av, bv, acc, 0, 0, 0);
    } else {
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        float v;
        if constexpr (BIAS == ATTN_BIAS_BINS) {
          const unsigned k = r.w[s];
          v = k < 68u ? pw2[k] : 0.f;
        } else {
          v = __uint_as_float(r.w[s]);
        }
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(v, (4 * g + s == n) ? 1.f : 0.f, acc, 0, 0, 0);
      }
    }
    return acc;
  }
};

template <typename T, int DP, int BIAS, bool WIN, bool FAST>
__global__ void __launch_bounds__(512) attn_bwd_kv2_kernel(AttnArgs a) {
  using K = EngKV<T, DP>;
  using M = Mfma<T, DP>;
  using KB = KVBias<T, BIAS, FAST>;
  constexpr int NT = K::NT, CH = K::CH, RS = K::RS, TS = K::TS, VEC = K::VEC, CB = K::CB, LD = K::LD;
  constexpr int SPW = K::SPW, KS = K::KS, RT = K::RT;
  constexpr int NC = DP / 16;
  constexpr bool HASB = BIAS != ATTN_BIAS_NONE;
  constexpr int QOFF = 0, DOFF = CH * RS * (int)sizeof(T), QTOFF = 2 * CH * RS * (int)sizeof(T);
  constexpr int DTOFF = QTOFF + DP * TS * (int)sizeof(T), LOFF = DTOFF + DP * TS * (int)sizeof(T);
  constexpr int BUF = lds_align(LOFF + 2 * CH * 4);
  extern __shared__ __align__(16) unsigned char smem[];
  float* s_pw = reinterpret_cast<float*>(smem + 2 * BUF);

  const int t = threadIdx.x, lane = t & (WAVE - 1), wave = t / WAVE, g = lane >> 4;
  const int rt = wave % RT, ks = wave / RT;
  const int BH = a.B * a.H, Mq = a.Mq, Nk = a.Nk, d = a.d;
  const int nkb = (Nk + K::RK - 1) / K::RK;
  // units: (b,h) x query split; the key blocks of a unit stream the same queries
  int kbk, unit;
  block_coords(nkb, BH * a.qsplit, kbk, unit);
  const int bh = unit / a.qsplit, split = unit % a.qsplit;
  const int b = bh / a.H, h = bh % a.H;
  const int k0 = kbk * K::RK;
  const int kt = k0 + 16 * rt;
  const int kj = kt + (lane & 15);
  const bool active = kt < Nk;
  const bool kok = kj < Nk && (!a.kmask || a.kmask[(size_t)b * Nk + kj] > 0.5f);
  const T* Qg = reinterpret_cast<const T*>(a.q) + (size_t)b * a.qsb + (size_t)h * a.qsh;
  const T* Kg = reinterpret_cast<const T*>(a.k) + (size_t)b * a.ksb + (size_t)h * a.ksh;
  const T* Vg = reinterpret_cast<const T*>(a.v) + (size_t)b * a.ksb + (size_t)h * a.ksh;
  const T* dOw = reinterpret_cast<const T*>(a.do_w) + (size_t)bh * Mq * DP;
  const float* qmask = a.qmask ? a.qmask + (size_t)b * Mq : nullptr;
  const float* lse = a.lse + (size_t)bh * Mq;
  const float* dco = a.dcoef + (size_t)bh * Mq;
  const float sc = a.scale * LOG2E;

  // query range: this split, intersected with the windows that see the block's keys
  const int per = (((Mq + a.qsplit - 1) / a.qsplit) + 31) / 32 * 32;
  int q_lo = split * per, q_hi = min(Mq, q_lo + per);
  int wq_lo = q_lo, wq_hi = q_hi;
  if (WIN) {
    int l1, h1;
    window_queries(k0, min(Nk, k0 + K::RK), Mq, l1, h1);
    q_lo = max(q_lo, l1);
    q_hi = min(q_hi, h1);
    window_queries(kt, min(Nk, kt + 16), Mq, l1, h1);
    wq_lo = max(wq_lo, l1);
    wq_hi = min(wq_hi, h1);
  }
  if (BIAS == ATTN_BIAS_BINS)
    for (int k = t; k < 68; k += NT) s_pw[k] = LOG2E * a.pos_w[h * 68 + k];

  typename M::Frag kf, vf;
  {
    constexpr int RUN = M::RUN;
    T tk[RUN], tv[RUN];
    const int c0 = g * RUN;
    const bool krow = kj < Nk;
    if constexpr (FAST) {
      // 16-byte blocks from a clamped row and block start; validity applied after
      static_assert(RUN % VEC == 0, "whole 16-byte blocks per lane");
      const size_t ro = (size_t)min(kj, Nk - 1) * a.ksn;
#pragma unroll
      for (int k = 0; k < RUN / VEC; ++k) {
        const int cb = min(c0 + VEC * k, d - VEC);
        *reinterpret_cast<uint4*>(tk + VEC * k) = *reinterpret_cast<const uint4*>(Kg + ro + cb);
        *reinterpret_cast<uint4*>(tv + VEC * k) = *reinterpret_cast<const uint4*>(Vg + ro + cb);
      }
#pragma unroll
      for (int e = 0; e < RUN; ++e) {
        const bool in = krow && c0 + e < d;
        tk[e] = in ? tk[e] : from_f32<T>(0.f);
        tv[e] = in ? tv[e] : from_f32<T>(0.f);
      }
    } else {
#pragma unroll
      for (int e = 0; e < RUN; ++e) {
        tk[e] = (krow && c0 + e < d) ? Kg[(size_t)kj * a.ksn + c0 + e] : from_f32<T>(0.f);
        tv[e] = (krow && c0 + e < d) ? Vg[(size_t)kj * a.ksn + c0 + e] : from_f32<T>(0.f);
      }
    }
    M::from_run(kf, tk);
    M::from_run(vf, tv);
  }
  // bias rows: A row (l % 16) of tile hf is query qp + perm_row(l, hf); keys kt + 4g ..
  const int bkey = kt + 4 * g;
  auto bias_row = [&](int q) -> const typename KB::BT* {
    const int qq = min(q, Mq - 1);
    if (BIAS == ATTN_BIAS_DENSE)
      return reinterpret_cast<const typename KB::BT*>(reinterpret_cast<const T*>(a.bias) + ((size_t)bh * Mq + qq) * Nk);
    if (BIAS == ATTN_BIAS_WINDOW) {
      const int w = qq / ATTN_WQ;
      const T* row = reinterpret_cast<const T*>(a.bias) + (((size_t)w * a.H + h) * ATTN_WQ + (qq - ATTN_WQ * w)) * ATTN_WK;
      return reinterpret_cast<const typename KB::BT*>(row - (ATTN_WQ * w - ATTN_WOFF));
    }
    return reinterpret_cast<const typename KB::BT*>(a.bins + ((size_t)b * Mq + qq) * Nk);
  };
  // key bound of the bias reads: the key tile is whole inside or outside each window
  const int bk_hi = WIN ? min(Nk, kt + 16) : Nk;

  Flight<T, LD, FAST> qfl, dfl;
  float lraw, draw, mraw;
  typename KB::Raw bcur[SPW][2], bnxt[SPW][2];
  auto prefetch = [&](int c0) {
#pragma unroll
    for (int u = 0; u < LD; ++u) {
      const int idx = t + NT * u;
      qfl.load(u, Qg, a.qsn, c0 + idx / CB, q_hi, (idx % CB) * VEC, d);
      dfl.load(u, dOw, DP, c0 + idx / CB, q_hi, (idx % CB) * VEC, DP);
    }
    {
      const int q = min(c0 + t % CH, q_hi - 1);
      lraw = lse[q];
      draw = dco[q];
      if (qmask) mraw = qmask[q];
    }
    if (HASB && FAST && active && wq_lo < wq_hi) {
#pragma unroll
      for (int j = 0; j < SPW; ++j)
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
          int q = c0 + 32 * (ks + KS * j) + perm_row(lane, hf);
          // windowed: steps outside the wave's windows are skipped; keep their reads
          // inside a window that holds this key tile
          if (WIN) q = min(max(q, wq_lo), wq_hi - 1);
          KB::load(bnxt[j][hf], bias_row(q), bkey, bk_hi);
        }
    }
  };

  f32x4 dk[NC], dv[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) dk[c] = dv[c] = f32x4{0.f, 0.f, 0.f, 0.f};
  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};

  if (q_lo < q_hi) prefetch(q_lo);
  int buf = 0;
  for (int c0 = q_lo; c0 < q_hi; c0 += CH, buf ^= 1) {
    unsigned char* base = smem + buf * BUF;
    T* Qs = reinterpret_cast<T*>(base + QOFF);
    T* dOs = reinterpret_cast<T*>(base + DOFF);
    T* QTs = reinterpret_cast<T*>(base + QTOFF);
    T* dOTs = reinterpret_cast<T*>(base + DTOFF);
    float* nl2 = reinterpret_cast<float*>(base + LOFF);
    float* Dq = nl2 + CH;
#pragma unroll
    for (int u = 0; u < LD; ++u) {
      const int idx = t + NT * u;
      const int row = idx / CB, col = (idx % CB) * VEC;
      const uint4 qv = qfl.get(u), dv4 = dfl.get(u);
      *reinterpret_cast<uint4*>(Qs + (size_t)row * RS + col) = qv;
      *reinterpret_cast<uint4*>(dOs + (size_t)row * RS + col) = dv4;
      st_transposed<T>(QTs, TS, row, col, qv);
      st_transposed<T>(dOTs, TS, row, col, dv4);
    }
    if (t < CH) {
      const bool ok = c0 + t < q_hi && (!qmask || mraw > 0.5f);
      nl2[t] = ok ? -lraw * LOG2E : -POS_BIG;
      Dq[t] = ok ? draw : 0.f;
    }
    if (HASB && FAST) {
#pragma unroll
      for (int j = 0; j < SPW; ++j)
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) bcur[j][hf] = bnxt[j][hf];
    }
    __syncthreads();
    if (c0 + CH < q_hi) prefetch(c0 + CH);
    if (!active) continue;
#pragma unroll
    for (int j = 0; j < SPW; ++j) {
      const int ql = 32 * (ks + KS * j);
      const int qp = c0 + ql;
      if (qp >= q_hi) break;
      if (WIN && (qp < wq_lo || qp >= wq_hi)) continue;  // 32-aligned: the step is wholly in or out
      const int pr = ql + perm_row(lane, 0);
      typename M::Frag f0, f1;
      M::load(f0, Qs + (size_t)pr * RS, lane);
      M::load(f1, Qs + (size_t)(pr + 4) * RS, lane);
      const f32x4 s0 = M::qk(f0, kf, zero);
      const f32x4 s1 = M::qk(f1, kf, zero);
      M::load(f0, dOs + (size_t)pr * RS, lane);
      M::load(f1, dOs + (size_t)(pr + 4) * RS, lane);
      const f32x4 dp0 = M::qk(f0, vf, zero);
      const f32x4 dp1 = M::qk(f1, vf, zero);
      f32x4 bb0 = *reinterpret_cast<const f32x4*>(nl2 + ql + 8 * g);
      f32x4 bb1 = *reinterpret_cast<const f32x4*>(nl2 + ql + 8 * g + 4);
      if (HASB) {
        typename KB::Raw r0, r1;
        if (FAST) {
          r0 = bcur[j][0];
          r1 = bcur[j][1];
        } else {
          KB::load(r0, bias_row(qp + perm_row(lane, 0)), bkey, bk_hi);
          KB::load(r1, bias_row(qp + perm_row(lane, 1)), bkey, bk_hi);
        }
        const f32x4 t0 = KB::transpose(r0, s_pw, lane);
        const f32x4 t1 = KB::transpose(r1, s_pw, lane);
        const float bsc = BIAS == ATTN_BIAS_BINS ? 1.f : LOG2E;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          bb0[e] = __builtin_fmaf(t0[e], bsc, bb0[e]);
          bb1[e] = __builtin_fmaf(t1[e], bsc, bb1[e]);
        }
      }
      const f32x4 d0 = *reinterpret_cast<const f32x4*>(Dq + ql + 8 * g);
      const f32x4 d1 = *reinterpret_cast<const f32x4*>(Dq + ql + 8 * g + 4);
      float p[8], ds[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        p[e] = fast_exp2(__builtin_fmaf(s0[e], sc, bb0[e]));
        p[4 + e] = fast_exp2(__builtin_fmaf(s1[e], sc, bb1[e]));
        ds[e] = p[e] * (dp0[e] - d0[e]);
        ds[4 + e] = p[4 + e] * (dp1[e] - d1[e]);
      }
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        dv[c] = PV8<T>::mma(dOTs + (size_t)(c * 16 + (lane & 15)) * TS + ql + 8 * g, p, dv[c]);
        dk[c] = PV8<T>::mma(QTs + (size_t)(c * 16 + (lane & 15)) * TS + ql + 8 * g, ds, dk[c]);
      }
    }
  }

  // merge the KS partials of each key tile
  __syncthreads();
  float* mg = reinterpret_cast<float*>(smem);
  if (ks > 0 && active) {
    float* dst = mg + ((size_t)((ks - 1) * RT + rt) * WAVE + lane) * 8 * NC;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      *reinterpret_cast<f32x4*>(dst + 4 * c) = dk[c];
      *reinterpret_cast<f32x4*>(dst + 4 * NC + 4 * c) = dv[c];
    }
  }
  __syncthreads();
  if (ks > 0 || !active || kj >= Nk) return;
#pragma unroll
  for (int s = 1; s < KS; ++s) {
    const float* src = mg + ((size_t)((s - 1) * RT + rt) * WAVE + lane) * 8 * NC;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const f32x4 ok = *reinterpret_cast<const f32x4*>(src + 4 * c);
      const f32x4 ov = *reinterpret_cast<const f32x4*>(src + 4 * NC + 4 * c);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        dk[c][r] += ok[r];
        dv[c][r] += ov[r];
      }
    }
  }
  // lane holds dK^T / dV^T [col = c*16 + 4g + r][key kj]; masked keys get zero
  const float kmul = kok ? 1.f : 0.f;
  if (a.qsplit > 1) {
    float* part = a.kv_part + (((size_t)split * BH + bh) * Nk + kj) * 2 * DP;
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int col = c * 16 + 4 * g + r;
        part[col] = kmul * a.scale * dk[c][r];
        part[DP + col] = kmul * dv[c][r];
      }
    return;
  }
  T* dK = reinterpret_cast<T*>(a.dk) + ((size_t)bh * Nk + kj) * d;
  T* dV = reinterpret_cast<T*>(a.dv) + ((size_t)bh * Nk + kj) * d;
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int col = c * 16 + 4 * g + r;
      if (col < d) {
        dK[col] = from_f32<T>(kmul * a.scale * dk[c][r]);
        dV[col] = from_f32<T>(kmul * dv[c][r]);
      }
    }
}

}  // namespace dfl
