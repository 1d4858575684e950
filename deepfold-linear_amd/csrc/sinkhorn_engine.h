// Sweep engine shared by the Sinkhorn forward and backward kernels.
//
// A "sweep" visits, for every resident 16-row tile owned by this workgroup, all
// streamed 16-row tiles of the same (b,h): the cost tile QK^T is recomputed on
// MFMA from LDS-resident operands and reduced on the fly.  In a row sweep the
// resident rows are Q (plan rows i) and the streamed rows are K (plan columns
// j); in a column sweep the roles swap.  NT = threads per workgroup.
#pragma once
#include "common.h"
#include "sinkhorn_args.h"

namespace dfl {

constexpr int SK_NT = 256;  // backward workgroup size
constexpr int SK_NW = SK_NT / WAVE;
constexpr int SK_RT = 4;    // resident tiles per register chunk

// Scratch floats needed by the sweeps of an NT-thread workgroup.
template <int NT> constexpr int sweep_scratch() { return 2 * (NT / WAVE) * SK_RT * 16; }
constexpr int LSE_SCRATCH = 2 * SK_NW * SK_RT * 16;
// Streamed tiles a wave keeps in registers per pass of a sweep.
template <typename T, int DP> constexpr int sweep_sch() { return (sizeof(T) == 2 && DP == 32) ? 6 : 4; }

// Position-bin / geometry bias of the cost, in log2 units of the logit:
//   bias(i, j) = -(log2 e / eps) * (pw[bins_ij] + w * d_ij / (r0 + d_ij)).
// Bins come as padded uint8 copies of the caller's int32 (B, N, N) array
// (bins8_kernel): row-major b8[i][j] and transposed b8t[j][i], row stride Np,
// BIN_NONE = 68 outside [0, 68) and on padding (its table entry is 0), so that four
// consecutive indices are one aligned 32-bit load in either sweep direction and the
// lookup needs no range test.  The geometry term is evaluated from the coordinates
// (LDS in resident storage): on MI355X that is cheaper than reading a precomputed
// fp32 d/(r0 + d) matrix from L2 (16-byte loads per quad made the forward 13% slower).
constexpr unsigned BIN_NONE = 68;
struct Bias {
  const uint8_t* b8;   // (Np, Np) bins of this batch row, or null
  const uint8_t* b8t;  // the transposed copy
  const float* posw;   // LDS: 69 pre-scaled weights of this head, posw[BIN_NONE] = 0
  const float* xs;     // coordinates [Np][3] (LDS or global), or null (no geometry term)
  float geo_scale;     // -log2e * w / eps
  float r0;
  int Np;
  // The same values computed once for this (b,h) (bias_mat_kernel): mat[i][j] =
  // bias(i, j) and matT[j][i] = bias(i, j), row stride Np; when set, the lookups
  // below read them instead of evaluating bins and distances.
  const float* mat = nullptr;
  const float* matT = nullptr;
  __device__ __forceinline__ float geo(float dx, float dy, float dz) const {
    const float dist = fmaxf(__builtin_amdgcn_sqrtf(dx * dx + dy * dy + dz * dz), 1e-8f);
    return geo_scale * dist * __builtin_amdgcn_rcpf(r0 + dist);
  }
  __device__ __forceinline__ float operator()(int i, int j) const {
    // Tile rounding can hand in indices up to 15 past the last tile; their results
    // are discarded, and clamping keeps every read inside the padded arrays.
    i = min(i, Np - 1);
    j = min(j, Np - 1);
    if (mat) return mat[(size_t)i * Np + j];
    float b = 0.f;
    if (b8) b += posw[b8[(size_t)i * Np + j]];
    if (xs) b += geo(xs[3 * i] - xs[3 * j], xs[3 * i + 1] - xs[3 * j + 1], xs[3 * i + 2] - xs[3 * j + 2]);
    return b;
  }
  // The biases of resident index r against the four streamed indices s0[k]..s0[k]+3
  // of each of S streamed tiles (s0 % 4 == 0, s0 + 3 < Np).  COL: the streamed
  // indices are plan rows (column sweep), so the bins come from the transposed copy;
  // the distance is symmetric.  All S bin words are loaded under one test, back to
  // back, so their latencies overlap (a test per word leaves one wait per load).
  template <bool COL, int S>
  __device__ __forceinline__ void quads(int r, const int (&s0)[S], f32x4 (&out)[S]) const {
    if (mat) {
      const float* row = (COL ? matT : mat) + (size_t)r * Np;
#pragma unroll
      for (int k = 0; k < S; ++k) out[k] = *reinterpret_cast<const f32x4*>(row + s0[k]);
      return;
    }
#pragma unroll
    for (int k = 0; k < S; ++k) out[k] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (b8) {
      const uint8_t* row = (COL ? b8t : b8) + (size_t)r * Np;
      uint32_t w[S];
#pragma unroll
      for (int k = 0; k < S; ++k) w[k] = *reinterpret_cast<const uint32_t*>(row + s0[k]);
#pragma unroll
      for (int k = 0; k < S; ++k)
#pragma unroll
        for (int e = 0; e < 4; ++e) out[k][e] = posw[(w[k] >> (8 * e)) & 0xffu];
    }
    if (xs) {
      const float r0x = xs[3 * r], r1x = xs[3 * r + 1], r2x = xs[3 * r + 2];
#pragma unroll
      for (int k = 0; k < S; ++k) {
        const float* c = xs + 3 * s0[k];
        const f32x4 p = *reinterpret_cast<const f32x4*>(c);      // rows s0, s0+1 (x, y, z, x)
        const f32x4 q = *reinterpret_cast<const f32x4*>(c + 4);  // (y, z, x, y)
        const f32x4 t = *reinterpret_cast<const f32x4*>(c + 8);  // (z, x, y, z)
        out[k][0] += geo(r0x - p[0], r1x - p[1], r2x - p[2]);
        out[k][1] += geo(r0x - p[3], r1x - q[0], r2x - q[1]);
        out[k][2] += geo(r0x - q[2], r1x - q[3], r2x - t[0]);
        out[k][3] += geo(r0x - t[1], r1x - t[2], r2x - t[3]);
      }
    }
  }
};


// Stage rows [0, n) of a row-strided slice into LDS row-major [Np][DP]
// (zero-filling columns >= d and rows >= n).  16-byte loads when the layout allows.
template <typename T, int DP>
__device__ __forceinline__ void stage_rows(T* dst, const T* __restrict__ src, long long sn, int n, int d, int Np) {
  constexpr int VE = 16 / sizeof(T);  // elements per 16-byte vector
  const bool vec = (d == DP) && (sn % VE == 0) && ((reinterpret_cast<uintptr_t>(src) & 15) == 0);
  if (vec) {
    typedef __attribute__((__vector_size__(16))) int i32x4;
    constexpr int CPR = DP / VE;  // vectors per row
    for (int c = threadIdx.x; c < Np * CPR; c += blockDim.x) {
      const int row = c / CPR, k = c - row * CPR;
      i32x4 v = {0, 0, 0, 0};
      if (row < n) v = *reinterpret_cast<const i32x4*>(src + (size_t)row * sn + k * VE);
      *reinterpret_cast<i32x4*>(dst + (size_t)row * DP + k * VE) = v;
    }
    return;
  }
  for (int e = threadIdx.x; e < Np * DP; e += blockDim.x) {
    const int row = e / DP, col = e - row * DP;
    T v = from_f32<T>(0.f);
    if (row < n && col < d) v = src[(size_t)row * sn + col];
    dst[e] = v;
  }
}
// Transposed: dst[col][row], row stride Np.
template <typename T, int DP>
__device__ __forceinline__ void stage_rows_t(T* dst, const T* __restrict__ src, long long sn, int n, int d, int Np) {
  constexpr int VE = 16 / sizeof(T);
  const bool vec = (d == DP) && (sn % VE == 0) && ((reinterpret_cast<uintptr_t>(src) & 15) == 0);
  if (vec) {
    constexpr int CPR = DP / VE;
    for (int c = threadIdx.x; c < Np * CPR; c += blockDim.x) {
      const int row = c % Np, k = c / Np;  // consecutive threads -> consecutive rows (LDS-friendly)
      T v[VE];
      if (row < n) {
        const T* p = src + (size_t)row * sn + k * VE;
#pragma unroll
        for (int e = 0; e < VE; ++e) v[e] = p[e];
      } else {
#pragma unroll
        for (int e = 0; e < VE; ++e) v[e] = from_f32<T>(0.f);
      }
#pragma unroll
      for (int e = 0; e < VE; ++e) dst[(size_t)(k * VE + e) * Np + row] = v[e];
    }
    return;
  }
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
  unsigned hi = 0;
  for (int i = threadIdx.x; i < N; i += blockDim.x) {
    const bool ok = mask ? (mask[i] > 0.5f) : true;
    valid[i] = ok ? 1 : 0;
    if (ok) hi = i + 1;
  }
  block_atomic_max_u32(reinterpret_cast<unsigned*>(s_tmp), hi);
  __syncthreads();
  const int n = *s_tmp;
  __syncthreads();
  return n;
}

// Polls this thread's words buf[idx[k]], k < W (idx[k] < 0: none) until each
// carries `tag`, calling take(k, word) once per word.  Every word has two loads in
// flight, issued one sleep unit apart and checked alternately, so a load that still
// saw the old word costs that stagger rather than a whole round trip (an exchange
// round of a 16-member group measured 1826 instead of 2285 clocks on MI355X).
// The loads are unconditional (absent words read word 0 and are ignored), so
// the compiler can wait for one set with the other still in flight.  Returns
// false if the wait expires (then it raises the error).
template <int W, typename Take>
__device__ __forceinline__ bool poll_words(const uint64_t* buf, const int (&idx)[W], uint32_t tag, ErrRef err,
                                           Take take) {
  const uint32_t salt = tag >> 12;
  // a limit of 1 (failure-path tests): the wait gives up at once, whatever has arrived,
  // so the expiry does not depend on how early the words were published
  if (err.spin_limit == 1u) { raise_error(err, salt, 2u); return false; }
  const uint64_t* addr[W];
  bool done[W];
#pragma unroll
  for (int k = 0; k < W; ++k) {
    done[k] = idx[k] < 0;
    addr[k] = buf + (done[k] ? 0 : idx[k]);
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
      if (!done[k] && (uint32_t)wa[k] == tag) { take(k, wa[k]); done[k] = true; }
    if (all()) return true;
#pragma unroll
    for (int k = 0; k < W; ++k) wa[k] = ld(k);
    __builtin_amdgcn_s_sleep(1);  // back off: tight polling slows the publishers' stores
#pragma unroll
    for (int k = 0; k < W; ++k)
      if (!done[k] && (uint32_t)wb[k] == tag) { take(k, wb[k]); done[k] = true; }
    if (all()) return true;
#pragma unroll
    for (int k = 0; k < W; ++k) wb[k] = ld(k);
    __builtin_amdgcn_s_sleep(1);
    // Only a scalar counter here: a vector load of the error word on some iterations
    // would leave the compiler unable to count the loads in flight, and it would then
    // wait for all of them.  A member that gave up stops publishing, so the others'
    // waits expire too, within the spin limit (well under a second).
    if (++spins > err.spin_limit / 2) { raise_error(err, salt, 2u); return false; }
  }
}
// poll_words for the words i = base + t + k * stride of [0, n).
template <int W, typename Take>
__device__ __forceinline__ bool poll_batch(const uint64_t* buf, int base, int n, int stride, uint32_t tag, ErrRef err,
                                           Take take) {
  int idx[W];
#pragma unroll
  for (int k = 0; k < W; ++k) {
    const int i = base + (int)threadIdx.x + k * stride;
    idx[k] = i < n ? i : -1;
  }
  return poll_words<W>(buf, idx, tag, err, take);
}

// All words [0, n) of a vector, NT threads, batches of W = 1, 2 or 4 words a
// thread (the smallest that covers n, else repeated batches of 4).
template <int NT, typename Take>
__device__ __forceinline__ bool poll_vector(const uint64_t* buf, int n, uint32_t tag, ErrRef err, Take take) {
  if (n <= NT) return poll_batch<1>(buf, 0, n, NT, tag, err, [&](int k, uint64_t w) { take(k * NT, w); });
  if (n <= 2 * NT) return poll_batch<2>(buf, 0, n, NT, tag, err, [&](int k, uint64_t w) { take(k * NT, w); });
  for (int base = 0; base < n; base += 4 * NT)
    if (!poll_batch<4>(buf, base, n, NT, tag, err, [&](int k, uint64_t w) { take(base + k * NT, w); }))
      return false;
  return true;
}

// Gather a published potential vector [0, n) into dst (log2 units), writing
// NEG_BIG for masked entries, and fold max |new - old| over valid entries into
// *s_delta (float bits, >= 0; reset by the caller before a barrier that
// precedes this call).  Entries [n, Np) are pinned once by the caller.
// Returns false (uniformly) if the error flag is raised or a wait expires.
template <int NT>
__device__ __forceinline__ bool gather_potential(const uint64_t* buf, int n, uint32_t tag, float* dst,
                                                 const unsigned char* valid, ErrRef err, int* s_flag,
                                                 unsigned* s_delta) {
  const int t = threadIdx.x;
  float dmax = 0.f;
  // take(off, w): word i = off + t
  const bool ok = poll_vector<NT>(buf, n, tag, err, [&](int off, uint64_t w) {
    const int i = off + t;
    if (valid[i]) {
      const float nv = __uint_as_float((uint32_t)(w >> 32)) * LOG2E;
      dmax = fmaxf(dmax, fabsf(nv - dst[i]));
      dst[i] = nv;
    } else {
      dst[i] = NEG_BIG;
    }
  });
  if (!ok) *s_flag = 1;
  // NaN-safe: a NaN delta forces the online path
  block_atomic_max_u32(s_delta, dmax == dmax ? __float_as_uint(dmax) : 0x7f800000u);
  lds_barrier();  // dst, the flag and the change word are LDS
  return *s_flag == 0;
}

// Log2-sum-exp of x_ij = sc * <res_i, str_j> + w2_j (+ bias) over all streamed
// rows j, for each resident row of tiles [rt0, rt0 + nr).  TRANS: the streamed
// index is the plan's row index (column sweep), which matters only for the bias.
//   ONLINE = true : running max per lane (robust for any range); mx2 (if non-null)
//                   receives the row maximum.
//   ONLINE = false: fixed shift shift2[q] per resident row (caller guarantees
//                   every exponent x - shift stays within fp32 range).
// lse2[q] receives the result for local resident row q in [0, nr*16).
// If publish != null, the threads that finish row q also call publish(q, lse2_q)
// before the closing barrier.  *s_reset (if non-null) is zeroed before the first
// barrier of each chunk.  Called by the whole block.
template <int NT, typename T, int DP, bool GENERAL, bool TRANS, bool ONLINE, typename Pub>
__device__ __forceinline__ void lse_sweep(const T* __restrict__ res_lds, const T* __restrict__ str_lds,
                          const float* __restrict__ w2, int n_str_tiles, int rt0, int nr, float sc,
                          const Bias& bias, const float* __restrict__ shift2, float* lse2, float* mx2,
                          float* scratch, unsigned* s_reset, Pub publish) {
  using M = Mfma<T, DP>;
  constexpr int NW = NT / WAVE;
  constexpr int SCH = sweep_sch<T, DP>();
  const int lane = threadIdx.x & (WAVE - 1);
  const int wave = threadIdx.x / WAVE;
  const int g = lane >> 4;
  const float isc = 1.f / sc;
  // this wave's streamed tiles: st = wave + NW * k, k < ks
  const int ks = wave < n_str_tiles ? (n_str_tiles - wave + NW - 1) / NW : 0;
  for (int c0 = 0; c0 < nr; c0 += SK_RT) {
    const int nc = min(SK_RT, nr - c0);
    float m[SK_RT], s[SK_RT];
#pragma unroll
    for (int r = 0; r < SK_RT; ++r) {
      m[r] = NEG_BIG;
      s[r] = 0.f;
    }
    for (int k0 = 0; k0 < ks; k0 += SCH) {
      // SCH streamed fragments and their column terms stay in registers for all
      // resident tiles; slots past the wave's last tile repeat a valid tile with
      // w = NEG_BIG, so they add exp2(-huge) = 0 without a branch.
      typename M::Frag af[SCH];
      f32x4 w[SCH];
#pragma unroll
      for (int k = 0; k < SCH; ++k) {
        const bool live = k0 + k < ks;
        const int st = live ? wave + NW * (k0 + k) : wave;
        M::load(af[k], str_lds + (size_t)(st * 16 + (lane & 15)) * DP, lane);
        w[k] = *reinterpret_cast<const f32x4*>(w2 + st * 16 + 4 * g);
        if (!live) w[k] = f32x4{NEG_BIG, NEG_BIG, NEG_BIG, NEG_BIG};
      }
#pragma unroll
      for (int r = 0; r < SK_RT; ++r) {
        if (r >= nc) continue;
        typename M::Frag bf;
        M::load(bf, res_lds + (size_t)((rt0 + c0 + r) * 16 + (lane & 15)) * DP, lane);
        f32x4 cinit = f32x4{0.f, 0.f, 0.f, 0.f};
        if (!ONLINE) {
          const float ci = -shift2[(c0 + r) * 16 + (lane & 15)] * isc;
          cinit = f32x4{ci, ci, ci, ci};
        }
        f32x4 bv[SCH];
        if (GENERAL) {  // dead slots repeat tile `wave` (their w is NEG_BIG)
          int s0[SCH];
#pragma unroll
          for (int k = 0; k < SCH; ++k) s0[k] = (k0 + k < ks ? wave + NW * (k0 + k) : wave) * 16 + 4 * g;
          bias.template quads<TRANS>((rt0 + c0 + r) * 16 + (lane & 15), s0, bv);
        }
        f32x4 x[SCH];
#pragma unroll
        for (int k = 0; k < SCH; ++k) x[k] = M::qk(af[k], bf, cinit);  // independent MFMAs
#pragma unroll
        for (int k = 0; k < SCH; ++k)
#pragma unroll
          for (int e = 0; e < 4; ++e) {  // no `+ 0.f` without a bias: the add is not folded
            const float xv = __builtin_fmaf(x[k][e], sc, w[k][e]);
            x[k][e] = GENERAL ? xv + bv[k][e] : xv;
          }
        if (ONLINE) {
          float tm = NEG_BIG;
#pragma unroll
          for (int k = 0; k < SCH; ++k) tm = fmaxf(tm, fmaxf(fmaxf(x[k][0], x[k][1]), fmaxf(x[k][2], x[k][3])));
          const float mn = fmaxf(m[r], tm);
          float acc_s = s[r] * fast_exp2(m[r] - mn);
#pragma unroll
          for (int k = 0; k < SCH; ++k)
            acc_s += (fast_exp2(x[k][0] - mn) + fast_exp2(x[k][1] - mn)) + (fast_exp2(x[k][2] - mn) + fast_exp2(x[k][3] - mn));
          s[r] = acc_s;
          m[r] = mn;
        } else {
          float acc_s = 0.f;
#pragma unroll
          for (int k = 0; k < SCH; ++k)
            acc_s += (fast_exp2(x[k][0]) + fast_exp2(x[k][1])) + (fast_exp2(x[k][2]) + fast_exp2(x[k][3]));
          s[r] += acc_s;
        }
      }
    }
#pragma unroll
    for (int r = 0; r < SK_RT; ++r) {
      if (r < nc) {
        float mm = 0.f, ss;
        if (ONLINE) {
          mm = max_groups(m[r]);
          ss = sum_groups(s[r] * fast_exp2(m[r] - mm));
        } else {
          ss = sum_groups(s[r]);
        }
        if (lane < 16) {
          scratch[(wave * SK_RT + r) * 16 + lane] = mm;
          scratch[NW * SK_RT * 16 + (wave * SK_RT + r) * 16 + lane] = ss;
        }
      }
    }
    // the change word of the coming gather is cleared before the barrier, so no
    // wave's post-barrier atomic can precede the clear
    if (s_reset && threadIdx.x == 0) *s_reset = 0u;
    __syncthreads();
    if ((int)threadIdx.x < nc * 16) {
      const int q = threadIdx.x;
      const int r = q >> 4, l = q & 15;
      float res;
      if (ONLINE) {
        float mm = NEG_BIG;
#pragma unroll
        for (int w = 0; w < NW; ++w) mm = fmaxf(mm, scratch[(w * SK_RT + r) * 16 + l]);
        float ss = 0.f;
#pragma unroll
        for (int w = 0; w < NW; ++w)
          ss += scratch[NW * SK_RT * 16 + (w * SK_RT + r) * 16 + l] * fast_exp2(scratch[(w * SK_RT + r) * 16 + l] - mm);
        res = mm + fast_log2(ss);
        if (mx2) mx2[c0 * 16 + q] = mm;
      } else {
        float ss = 0.f;
#pragma unroll
        for (int w = 0; w < NW; ++w) ss += scratch[NW * SK_RT * 16 + (w * SK_RT + r) * 16 + l];
        res = shift2[c0 * 16 + q] + fast_log2(ss);
      }
      lse2[c0 * 16 + q] = res;
      publish(c0 * 16 + q, res);
    }
    __syncthreads();
  }
}

struct NoPublish {
  __device__ __forceinline__ void operator()(int, float) const {}
};

// ---------------------------------------------------------------------------
// Fixed-shift LSE sweep of resident storage, the sweep of every Sinkhorn
// half-iteration after the first.  Same result as lse_sweep<..., ONLINE = false>
// (lse2[q] = shift2[q] + log2 sum_j exp2(x_qj - shift2[q]), in place), organised
// for issue rate:
//  * NR resident tiles per call, known at compile time; their fragments and
//    shifts are loaded once;
//  * a wave's streamed tiles st = wave + NW k are read from one base address at
//    compile-time offsets, SCH per group; slots past the last tile read padding
//    rows (zero operands) whose column term is NEG_BIG, so no slot is tested
//    (the caller pads res/str to lean_rows() rows and w2 with NEG_BIG);
//  * all MFMAs of a group are issued before the exponentials, and each resident
//    tile's 4 * SCH exponentials are summed as a tree.
// A sweep-only microbenchmark at the headline member shape (3 resident tiles
// against 48 streamed tiles, bf16, d = 32) measured 1.80 us against 2.34 us for
// lse_sweep, and 0.96 against 1.72 us at 2 against 32.
template <typename T, int DP> constexpr int lean_sch() {
  return (sizeof(T) == 2 && DP == 32) ? 6 : ((sizeof(T) == 4 && DP == 64) ? 2 : 4);
}
// Rows of a resident Q / K array (and entries of a potential vector) that the
// lean sweep may read: Np rounded up to whole groups of NW * SCH streamed tiles.
template <int NT> __host__ __device__ inline int lean_rows(int Np, int sch) {
  const int unit = (NT / WAVE) * sch * 16;
  return ((Np + unit - 1) / unit) * unit;
}

template <int N>
__device__ __forceinline__ float tree_sum(float (&v)[N]) {
#pragma unroll
  for (int w = 1; w < N; w *= 2)
#pragma unroll
    for (int i = 0; i + w < N; i += 2 * w) v[i] += v[i + w];
  return v[0];
}

// One chunk of NR resident tiles (absolute tiles rt0 .. rt0 + NR - 1, local rows
// q0 .. q0 + 16 NR - 1) against `groups` groups of SCH streamed slots per wave.
template <int NT, typename T, int DP, int NR, int SCH, bool GENERAL, bool TRANS, typename Pub>
__device__ __forceinline__ void lean_chunk(const T* __restrict__ res, const T* __restrict__ str,
                                           const float* __restrict__ w2, int groups, int rt0, int q0, float sc,
                                           const Bias& bias, float* lse, float* scratch, unsigned* s_reset,
                                           Pub publish) {
  using M = Mfma<T, DP>;
  using Frag = typename M::Frag;
  constexpr int NW = NT / WAVE;
  const int lane = threadIdx.x & (WAVE - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE);
  const int g = lane >> 4;
  const float isc = 1.f / sc;
  Frag bf[NR];
  f32x4 ci[NR];
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    M::load(bf[r], res + (size_t)((rt0 + r) * 16 + (lane & 15)) * DP, lane);
    const float c = -lse[q0 + r * 16 + (lane & 15)] * isc;
    ci[r] = f32x4{c, c, c, c};
  }
  float s[NR];
#pragma unroll
  for (int r = 0; r < NR; ++r) s[r] = 0.f;
  const T* sb = str + (size_t)(wave * 16 + (lane & 15)) * DP;
  const float* wb = w2 + wave * 16 + 4 * g;
  for (int kg = 0; kg < groups; ++kg) {
    Frag af[SCH];
    f32x4 w[SCH];
#pragma unroll
    for (int k = 0; k < SCH; ++k) {
      M::load(af[k], sb + (size_t)(kg * SCH + k) * NW * 16 * DP, lane);
      w[k] = *reinterpret_cast<const f32x4*>(wb + (kg * SCH + k) * NW * 16);
    }
    f32x4 x[NR][SCH];
#pragma unroll
    for (int r = 0; r < NR; ++r)
#pragma unroll
      for (int k = 0; k < SCH; ++k) x[r][k] = M::qk(af[k], bf[r], ci[r]);  // independent MFMAs
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      f32x4 bv[SCH];
      if (GENERAL) {
        // padding slots index past the last tile: clamp inside the padded arrays
        // (their w is NEG_BIG, so the bias value is irrelevant)
        int s0[SCH];
#pragma unroll
        for (int k = 0; k < SCH; ++k) s0[k] = min((wave + NW * (kg * SCH + k)) * 16 + 4 * g, bias.Np - 4);
        bias.template quads<TRANS>((rt0 + r) * 16 + (lane & 15), s0, bv);
      }
      float e[4 * SCH];
#pragma unroll
      for (int k = 0; k < SCH; ++k)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float xv = __builtin_fmaf(x[r][k][q], sc, w[k][q]);
          e[4 * k + q] = fast_exp2(GENERAL ? xv + bv[k][q] : xv);
        }
      s[r] += tree_sum(e);
    }
  }
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    const float ss = sum_groups(s[r]);
    if (lane < 16) scratch[(wave * NR + r) * 16 + lane] = ss;
  }
  // the change word of the coming gather is cleared before the barrier, so no
  // wave's post-barrier atomic can precede the clear
  if (s_reset && threadIdx.x == 0) *s_reset = 0u;
  lds_barrier();
  if ((int)threadIdx.x < NR * 16) {
    const int q = threadIdx.x, r = q >> 4, l = q & 15;
    float ss = 0.f;
#pragma unroll
    for (int w_ = 0; w_ < NW; ++w_) ss += scratch[(w_ * NR + r) * 16 + l];
    const float v = lse[q0 + q] + fast_log2(ss);
    lse[q0 + q] = v;
    publish(q0 + q, v);
  }
  // the published words complete on their own: the coming gather polls them
  lds_barrier();
}

// Chunks of at most 4 resident tiles (2 with a bias: its per-element values would
// not fit in registers beside 4 tiles' accumulators).
template <int NT, typename T, int DP, int SCH, bool GENERAL, bool TRANS, typename Pub>
__device__ __forceinline__ void lean_chunks(const T* res, const T* str, const float* w2, int groups, int t0, int nr,
                                            float sc, const Bias& bias, float* lse, float* scratch,
                                            unsigned* s_reset, Pub publish) {
  constexpr int CMAX = GENERAL ? 2 : 4;
  for (int c0 = 0; c0 < nr; c0 += CMAX) {
    const int nc = min(CMAX, nr - c0);
    if (CMAX == 4 && nc == 4)
      lean_chunk<NT, T, DP, CMAX, SCH, GENERAL, TRANS>(res, str, w2, groups, t0 + c0, c0 * 16, sc, bias, lse, scratch,
                                                    s_reset, publish);
    else if (CMAX == 4 && nc == 3)
      lean_chunk<NT, T, DP, CMAX - 1, SCH, GENERAL, TRANS>(res, str, w2, groups, t0 + c0, c0 * 16, sc, bias, lse, scratch,
                                                    s_reset, publish);
    else if (nc == 2)
      lean_chunk<NT, T, DP, 2, SCH, GENERAL, TRANS>(res, str, w2, groups, t0 + c0, c0 * 16, sc, bias, lse, scratch,
                                                    s_reset, publish);
    else
      lean_chunk<NT, T, DP, 1, SCH, GENERAL, TRANS>(res, str, w2, groups, t0 + c0, c0 * 16, sc, bias, lse, scratch,
                                                    s_reset, publish);
  }
}

// Resident fixed-shift sweep over n_str_tiles streamed tiles for resident tiles
// [t0, t0 + nr): lse (local rows) holds the shift on entry and the result on exit.
// For (bf16, DP 32) a wave with at most 4 streamed tiles takes groups of 4 slots,
// else of 6.  res, str and w2 must hold lean_rows<NT>(Np, lean_sch<T, DP>()) rows.
template <int NT, typename T, int DP, bool GENERAL, bool TRANS, typename Pub>
__device__ __forceinline__ void lean_sweep(const T* res, const T* str, const float* w2, int n_str_tiles, int t0,
                                           int nr, float sc, const Bias& bias, float* lse, float* scratch,
                                           unsigned* s_reset, Pub publish) {
  constexpr int NW = NT / WAVE;
  constexpr int SMAX = lean_sch<T, DP>();
  const int ks = (n_str_tiles + NW - 1) / NW;  // streamed tiles of the busiest wave
  if (SMAX == 6 && ks <= 4)
    lean_chunks<NT, T, DP, 4, GENERAL, TRANS>(res, str, w2, 1, t0, nr, sc, bias, lse, scratch, s_reset, publish);
  else
    lean_chunks<NT, T, DP, SMAX, GENERAL, TRANS>(res, str, w2, (ks + SMAX - 1) / SMAX, t0, nr, sc, bias, lse,
                                                 scratch, s_reset, publish);
}

// ---------------------------------------------------------------------------
// Potentials added to logits held in registers (register storage): a rank-2 bf16
// MFMA whose operands carry three-part splits of the potentials.
// Three-part bf16 split of x in the first three slots (hi + mid + lo = x to fp32
// rounding); slot 3 is zero.
__device__ __forceinline__ bf16x4 split3(float x) {
  const bf16 h = (bf16)x;
  const float r1 = x - (float)h;
  const bf16 m = (bf16)r1;
  const bf16 l = (bf16)(r1 - (float)m);
  return bf16x4{h, m, l, (bf16)0.f};
}

// D = S + A B^T on v_mfma_f32_16x16x16_bf16: lane l supplies A[m = l%16][k = 4(l/16)..+3]
// and B[n = l%16][same k], and holds D[4(l/16) + e][l%16] (the layout of S).
__device__ __forceinline__ f32x4 mfma_rank(bf16x4 a, bf16x4 b, f32x4 s) {
  typedef short s16x4 __attribute__((ext_vector_type(4)));
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, a), __builtin_bit_cast(s16x4, b), s,
                                                   0, 0, 0);
}

// Operands of the rank-2 update.  The column side (A, m = plan column j) carries the
// column term's parts in lane group 0 and ones in group 1; the row side (B, n = plan
// row i) carries ones in group 0 and the row term's parts in group 1; groups 2-3 are
// zero.  So sum_k A[j][k] B[i][k] = colterm_j + rowterm_i.
__device__ __forceinline__ bf16x4 blk_col_operand(const bf16x4* parts, int tile, int lane) {
  const int g = lane >> 4;
  const bf16x4 one = {(bf16)1.f, (bf16)1.f, (bf16)1.f, (bf16)0.f};
  const bf16x4 zero = {(bf16)0.f, (bf16)0.f, (bf16)0.f, (bf16)0.f};
  const bf16x4 p = parts[tile * 16 + (lane & 15)];
  return g == 0 ? p : (g == 1 ? one : zero);
}
__device__ __forceinline__ bf16x4 blk_row_operand(const bf16x4* parts, int tile, int lane) {
  const int g = lane >> 4;
  const bf16x4 one = {(bf16)1.f, (bf16)1.f, (bf16)1.f, (bf16)0.f};
  const bf16x4 zero = {(bf16)0.f, (bf16)0.f, (bf16)0.f, (bf16)0.f};
  const bf16x4 p = parts[tile * 16 + (lane & 15)];
  return g == 1 ? p : (g == 0 ? one : zero);
}

// acc += P V for one 16x16 pair held in the accumulator layout of S (lane: plan row
// l % 16, plan columns 4(l/16) + e of the streamed tile), giving the output layout
// (lane: rows 4(l/16) + e, V column l % 16).  vt: V^T row (c0 + l%16) at column
// st*16 + 4(l/16).  bf16: P as a hi + lo pair of bf16 A operands (two
// 16x16x16 MFMAs on the same V operand); fp32: four 16x16x4 steps.
template <typename T> __device__ __forceinline__ f32x4 reg_pv(const float (&p)[4], const T* vt, f32x4 acc);
template <> __device__ __forceinline__ f32x4 reg_pv<bf16>(const float (&p)[4], const bf16* vt, f32x4 acc) {
  bf16x4 hi, lo;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    hi[e] = (bf16)p[e];
    lo[e] = (bf16)(p[e] - (float)hi[e]);
  }
  const bf16x4 v = *reinterpret_cast<const bf16x4*>(vt);
  acc = mfma_rank(hi, v, acc);
  return mfma_rank(lo, v, acc);
}
template <> __device__ __forceinline__ f32x4 reg_pv<float>(const float (&p)[4], const float* vt, f32x4 acc) {
  const f32x4 v = *reinterpret_cast<const f32x4*>(vt);
#pragma unroll
  for (int e = 0; e < 4; ++e) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(p[e], v[e], acc, 0, 0, 0);
  return acc;
}

// ---------------------------------------------------------------------------
// Dataflow half-iterations of resident storage.  A wave of a lean sweep reads the
// potentials of its own streamed tiles st = wave + NW k only, so it needs no other
// wave's gather: it polls those words itself (wave_gather) and starts its sweep as
// soon as they carry the previous half-iteration's tag.  The fixed / online choice
// is the wave's own (the largest change over its tiles), and each wave leaves an
// absolute log2 partial per resident row; the partials of the NW waves are combined
// after the chunk's barrier (flow_chunk), the only barrier of a half-iteration
// with at most 4 resident tiles (2 with a bias).

// Polls the words of this wave's streamed tiles (entries i < n) until they carry
// `tag`, writes dst[i] = word * log2 e (NEG_BIG for a masked entry), and its split
// parts[i] = split3(dst[i]) if parts is given, and sets dmax, in every lane, to the
// largest |change| over the wave's valid entries (+inf for a NaN).  Returns false,
// uniformly over the wave, if a wait expired (then the error has been raised).
template <int NW>
__device__ __forceinline__ bool wave_gather(const uint64_t* buf, int n, int n_tiles, uint32_t tag, float* dst,
                                            const unsigned char* valid, ErrRef err, float& dmax,
                                            bf16x4* parts = nullptr) {
  const int lane = threadIdx.x & (WAVE - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE);
  const int nwords = wave < n_tiles ? ((n_tiles - 1 - wave) / NW + 1) * 16 : 0;
  float dm = 0.f;
  bool ok = true;
  for (int base = 0; base < nwords && ok; base += 2 * WAVE) {
    int idx[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int e = base + k * WAVE + lane;
      const int i = (wave + NW * (e >> 4)) * 16 + (e & 15);
      idx[k] = (e < nwords && i < n) ? i : -1;
    }
    ok = poll_words<2>(buf, idx, tag, err, [&](int k, uint64_t w) {
      const int i = idx[k];
      float nv = NEG_BIG;
      if (valid[i]) {
        nv = __uint_as_float((uint32_t)(w >> 32)) * LOG2E;
        dm = fmaxf(dm, fabsf(nv - dst[i]));
      }
      dst[i] = nv;
      if (parts) parts[i] = split3(nv);
    });
    ok = wave_max_u32(ok ? 0u : 1u) == 0u;
  }
  dmax = __uint_as_float(wave_max_u32(dm == dm ? __float_as_uint(dm) : 0x7f800000u));
  return ok;
}

// Combine of the NW wave partials part[q * NW + w] of the nr * 16 rows q (threads
// q < 16 nr): lse[q] = m + log2 sum_w exp2(p_w - m), m = max_w p_w, in wave order,
// then publish(q, lse[q]).  A row's partials are adjacent: 16-byte reads.
template <int NW, typename Pub>
__device__ __forceinline__ void flow_combine(const float* part, int nr, float* lse, Pub publish) {
  static_assert(NW % 4 == 0, "partials are read 4 at a time");
  if ((int)threadIdx.x < nr * 16) {
    const int q = threadIdx.x;
    float p[NW];
#pragma unroll
    for (int w4 = 0; w4 < NW; w4 += 4) {
      const f32x4 v = *reinterpret_cast<const f32x4*>(part + q * NW + w4);
#pragma unroll
      for (int k = 0; k < 4; ++k) p[w4 + k] = v[k];
    }
    float m = p[0];
#pragma unroll
    for (int w_ = 1; w_ < NW; ++w_) m = fmaxf(m, p[w_]);
    float ss = 0.f;
#pragma unroll
    for (int w_ = 0; w_ < NW; ++w_) ss += fast_exp2(p[w_] - m);
    const float v = m + fast_log2(ss);
    lse[q] = v;
    publish(q, v);
  }
}

// One chunk of NR resident tiles (absolute rt0.., local rows q0..) in dataflow form.
// Each wave takes the shift of its partial from lse[q] (fixed: every term of its
// tiles is then <= 2^delta, delta the wave's largest potential change) or, online,
// from a first pass over its tiles (the row maximum of its streamed entries), and
// writes p_w = shift + log2 sum_(its j) exp2(x_qj - shift) (NEG_BIG for an empty
// sum) to part (flow_combine's layout).  After the barrier the threads of the chunk's rows combine the NW
// partials in wave order, lse = m + log2 sum_w exp2(p_w - m) with m = max_w p_w,
// store it and publish it.  part must not be written again before every wave has
// passed one more barrier (flow_sweep alternates two slots).
template <int NT, typename T, int DP, int NR, int SCH, bool GENERAL, bool TRANS, typename Pub>
__device__ __forceinline__ void flow_chunk(bool online, const T* __restrict__ res, const T* __restrict__ str,
                                           const float* __restrict__ w2, int groups, int rt0, int q0, float sc,
                                           const Bias& bias, float* lse, float* part, Pub publish) {
  using M = Mfma<T, DP>;
  using Frag = typename M::Frag;
  constexpr int NW = NT / WAVE;
  const int lane = threadIdx.x & (WAVE - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE);
  const int g = lane >> 4;
  const float isc = 1.f / sc;
  Frag bf[NR];
#pragma unroll
  for (int r = 0; r < NR; ++r) M::load(bf[r], res + (size_t)((rt0 + r) * 16 + (lane & 15)) * DP, lane);
  const T* sb = str + (size_t)(wave * 16 + (lane & 15)) * DP;
  const float* wb = w2 + wave * 16 + 4 * g;
  // x_qj - shift_q for the wave's streamed entries (MFMA C operand -shift / sc), in
  // groups of SCH tiles, handed to f(r, e[4 SCH]) per resident tile r
  auto pass = [&](const f32x4(&ci)[NR], auto&& f) __attribute__((always_inline)) {
    for (int kg = 0; kg < groups; ++kg) {
      Frag af[SCH];
      f32x4 w[SCH];
#pragma unroll
      for (int k = 0; k < SCH; ++k) {
        M::load(af[k], sb + (size_t)(kg * SCH + k) * NW * 16 * DP, lane);
        w[k] = *reinterpret_cast<const f32x4*>(wb + (kg * SCH + k) * NW * 16);
      }
      f32x4 x[NR][SCH];
#pragma unroll
      for (int r = 0; r < NR; ++r)
#pragma unroll
        for (int k = 0; k < SCH; ++k) x[r][k] = M::qk(af[k], bf[r], ci[r]);
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        f32x4 bv[SCH];
        if (GENERAL) {
          int s0[SCH];
#pragma unroll
          for (int k = 0; k < SCH; ++k) s0[k] = min((wave + NW * (kg * SCH + k)) * 16 + 4 * g, bias.Np - 4);
          bias.template quads<TRANS>((rt0 + r) * 16 + (lane & 15), s0, bv);
        }
        float e[4 * SCH];
#pragma unroll
        for (int k = 0; k < SCH; ++k)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const float xv = __builtin_fmaf(x[r][k][q], sc, w[k][q]);
            e[4 * k + q] = GENERAL ? xv + bv[k][q] : xv;
          }
        f(r, e);
      }
    }
  };
  float sh[NR];
  if (online) {
    f32x4 zero[NR];
    float m[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      zero[r] = f32x4{0.f, 0.f, 0.f, 0.f};
      m[r] = NEG_BIG;
    }
    pass(zero, [&](int r, float(&e)[4 * SCH]) {
#pragma unroll
      for (int w_ = 1; w_ < 4 * SCH; w_ *= 2)
#pragma unroll
        for (int i = 0; i + w_ < 4 * SCH; i += 2 * w_) e[i] = fmaxf(e[i], e[i + w_]);
      m[r] = fmaxf(m[r], e[0]);
    });
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      const float mr = max_groups(m[r]);
      sh[r] = mr > 0.5f * NEG_BIG ? mr : 0.f;  // no live entry: the sum is 0 whatever the shift
    }
  } else {
#pragma unroll
    for (int r = 0; r < NR; ++r) sh[r] = lse[q0 + r * 16 + (lane & 15)];
  }
  f32x4 ci[NR];
  float s[NR];
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    const float c = -sh[r] * isc;
    ci[r] = f32x4{c, c, c, c};
    s[r] = 0.f;
  }
  pass(ci, [&](int r, float(&e)[4 * SCH]) {
#pragma unroll
    for (int i = 0; i < 4 * SCH; ++i) e[i] = fast_exp2(e[i]);
    s[r] += tree_sum(e);
  });
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    const float ss = sum_groups(s[r]);
    if (lane < 16) part[(r * 16 + lane) * NW + wave] = ss > 0.f ? sh[r] + fast_log2(ss) : NEG_BIG;
  }
  lds_barrier();
  flow_combine<NW>(part, NR, lse + q0, [&](int q, float v) { publish(q0 + q, v); });
}

// Dataflow sweep of resident tiles [t0, t0 + nr) against n_str_tiles streamed tiles
// (the lean sweep's layout and padding): chunks of at most SK_RT resident tiles (2
// with a bias), partial slots alternating with the caller's chunk counter, which
// every wave advances alike.  lse holds the fixed shifts on entry (unused online)
// and the combined LSEs on exit (written by the combining threads only: visible to
// the other waves after their next barrier).
template <int NT, typename T, int DP, bool GENERAL, bool TRANS, typename Pub>
__device__ __forceinline__ void flow_sweep(bool online, const T* res, const T* str, const float* w2, int n_str_tiles,
                                           int t0, int nr, float sc, const Bias& bias, float* lse, float* scratch,
                                           int& chunk, Pub publish) {
  constexpr int NW = NT / WAVE;
  constexpr int SMAX = lean_sch<T, DP>();
  constexpr int CMAX = GENERAL ? 2 : SK_RT;
  const int ks = (n_str_tiles + NW - 1) / NW;
  const bool small = SMAX == 6 && ks <= 4;
  const int groups = small ? 1 : (ks + SMAX - 1) / SMAX;
  for (int c0 = 0; c0 < nr; c0 += CMAX, ++chunk) {
    float* part = scratch + (chunk & 1) * (NW * SK_RT * 16);
    const int nc = min(CMAX, nr - c0);
    const int rt0 = t0 + c0, q0 = c0 * 16;
#define DFL_FLOW(NRV, SCHV)                                                                                      \
  flow_chunk<NT, T, DP, NRV, SCHV, GENERAL, TRANS>(online, res, str, w2, groups, rt0, q0, sc, bias, lse, part, \
                                                   publish)
    if (small) {
      if (CMAX == 4 && nc == 4) DFL_FLOW(CMAX, 4);
      else if (CMAX == 4 && nc == 3) DFL_FLOW(CMAX - 1, 4);
      else if (nc == 2) DFL_FLOW(2, 4);
      else DFL_FLOW(1, 4);
    } else {
      if (CMAX == 4 && nc == 4) DFL_FLOW(CMAX, SMAX);
      else if (CMAX == 4 && nc == 3) DFL_FLOW(CMAX - 1, SMAX);
      else if (nc == 2) DFL_FLOW(2, SMAX);
      else DFL_FLOW(1, SMAX);
    }
#undef DFL_FLOW
  }
}

// ---------------------------------------------------------------------------
// Register storage of the resident layout.  A wave keeps the logits of its (resident
// tile r, streamed slot k) pairs in VGPRs, S[r KS + k] for r < nr, k < KS (streamed
// tile st = wave + NW k; slots of tiles the wave does not have hold NEG_BIG), computed
// once per launch.  A sweep adds the potentials with one rank-2 MFMA per pair
// (streamed term in the A operand, -shift of the resident row in B) and sums exp2;
// each row's partial p_w goes to part as in flow_chunk.  Online (the first sweep, or
// a wave whose streamed potentials moved by more than the fixed-shift bound) takes
// the row maxima of its pairs first and uses them as its shifts.
//   colp : split parts of the streamed potentials (by absolute streamed index)
//   rowp : split parts of -shift of the resident rows (local), for the fixed mode
//   shift: the fixed shifts (local rows)
// pmax (online only): the wave's row maxima, pmax[(r 16 + l) NW + wave], NEG_BIG
// where the wave has no live entry.
template <int KS, int NRM, int NW>
__device__ __forceinline__ void reg_sweep(bool online, const f32x4 (&S)[NRM * KS], int nr, const bf16x4* colp,
                                          const bf16x4* rowp, const float* shift, float* part,
                                          float* pmax = nullptr) {
  const int lane = threadIdx.x & (WAVE - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE);
  const int g = lane >> 4;
  const bf16x4 one = {(bf16)1.f, (bf16)1.f, (bf16)1.f, (bf16)0.f};
  const bf16x4 zero = {(bf16)0.f, (bf16)0.f, (bf16)0.f, (bf16)0.f};
  bf16x4 A[KS];
#pragma unroll
  for (int k = 0; k < KS; ++k) A[k] = blk_col_operand(colp, wave + NW * k, lane);
#pragma unroll
  for (int r = 0; r < NRM; ++r) {
    if (r < nr) {
      float sh;
      bf16x4 Bv;
      if (online) {
        const bf16x4 b0 = g == 0 ? one : zero;  // row term 0
        float m = NEG_BIG;
#pragma unroll
        for (int k = 0; k < KS; ++k) {
          const f32x4 x = mfma_rank(A[k], b0, S[r * KS + k]);
          m = fmaxf(m, fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3])));
        }
        m = max_groups(m);
        if (pmax && lane < 16) pmax[(r * 16 + lane) * NW + wave] = m;
        sh = m > 0.5f * NEG_BIG ? m : 0.f;  // no live entry: the sum is 0 whatever the shift
        Bv = g == 1 ? split3(-sh) : b0;
      } else {
        sh = shift[r * 16 + (lane & 15)];
        Bv = blk_row_operand(rowp, r, lane);
      }
      float e[4 * KS];
      // software pipelined: the MFMA of pair k + 1 issues before the exponentials of
      // pair k (two accumulators live), so the exponentials rarely wait on an MFMA
      f32x4 xc = mfma_rank(A[0], Bv, S[r * KS]);
#pragma unroll
      for (int k = 0; k < KS; ++k) {
        f32x4 xn;
        if (k + 1 < KS) xn = mfma_rank(A[k + 1], Bv, S[r * KS + k + 1]);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int q = 0; q < 4; ++q) e[4 * k + q] = fast_exp2(xc[q]);
        __builtin_amdgcn_sched_barrier(0);
        if (k + 1 < KS) xc = xn;
      }
      const float ss = sum_groups(tree_sum(e));
      if (lane < 16) part[(r * 16 + lane) * NW + wave] = ss > 0.f ? sh + fast_log2(ss) : NEG_BIG;
    }
  }
}

// Exchange-placement agreement of a group.  At the start of a launch every member
// publishes whether it runs on its expected XCD (publish_placement); after the
// launch's first gather, by when every member has published, each member reads
// the G words (read_placement): plain-store publishing (xch_put_local) is used
// only if all members are placed.  The answer is uniform over the block and
// identical in every member.  Returns false (uniformly) if a wait expires.
__device__ __forceinline__ void publish_placement(uint64_t* pw, int member, uint32_t salt) {
  if (threadIdx.x == 0) xch_put(pw + member, xcc_placed() ? 1.f : 0.f, salt << 12);
}
// Members that own no tiles (stripe empty: n_tiles < G) return before publishing
// and are skipped.
__device__ __forceinline__ bool read_placement(const uint64_t* pw, int G, int n_tiles, uint32_t salt, ErrRef err,
                                               int* s_flag, int* s_local) {
  const uint32_t tag = salt << 12;
  const int t = threadIdx.x;
  if (t < G && (long long)n_tiles * (t + 1) / G > (long long)n_tiles * t / G) {
    uint32_t spins = 0;
    while (true) {
      const uint64_t w = __hip_atomic_load(const_cast<uint64_t*>(pw + t), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if ((uint32_t)w == tag) {
        if (__uint_as_float((uint32_t)(w >> 32)) != 1.f) *s_local = 0;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
      if (++spins > err.spin_limit) { raise_error(err, salt, 2u); *s_flag = 1; break; }
      if ((spins & 255u) == 0u && error_raised(err, salt)) { *s_flag = 1; break; }
    }
  }
  __syncthreads();
  return *s_flag == 0;
}

// Workgroup -> (group, member).  Workgroups are dispatched round-robin over the
// 8 XCDs (id % 8), so the members of one group are taken from a single XCD:
// local index l = id / 8 on XCD x = id % 8, slot s = l / G, member = l % G,
// group = 8 s + x.  Exchanges between workgroups of one XCD measured ~2.5x
// faster than across XCDs; the mapping affects speed only, never correctness.
// Returns false for surplus workgroups (group >= n_groups), which own nothing.
__device__ __forceinline__ bool group_of(int n_groups, int G, int& group, int& member) {
  const int id = blockIdx.x, x = id & 7, l = id >> 3;
  member = l % G;
  group = 8 * (l / G) + x;
  return group < n_groups;
}

// Stripe of 16-row tiles owned by `member` out of G.
__device__ __forceinline__ void stripe(int n_tiles, int member, int G, int& t0, int& t1) {
  t0 = (int)((long long)n_tiles * member / G);
  t1 = (int)((long long)n_tiles * (member + 1) / G);
}

// ---------------------------------------------------------------------------
// Stream mode (sequences whose Q and K do not fit in LDS).
//
// Only the workgroup's own stripe of resident rows sits in LDS ([nr*16][DP],
// local tile index).  The streamed operand is read straight from a zero-padded
// copy in global memory ([Np][DP], rows >= n and masked rows zero), which stays
// L2-resident.  A wave takes streamed tiles st = wave + NW*k and keeps the
// accumulators of up to STREAM_RB resident tiles in registers, so each streamed
// tile is fetched once per batch of STREAM_RB resident tiles; the next group of
// SCH streamed fragments is in flight while the current group is consumed.
constexpr int STREAM_RB = 8;
// Streamed fragments per group (double-buffered in registers).  The weighted
// sum also carries the streamed weights, so it takes half the group where
// fragments are wide (d = 64 or fp32).
template <typename T, int DP, int KIND>
constexpr int stream_sch() {
  return (KIND == 2 && (DP == 64 || sizeof(T) == 4)) || (sizeof(T) == 4 && DP == 64) ? 2 : 4;
}
template <int NT> constexpr int stream_scratch() { return 2 * (NT / WAVE) * STREAM_RB * 16; }

enum { SW_LSE_ONLINE = 0, SW_LSE_FIXED = 1, SW_WSUM = 2 };

// For every local resident row q in [0, nr*16), with
//   x_qj = sc * <res_q, str_j> + w2_j (+ bias(i_q, j)),  i_q = 16*t0 + q:
//   SW_LSE_ONLINE: out[q] = log2 sum_j exp2(x_qj)            (running max; mx[q] = max_j x_qj if mx)
//   SW_LSE_FIXED : out[q] = c_q + log2 sum_j exp2(x_qj - c_q) (c_q = cres[q]; caller guarantees range)
//   SW_WSUM      : out[q] = sum_j exp2(x_qj + cres[q]) z_j    (every exponent <= 0)
// out may alias cres.  publish(q, out_q) runs on the thread that finishes row q.
// TRANS: the streamed index is the plan's row index (only matters for the bias).
// Called by the whole block.
template <int NT, typename T, int DP, int KIND, bool GENERAL, bool TRANS, typename Pub>
__device__ __forceinline__ void stream_sweep(const T* __restrict__ res, const T* __restrict__ str,
                                             const float* __restrict__ w2, const float* __restrict__ zv,
                                             int n_str_tiles, int t0, int nr, float sc,
                                             const float* __restrict__ cres, const Bias& bias, float* out,
                                             float* mx, float* scratch, unsigned* s_reset, Pub publish) {
  using M = Mfma<T, DP>;
  using Frag = typename M::Frag;
  constexpr int NW = NT / WAVE;
  constexpr int RB = STREAM_RB;
  constexpr int SCH = stream_sch<T, DP, KIND>();
  const int lane = threadIdx.x & (WAVE - 1);
  const int wave = threadIdx.x / WAVE;
  const int g = lane >> 4;
  const float isc = 1.f / sc;
  const int ks = wave < n_str_tiles ? (n_str_tiles - wave + NW - 1) / NW : 0;
  {
    // An opaque zero offset on every base pointer: a kernel inlines several
    // instances of this sweep inside its iteration loop, and without it the
    // compiler hoists each instance's address arithmetic out of that loop,
    // where the sum no longer fits the register file.
    int opq = 0;
    asm volatile("" : "+s"(opq));
    res += opq;
    str += opq;
    w2 += opq;
    zv += opq;
    cres += opq;
  }
  // slots past the wave's last tile repeat tile `wave` with w = NEG_BIG (exp2 -> 0), z = 0
  auto load_group = [&](int k0, Frag* af, f32x4* w, f32x4* z) {
#pragma unroll
    for (int k = 0; k < SCH; ++k) {
      const bool live = k0 + k < ks;
      const int st = live ? wave + NW * (k0 + k) : wave;
      M::load(af[k], str + (size_t)(st * 16 + (lane & 15)) * DP, lane);
      w[k] = *reinterpret_cast<const f32x4*>(w2 + st * 16 + 4 * g);
      if (KIND == SW_WSUM) z[k] = *reinterpret_cast<const f32x4*>(zv + st * 16 + 4 * g);
      if (!live) {
        w[k] = f32x4{NEG_BIG, NEG_BIG, NEG_BIG, NEG_BIG};
        z[k] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
    }
  };
  for (int rb0 = 0; rb0 < nr; rb0 += RB) {
    const int nb = min(RB, nr - rb0);
    float m[RB], s[RB];
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      m[r] = NEG_BIG;
      s[r] = 0.f;
    }
    // Two register sets alternate (the loop is unrolled by two): group k0's fragments
    // sit in one set while group k0 + SCH's loads fill the other, with no copies
    // between them (with a copy at the end of every iteration the compiler waited on
    // the loads just issued before the group's MFMAs).
    Frag fa[SCH], fb[SCH];
    f32x4 wa[SCH], wb[SCH], za[SCH], zb[SCH];
    if (ks > 0) load_group(0, fa, wa, za);
    auto group = [&](int k0, Frag (&af)[SCH], f32x4 (&w)[SCH], f32x4 (&z)[SCH], Frag (&an)[SCH], f32x4 (&wn)[SCH],
                     f32x4 (&zn)[SCH]) __attribute__((always_inline)) {
      const bool more = k0 + SCH < ks;
      if (more) load_group(k0 + SCH, an, wn, zn);
      // The resident fragments are loop-invariant; an opaque row offset keeps
      // them as LDS reads inside the loop instead of RB hoisted register copies.
      int lrow = lane & 15;
      asm volatile("" : "+v"(lrow));
#pragma unroll
      for (int r = 0; r < RB; ++r) {
        if (r < nb) {
          const int q = (rb0 + r) * 16 + (lane & 15);
          Frag bf;
          M::load(bf, res + (size_t)((rb0 + r) * 16 + lrow) * DP, lane);
          f32x4 cinit = f32x4{0.f, 0.f, 0.f, 0.f};
          if (KIND != SW_LSE_ONLINE) {
            const float ci = (KIND == SW_LSE_FIXED ? -cres[q] : cres[q]) * isc;
            cinit = f32x4{ci, ci, ci, ci};
          }
          f32x4 bv[SCH];
          if (GENERAL) {  // dead slots repeat tile `wave` (their w is NEG_BIG)
            int s0[SCH];
#pragma unroll
            for (int k = 0; k < SCH; ++k) s0[k] = (k0 + k < ks ? wave + NW * (k0 + k) : wave) * 16 + 4 * g;
            bias.template quads<TRANS>(t0 * 16 + q, s0, bv);
          }
          f32x4 x[SCH];
#pragma unroll
          for (int k = 0; k < SCH; ++k) x[k] = M::qk(af[k], bf, cinit);  // independent MFMAs
#pragma unroll
          for (int k = 0; k < SCH; ++k)
#pragma unroll
            for (int e = 0; e < 4; ++e) {  // no `+ 0.f` without a bias: the add is not folded
              const float xv = __builtin_fmaf(x[k][e], sc, w[k][e]);
              x[k][e] = GENERAL ? xv + bv[k][e] : xv;
            }
          if (KIND == SW_LSE_ONLINE) {
            float tm = NEG_BIG;
#pragma unroll
            for (int k = 0; k < SCH; ++k) tm = fmaxf(tm, fmaxf(fmaxf(x[k][0], x[k][1]), fmaxf(x[k][2], x[k][3])));
            const float mn = fmaxf(m[r], tm);
            float acc_s = s[r] * fast_exp2(m[r] - mn);
#pragma unroll
            for (int k = 0; k < SCH; ++k)
              acc_s += (fast_exp2(x[k][0] - mn) + fast_exp2(x[k][1] - mn)) +
                       (fast_exp2(x[k][2] - mn) + fast_exp2(x[k][3] - mn));
            s[r] = acc_s;
            m[r] = mn;
          } else if (KIND == SW_LSE_FIXED) {
            float acc_s = 0.f;
#pragma unroll
            for (int k = 0; k < SCH; ++k)
              acc_s += (fast_exp2(x[k][0]) + fast_exp2(x[k][1])) + (fast_exp2(x[k][2]) + fast_exp2(x[k][3]));
            s[r] += acc_s;
          } else {
            float acc_s = 0.f;
#pragma unroll
            for (int k = 0; k < SCH; ++k)
#pragma unroll
              for (int e = 0; e < 4; ++e) acc_s = __builtin_fmaf(fast_exp2(x[k][e]), z[k][e], acc_s);
            s[r] += acc_s;
          }
        }
      }
    };
    if constexpr (KIND != SW_WSUM) {
      for (int k0 = 0; k0 < ks; k0 += 2 * SCH) {
        group(k0, fa, wa, za, fb, wb, zb);
        if (k0 + SCH < ks) group(k0 + SCH, fb, wb, zb, fa, wa, za);
      }
    } else {
      // the weighted sum (inside the backward kernel, at its register limit) keeps one
      // body: the unrolled pair of sets there pushed arrays to scratch
      for (int k0 = 0; k0 < ks; k0 += SCH) {
        group(k0, fa, wa, za, fb, wb, zb);
        if (k0 + SCH < ks) {
#pragma unroll
          for (int k = 0; k < SCH; ++k) {
            fa[k] = fb[k];
            wa[k] = wb[k];
            za[k] = zb[k];
          }
        }
      }
    }
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      if (r < nb) {
        float mm = 0.f, ss;
        if (KIND == SW_LSE_ONLINE) {
          mm = max_groups(m[r]);
          ss = sum_groups(s[r] * fast_exp2(m[r] - mm));
        } else {
          ss = sum_groups(s[r]);
        }
        if (lane < 16) {
          scratch[(wave * RB + r) * 16 + lane] = mm;
          scratch[NW * RB * 16 + (wave * RB + r) * 16 + lane] = ss;
        }
      }
    }
    __syncthreads();
    if (s_reset && threadIdx.x == 0) *s_reset = 0u;
    for (int q = threadIdx.x; q < nb * 16; q += NT) {
      const int r = q >> 4, l = q & 15;
      float res_q;
      if (KIND == SW_LSE_ONLINE) {
        float mm = NEG_BIG;
#pragma unroll
        for (int w_ = 0; w_ < NW; ++w_) mm = fmaxf(mm, scratch[(w_ * RB + r) * 16 + l]);
        float ss = 0.f;
#pragma unroll
        for (int w_ = 0; w_ < NW; ++w_)
          ss += scratch[NW * RB * 16 + (w_ * RB + r) * 16 + l] * fast_exp2(scratch[(w_ * RB + r) * 16 + l] - mm);
        res_q = mm + fast_log2(ss);
        if (mx) mx[rb0 * 16 + q] = mm;
      } else {
        float ss = 0.f;
#pragma unroll
        for (int w_ = 0; w_ < NW; ++w_) ss += scratch[NW * RB * 16 + (w_ * RB + r) * 16 + l];
        res_q = KIND == SW_LSE_FIXED ? cres[rb0 * 16 + q] + fast_log2(ss) : ss;
      }
      out[rb0 * 16 + q] = res_q;
      publish(rb0 * 16 + q, res_q);
    }
    __syncthreads();
  }
}


// One thread per (b, h, i, c), i < Np, c < DP: copies of Q, K (row-major) and V
// (transposed) with zeros on masked rows, rows >= N and columns >= d.
template <typename T, int DP>
__global__ void __launch_bounds__(256) sinkhorn_pad_kernel(PadArgs p) {
  const int N = p.N, d = p.d;
  const int Np = ((N + 31) / 32) * 32;
  const size_t e = (size_t)blockIdx.x * 256 + threadIdx.x;
  const size_t row = e / DP;
  const int c = (int)(e % DP);
  const int bh = (int)(row / Np), i = (int)(row % Np);
  if (bh >= p.B * p.H) return;
  const int b = bh / p.H, h = bh % p.H;
  const bool ok = i < N && (p.mask ? p.mask[(size_t)b * N + i] > 0.5f : true);
  const size_t off = (size_t)b * p.sb + (size_t)h * p.sh + (size_t)i * p.sn + c;
  T qv = from_f32<T>(0.f), kv = from_f32<T>(0.f), vv = from_f32<T>(0.f);
  if (ok && c < d) {
    qv = reinterpret_cast<const T*>(p.q)[off];
    kv = reinterpret_cast<const T*>(p.k)[off];
    if (p.v) vv = reinterpret_cast<const T*>(p.v)[off];
  }
  reinterpret_cast<T*>(p.qp)[row * DP + c] = qv;
  reinterpret_cast<T*>(p.kp)[row * DP + c] = kv;
  if (p.vt) reinterpret_cast<T*>(p.vt)[((size_t)bh * DP + c) * Np + i] = vv;
  if (p.xs_p && h == 0 && c < 3)
    p.xs_p[((size_t)b * Np + i) * 3 + c] = (p.x && i < N) ? p.x[((size_t)b * N + i) * 3 + c] : 0.f;
}

}  // namespace dfl
