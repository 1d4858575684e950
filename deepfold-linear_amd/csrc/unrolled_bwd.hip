// Unrolled backward of the UOT flash-Sinkhorn on gfx950 (persistent per-(b,h)
// workgroup groups, fp32 sweeps).
//
// Restates the GPU-path backward of vv137/deepfold-linear's FlashSinkhornFunction
// (src/deepfold/model/kernels/sinkhorn_kernel.py:2085-2382; its dense autograd
// check is tests/test_triton_fallback_consistency.py:312-430): the exact gradient
// through the K executed iterations of
//   u^k_i = kappa (lmu_i - LSE_j(L_ij + v^{k-1}_j))   (v^{-1} = v_init or 0)   row update
//   v^k_j = kappa (lnu_j - LSE_i(L_ij + u^k_i))                              column update
//   P_ij  = exp(L_ij + v^{K-1}_j - LSE_j(L_ij + v^{K-1}_j))  (row softmax; u cancels)
//   O = P V (gated by sigma(G) outside), xc = P x,
//   L = -C / eps,  C = -q.k / sqrt(d) + pw_h[bins] + w_dist d / (r0 + d),
// on the valid tokens of each sample.  With the plans of each half-iteration
//   s^{R,k} = exp(L + v^{k-1}_j + u^k_i / kappa - lmu_i)   (rows sum to 1)
//   s^{C,k} = exp(L + u^k_i + v^k_j / kappa - lnu_j)       (columns sum to 1)
// and D_i = gO_i.O_i + dxc_i.xc_i, W0 = -P (gO_i.V_j + dxc_i.x_j - D_i):
//   gl_v^{K-1} = -sum_i W0_ij,                 gl_u^k = -kappa s^{C,k} gl_v^k,
//   gl_v^{k-1} = -kappa (s^{R,k})^T gl_u^k,     d lmu = kappa sum_k gl_u^k, d lnu = kappa sum_k gl_v^k,
//   eps dC = W0 + kappa sum_k [ s^{C,k} diag(gl_v^k) + diag(gl_u^k) s^{R,k} ],
//   d v_init = gl_v^{-1}.
// As in the balanced backward (balanced_bwd.hip), each term is produced once in a
// row-owned sweep (dQ, row ends of dx, d pos_weight, d w_dist) and once in a
// column-owned sweep (dK, column ends of dx).  Sweep order:
//   CS_cent: P, W0 -> gl_v^{K-1}, dV, P^T dxc
//   RS(k), k = K-1..0: s^{C,k} gl_v^k (+ diag(gl_u^{k+1}) s^{R,k+1} for k < K-1, W0 for k = K-1) -> gl_u^k
//   CS(k), k = K-1..0: diag(gl_u^k) s^{R,k} + s^{C,k} diag(gl_v^k) -> gl_v^{k-1}
//   RS(-1): diag(gl_u^0) s^{R,0}
// 2K + 2 sweeps, at most two exponentials per element each.
#include <type_traits>

#include "sinkhorn_bwd_kernel.h"

namespace dfl {

constexpr int UNR_NT = 512;
constexpr int UNR_NW = UNR_NT / WAVE;
template <int DP> constexpr int unr_maxt() { return DP <= 32 ? 2 : 1; }
constexpr int UNR_MAXT_ANY = 2;
constexpr int UNR_MAX_LOCAL = 16 * UNR_MAXT_ANY * UNR_NW;  // rows of a stripe (unrolled_max_tiles)


// Prep: one thread per (b, h, i, c), c < DP.  fp32 copies of Q, K, V, gO and gO^T,
// D, grad x_c, coordinates; dG = sigma(1 - sigma) O dO (flash_sinkhorn_attn.py:278-292).
template <typename T, int DP>
__global__ void __launch_bounds__(256) unrolled_prep_kernel(UnrPrepArgs p) {
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
  float qv = 0.f, kv = 0.f, vv = 0.f, go = 0.f, oa = 0.f;
  if (ok && c < d) {
    qv = to_f32(reinterpret_cast<const T*>(p.q)[off]);
    kv = to_f32(reinterpret_cast<const T*>(p.k)[off]);
    vv = to_f32(reinterpret_cast<const T*>(p.v)[off]);
    const float dO = p.grad_o[((size_t)b * N + i) * p.H * d + (size_t)h * d + c];
    oa = p.o_avg[((size_t)bh * N + i) * d + c];
    float s = 1.f;
    if (p.g) {
      s = 1.f / (1.f + __expf(-to_f32(reinterpret_cast<const T*>(p.g)[off])));
      static_cast<T*>(p.dg)[((size_t)bh * N + i) * d + c] = from_f32<T>(s * (1.f - s) * oa * dO);
    }
    go = s * dO;
  } else if (p.g && i < N && c < d) {
    static_cast<T*>(p.dg)[((size_t)bh * N + i) * d + c] = from_f32<T>(0.f);
  }
  static_cast<T*>(p.qp)[row * DP + c] = from_f32<T>(qv);  // exact: qv, kv come from T
  static_cast<T*>(p.kp)[row * DP + c] = from_f32<T>(kv);
  p.vp[row * DP + c] = vv;
  p.gp[row * DP + c] = go;
  static_cast<T*>(p.qt)[((size_t)bh * DP + c) * Np + i] = from_f32<T>(qv);
  static_cast<T*>(p.kt)[((size_t)bh * DP + c) * Np + i] = from_f32<T>(kv);
  p.gt[((size_t)bh * DP + c) * Np + i] = go;
  float part = go * oa;
#pragma unroll
  for (int o = DP / 2; o >= 1; o >>= 1) part += __shfl_xor(part, o, WAVE);
  if (c < 3) p.gxs[((size_t)bh * 3 + c) * Np + i] = (ok && p.grad_xc) ? p.grad_xc[((size_t)bh * N + i) * 3 + c] : 0.f;
  if (c < 3 && h == 0) p.xs[((size_t)b * 3 + c) * Np + i] = (p.x && i < N) ? p.x[((size_t)b * N + i) * 3 + c] : 0.f;
  if (c == 0) {
    if (ok && p.grad_xc)
      for (int t = 0; t < 3; ++t) part += p.grad_xc[((size_t)bh * N + i) * 3 + t] * p.xc[((size_t)bh * N + i) * 3 + t];
    p.dcoef[(size_t)bh * Np + i] = ok ? part : 0.f;
  }
}

// Finalize: dx = sum_h dx_part; d pos_weight, d w_dist = sums of the workgroup partials.
__global__ void __launch_bounds__(256) unrolled_finalize_kernel(UnrBwdArgs a, float* dx, float* dpw, float* dw) {
  const int e = blockIdx.x * 256 + threadIdx.x;
  const int nx = a.B * a.N * 3;
  if (dx && e < nx) {
    const int b = e / (a.N * 3), r = e % (a.N * 3);
    dx[e] = ordered_sum(a.dx_part + (size_t)b * a.H * a.N * 3 + r, (size_t)a.N * 3, a.H, 0.f);
  }
  if (dpw && e < a.H * 68) {
    const int h = e / 68, k = e % 68;
    float s = 0.f;
    for (int b = 0; b < a.B; ++b) s = ordered_sum(a.dpw_part + (((size_t)b * a.H + h) * a.G) * 68 + k, 68, a.G, s);
    dpw[e] = s;
  }
  if (dw && e < a.H) {
    float s = 0.f;
    for (int b = 0; b < a.B; ++b) s = ordered_sum(a.dw_part + ((size_t)b * a.H + e) * a.G, 1, a.G, s);
    dw[e] = s;
  }
}

// gather_vector (sinkhorn_bwd_kernel.h) storing scale * value at valid entries.
__device__ __forceinline__ bool gather_scaled(const uint64_t* buf, int n, int Np, uint32_t tag, float* dst,
                                              const unsigned char* valid, ErrRef err, int* s_flag, float scale) {
  const int t = threadIdx.x;
  for (int i = n + t; i < Np; i += UNR_NT) dst[i] = 0.f;
  const bool ok = poll_vector<UNR_NT>(buf, n, tag, err, [&](int off, uint64_t w) {
    const int i = off + t;
    dst[i] = valid[i] ? scale * __uint_as_float((uint32_t)(w >> 32)) : 0.f;
  });
  if (!ok) *s_flag = 1;
  __syncthreads();
  return *s_flag == 0;
}

// A lane's share of the transposed operand of one dQ / dK product (row l % 16 of the
// operand, streamed columns 4g .. 4g + 3 and 16 + 4g .. 16 + 4g + 3), loaded ahead of
// the product, and the product itself (Mfma<T, DP>::pv_split with the loads done).
template <typename T> struct VtQuad;
template <> struct VtQuad<bf16> { using type = bf16x4; };
template <> struct VtQuad<float> { using type = f32x4; };
template <typename T>
__device__ __forceinline__ void load_vt(const T* vt_row, int lane, typename VtQuad<T>::type& lo,
                                        typename VtQuad<T>::type& hi) {
  const int g = lane >> 4;
  lo = *reinterpret_cast<const typename VtQuad<T>::type*>(vt_row + 4 * g);
  hi = *reinterpret_cast<const typename VtQuad<T>::type*>(vt_row + 16 + 4 * g);
}
// The hi + lo split works on packed pairs: one rounding conversion gives the hi
// halves of two values, whose fp32 values are bit masks of the packed word (no second
// conversion), then one conversion packs the two remainders.
__device__ __forceinline__ void split_pair(float x0, float x1, uint32_t& hp, uint32_t& lp) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  const bf16x2_t h = {(bf16)x0, (bf16)x1};
  hp = __builtin_bit_cast(uint32_t, h);
  const float h0 = __uint_as_float(hp << 16), h1 = __uint_as_float(hp & 0xffff0000u);
  const bf16x2_t l = {(bf16)(x0 - h0), (bf16)(x1 - h1)};
  lp = __builtin_bit_cast(uint32_t, l);
}
// W of a lane's two tiles (p0: streamed rows 0..15, p1: 16..31) as the A operand of
// the dQ / dK product: bf16 inputs carry it as a hi + lo pair of bf16 fragments (split
// once, used for every output column block), fp32 inputs as the values themselves.
template <typename T> struct WOperand;
template <> struct WOperand<bf16> { bf16x8 hi, lo; };
template <> struct WOperand<float> { f32x4 p0, p1; };
template <typename T> __device__ __forceinline__ WOperand<T> w_operand(const f32x4& p0, const f32x4& p1);
template <> __device__ __forceinline__ WOperand<bf16> w_operand<bf16>(const f32x4& p0, const f32x4& p1) {
  typedef __attribute__((__vector_size__(16))) uint32_t u32x4;
  uint32_t h[4], l[4];
  split_pair(p0[0], p0[1], h[0], l[0]);
  split_pair(p0[2], p0[3], h[1], l[1]);
  split_pair(p1[0], p1[1], h[2], l[2]);
  split_pair(p1[2], p1[3], h[3], l[3]);
  const u32x4 ah = {h[0], h[1], h[2], h[3]}, al = {l[0], l[1], l[2], l[3]};
  return WOperand<bf16>{__builtin_bit_cast(bf16x8, ah), __builtin_bit_cast(bf16x8, al)};
}
template <> __device__ __forceinline__ WOperand<float> w_operand<float>(const f32x4& p0, const f32x4& p1) {
  return WOperand<float>{p0, p1};
}
__device__ __forceinline__ f32x4 pv_regs(const WOperand<bf16>& w, const bf16x4& lo, const bf16x4& hi, f32x4 acc) {
  bf16x8 b;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    b[r] = lo[r];
    b[4 + r] = hi[r];
  }
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(w.hi, b, acc, 0, 0, 0);
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(w.lo, b, acc, 0, 0, 0);
}
__device__ __forceinline__ f32x4 pv_regs(const WOperand<float>& w, const f32x4& lo, const f32x4& hi, f32x4 acc) {
#pragma unroll
  for (int r = 0; r < 4; ++r) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(w.p0[r], lo[r], acc, 0, 0, 0);
#pragma unroll
  for (int r = 0; r < 4; ++r) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(w.p1[r], hi[r], acc, 0, 0, 0);
  return acc;
}

// GEN: the cost may carry position bins or geometry (set by the host when either is
// passed); GEN = false compiles none of their per-element code.
// T: the input type.  The cost recompute q.k and the products dQ += W K, dK += W^T Q
// run on Mfma<T, DP> (bf16 inputs: the bf16 MFMA with exact operands, W as a hi + lo
// bf16 pair, fp32 accumulation, as the forward); the centroid sweep's products, whose
// operands (sigma(G) dO) are not bf16-exact, run on the fp32 MFMA.
// Operand modes of the kernel: streamed operands read from L2 (their padded copies
// [Np][DP] and transposed [DP][Np] written by the prep kernel: GLOBAL), or Q and K
// resident in LDS (RES).
constexpr int UNR_OPS_GLOBAL = 0, UNR_OPS_RES = 2;
// Floats of the part hand-over region: the write_rows hand-over [NW][16][DP] (which
// also holds the dx hand-over [NW][2][16][6]).
__host__ __device__ inline int unr_region_floats(int DP) { return UNR_NW * 16 * DP; }

// Resident operands (OPS = UNR_OPS_RES: bf16 inputs, DP = 32, when LDS has room): Q and
// K stay in LDS for the whole launch, row-major [Np][32] bf16 without padding, under a
// swizzle that keeps both of their readers free of bank conflicts (64 banks of 4 bytes):
//   row j lies in 256-byte line L = j / 4, at 64-byte window (j + L) mod 4 of it, and its
//   16-byte chunk q (columns 8q .. 8q + 7) at chunk position q ^ sw(L),
//   sw(L) = 2 (L mod 2) + (L / 2 mod 2).
// Readers: the cost products' fragments (a lane reads 16 bytes of row l % 16 of a 16-row
// tile, chunk l / 16) and the transposed reads of the dQ / dK products
// (ds_read_b64_tr_b16: in each 16-lane block, source lane 4i + s reads 4 columns 4s ..
// 4s + 3 of row i of a 4-row block, and output lane t receives column t of the block's
// rows 0..3 -- the B operand of the 16x16x32 MFMA for 4 consecutive streamed rows).
__device__ __forceinline__ int res_off(int j, int c) {  // element offset of (row j, column c)
  const int L = j >> 2;
  const int sw = ((L & 1) << 1) | ((L >> 1) & 1);
  return L * 128 + ((j + L) & 3) * 32 + (((c >> 3) ^ sw) << 3) + (c & 7);
}
// 4 consecutive rows j0 + 4 (l / 16) .. + 3 of column cb * 16 + l % 16 (a lane's share of
// the B operand for streamed rows j0 + 4 (l / 16) + i, i = 0..3)
__device__ __forceinline__ bf16x4 res_tr4(const bf16* op, int j0, int cb, int lane) {
  typedef short s16x4 __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) s16x4* lds_s16x4;
  const int g = lane >> 4, t = lane & 15;
  const bf16* src = op + res_off(j0 + 4 * g + (t >> 2), cb * 16 + 4 * (t & 3));
  const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4)(src));
  return __builtin_bit_cast(bf16x4, v);
}

template <typename T, int DP, bool GEN, int OPS>
__global__ void __launch_bounds__(UNR_NT) unrolled_bwd_kernel(UnrBwdArgs a) {
  constexpr bool RES = OPS == UNR_OPS_RES;
  static_assert(!RES || (sizeof(T) == 2 && DP == 32), "resident operands: bf16, DP = 32");
  using M = Mfma<float, DP>;
  using MQ = Mfma<T, DP>;
  constexpr int NC = DP / 16;
  constexpr int NW = UNR_NW;
  constexpr int MAXT = unr_maxt<DP>();
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ int s_flag, s_tmp, s_local;
  __shared__ int s_exact;  // number of a sweep whose factors are out of range (exact path)
  __shared__ float s_pw[68];   // pos_weight of this head (natural units)
  __shared__ float s_dpw[68];  // d pos_weight partial of this workgroup (times eps)
  int grp, member;
  if (!group_of(a.B * a.H, a.G, grp, member)) return;
  const int b = grp / a.H, h = grp % a.H;
  const int N = a.N, d = a.d, K = a.K;
  const int Np = ((N + 31) / 32) * 32;
  const int BH = a.B * a.H;
  const size_t bh = (size_t)grp;
  const int tid = threadIdx.x, lane = tid & (WAVE - 1), wave = tid / WAVE, g = lane >> 4;
  if (tid == 0) {
    s_flag = 0;
    s_local = 1;
    s_exact = -1;
  }
  if (tid < 68) {
    s_pw[tid] = a.pos_w ? a.pos_w[h * 68 + tid] : 0.f;
    s_dpw[tid] = 0.f;
  }
  if (blockIdx.x == 0 && tid == 0)
    __hip_atomic_store(a.err.ws + 1, a.salt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

  // ---- LDS carve-up (must match unrolled_bwd_lds_bytes)
  unsigned char* valid = smem;
  float* xs0 = reinterpret_cast<float*>(smem + ((Np + 15) / 16) * 16);
  float* xs1 = xs0 + Np;
  float* xs2 = xs1 + Np;
  float* gx0 = xs2 + Np;
  float* gx1 = gx0 + Np;
  float* gx2 = gx1 + Np;
  float* dcf = gx2 + Np;
  float* GLU = dcf + Np;
  float* GLV = GLU + Np;
  float* STA = GLV + Np;  // streamed exponent terms of term 1 (or of P in CS_cent)
  float* STB = STA + Np;  // streamed exponent terms of term 2 (or of P in RS(K-1))
  float* STG = STB + Np;  // exp2(STB - STA) of a sweep with both terms (the column factor)
  float* sred = STG + Np;                        // [NW][MAXT][16]
  float* spart = sred + NW * UNR_MAXT_ANY * 16;  // [NW][16][DP] part hand-over
  float* sscal = spart + unr_region_floats(DP);  // [NW]
  float* ldmu = sscal + NW;                      // d log_mu of my rows, summed over the sweeps
  float* ldnu = ldmu + UNR_MAX_LOCAL;            // d log_nu of my columns
  T* opq = reinterpret_cast<T*>(ldnu + UNR_MAX_LOCAL);  // RES: Q, then K, swizzled [Np][32]
  T* opk = opq + (size_t)Np * DP;

  const int n = mask_setup(a.mask ? a.mask + (size_t)b * N : nullptr, N, valid, &s_tmp);
  const int n_tiles = (n + 15) / 16;
  int t0, t1;
  stripe(n_tiles, member, a.G, t0, t1);
  const int nr = t1 - t0;
  for (int i = n_tiles * 16 + member; i < N; i += a.G) {
    for (int c = tid; c < d; c += UNR_NT) {
      static_cast<T*>(a.dq)[(bh * N + i) * d + c] = from_f32<T>(0.f);
      static_cast<T*>(a.dk)[(bh * N + i) * d + c] = from_f32<T>(0.f);
      static_cast<T*>(a.dv)[(bh * N + i) * d + c] = from_f32<T>(0.f);
    }
    if (tid < 3) a.dx_part[(bh * N + i) * 3 + tid] = 0.f;
    if (tid == 0) {
      a.dlog_mu[bh * N + i] = 0.f;
      a.dlog_nu[bh * N + i] = 0.f;
      if (a.dv_init) a.dv_init[bh * N + i] = 0.f;
    }
  }
  if (n == 0 || nr <= 0) {
    if (tid < 68) a.dpw_part[(bh * a.G + member) * 68 + tid] = 0.f;
    if (tid == 0) a.dw_part[bh * a.G + member] = 0.f;
    return;  // owns nothing; no other member waits on it
  }
  for (int i = tid; i < Np; i += UNR_NT) {
    xs0[i] = a.xs[((size_t)b * 3 + 0) * Np + i];
    xs1[i] = a.xs[((size_t)b * 3 + 1) * Np + i];
    xs2[i] = a.xs[((size_t)b * 3 + 2) * Np + i];
    gx0[i] = a.gxs[(bh * 3 + 0) * Np + i];
    gx1[i] = a.gxs[(bh * 3 + 1) * Np + i];
    gx2[i] = a.gxs[(bh * 3 + 2) * Np + i];
    dcf[i] = a.dcoef[bh * Np + i];
    GLU[i] = 0.f;
    GLV[i] = 0.f;
  }
  for (int q = tid; q < UNR_MAX_LOCAL; q += UNR_NT) ldmu[q] = ldnu[q] = 0.f;
  if constexpr (RES) {  // Q and K into LDS, swizzled (16-byte chunks)
    typedef __attribute__((__vector_size__(16))) int i32x4;
    const T* gq = static_cast<const T*>(a.qp) + bh * Np * DP;
    const T* gk = static_cast<const T*>(a.kp) + bh * Np * DP;
    for (int e = tid; e < Np * 4; e += UNR_NT) {
      const int j = e >> 2, q = e & 3;
      const i32x4 vq = *reinterpret_cast<const i32x4*>(gq + (size_t)j * DP + 8 * q);
      const i32x4 vk = *reinterpret_cast<const i32x4*>(gk + (size_t)j * DP + 8 * q);
      *reinterpret_cast<i32x4*>(opq + res_off(j, 8 * q)) = vq;
      *reinterpret_cast<i32x4*>(opk + res_off(j, 8 * q)) = vk;
    }
  }
  __syncthreads();
  const float eps = a.eps[h];
  const float kappa = a.lam / (a.lam + eps);
  const float ik = 1.f / kappa;
  const float sc = LOG2E / (sqrtf((float)d) * eps);
  const float isc = 1.f / sc;
  const float bsc = -LOG2E / eps;  // bias (pw + w d/(r0 + d)) -> log2 logit
  const float wd = a.w_dist ? a.w_dist[h] : 0.f;
  const bool geo = GEN && a.has_geo != 0 && wd != 0.f;
  const bool use_bins = GEN && a.bins8 != nullptr;
  const uint8_t* bins_b = use_bins ? a.bins8 + (size_t)b * Np * Np : nullptr;
  const float r0 = a.r0;
  const int r_lo = t0 * 16;
  const float* hist = a.hist;
  const size_t bhN = bh * N;
  auto Un = [&](int k, int i) { return hist[((size_t)(2 * k + 1) * BH + bh) * N + i]; };  // natural
  auto Vn = [&](int k, int j) {
    if (k >= 0) return hist[((size_t)(2 * k) * BH + bh) * N + j];
    return a.v_init ? a.v_init[bhN + j] : 0.f;
  };
  // Prefetch loads: relaxed atomic loads, which the compiler issues where they stand
  // (it may not sink them to their first use past the main loop).
  auto pld = [&](const float* p_) { return __hip_atomic_load(const_cast<float*>(p_), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); };
  auto UnP = [&](int k, int i) { return pld(hist + ((size_t)(2 * k + 1) * BH + bh) * N + i); };
  auto VnP = [&](int k, int j) {
    if (k >= 0) return pld(hist + ((size_t)(2 * k) * BH + bh) * N + j);
    return a.v_init ? pld(a.v_init + bhN + j) : 0.f;
  };

  // Wave -> resident tiles and streamed pairs.  Waves w and w + 4 of a workgroup share
  // a SIMD, and a SIMD's main-loop time follows the work of its two waves together, so
  // the work is balanced per SIMD:
  //  - nr <= 4: the nr * n_pairs (tile, pair) units are cut into four equal ranges in
  //    SIMD order; a SIMD's range is split between its two waves at the tile boundary
  //    it contains, else at its middle, so that every wave takes one tile and a
  //    contiguous pair range of it (the larger part to the older wave, which the SIMD
  //    issues for first);
  //  - 4 < nr <= NW: wave takes tile wave % nr, and of its pairs every
  //    (NW - tile + nr - 1) / nr-th from wave / nr (the waves of a tile interleave);
  //  - nr > NW: wave owns tiles wave and wave + NW (slots 0 and 1), all pairs.
  // Each tile's partial sums are then combined over the waves of tile_mask(tile).
  const bool spread = nr <= NW;
  const int n_pairs = (n_tiles + 1) / 2;
  auto work_of = [&](int w, int& tile, int& p0, int& p1, int& step) {
    if (!spread) {
      tile = w; p0 = 0; p1 = n_pairs; step = 1;
    } else if (nr <= 4) {
      const int U = nr * n_pairs, o = 2 * (w & 3) + (w >> 2);
      const int sb = (o >> 1) * U / 4, se = ((o >> 1) + 1) * U / 4;
      const int tb = (sb / n_pairs + 1) * n_pairs;  // first tile boundary after sb
      const int cut = tb < se ? tb : (sb + se) / 2;
      // the SIMD issues for its older wave (w < 4) first: that wave takes the larger part
      const bool first = ((o & 1) == 0) == (cut - sb >= se - cut);
      const int ub = first ? sb : cut, ue = first ? cut : se;
      tile = min(ub / n_pairs, nr - 1);
      p0 = ub - tile * n_pairs; p1 = ue - tile * n_pairs; step = 1;
    } else {
      tile = w % nr; p0 = w / nr; p1 = n_pairs; step = (NW - tile + nr - 1) / nr;
    }
  };
  int ts, wp0, wp1, wstep;
  work_of(wave, ts, wp0, wp1, wstep);
  uint64_t tmasks = 0;  // byte rt: the waves holding partials of tile rt (spread)
  if (spread)
    for (int w = 0; w < NW; ++w) {
      int t_, a_, b_, c_;
      work_of(w, t_, a_, b_, c_);
      tmasks |= 1ull << (8 * t_ + w);
    }
  auto tile_mask = [&](int rt) -> unsigned { return spread ? (unsigned)(tmasks >> (8 * rt)) & 0xffu : 1u << (rt % NW); };
  const int nts = spread ? nr : NW;  // slot s holds tile ts + nts s
  auto slot_of = [&](int rt) { return spread ? 0 : rt / NW; };
  // the wave that writes tile ts's rows (the lowest of its tile's waves)
  const bool lead = (tile_mask(ts) & ((1u << wave) - 1u)) == 0u;
  const T* qp = static_cast<const T*>(a.qp) + bh * Np * DP;
  const T* kp = static_cast<const T*>(a.kp) + bh * Np * DP;
  const T* qt = static_cast<const T*>(a.qt) + bh * DP * Np;
  const T* kt = static_cast<const T*>(a.kt) + bh * DP * Np;
  const float* vp = a.vp + bh * Np * DP;
  const float* gp = a.gp + bh * Np * DP;
  const float* gt = a.gt + bh * DP * Np;

  // Copy of the streamed operand of a sweep of orientation `row` into LDS: the
  // row-major copy from L2 (batches of 8 16-byte chunks a thread, all loads of a batch
  // before its stores; one batch up to Np = 1024), then, after a barrier, the
  // transposed copy built from it inside LDS (8 bf16 of one column per 16-byte chunk).
  // Loads are unconditional, from clamped chunk indices.  Every thread calls it.
  // (valid, row, cent, use_c, term2, k) of a sweep: the fill of its streamed terms
  // (fill_streamed, or with the operand copy) precedes it
  struct SweepDesc { bool valid, row, cent, use_c, term2; int k; };
  // With the operand copy go the next sweep's streamed terms (fill_streamed's values
  // for this thread's entries i = tid, tid + UNR_NT, which cover Np <= 1024): their raw
  // loads are issued first, then the copy's, so the two share one wait.
  // Sweeps with both terms (use_c and term2, no centroid): the two exponentials of an
  // element differ by a row factor times a column factor,
  //   exp2(x sc + sb_j) = exp2(x sc + sa_j) * exp2(sb_j - sa_j) * exp2(rb_i - ra_i)
  // (the cost and the bias are common), so such a sweep takes one exponential an
  // element and no second cost product.  The column factors exp2(sb_j - sa_j) are
  // kept in STG; a sweep with a factor outside [2^-FLIM, 2^FLIM] (row or column) takes
  // the exact two-exponential path instead (s_exact holds its number, rows are checked
  // per wave), so that no factor product can overflow or hide a term.
  constexpr float FLIM = 40.f;
  int sweep_no = 0;  // number of the running sweep (1, 2, ...); the fills are for the next
  auto both_factor = [&](const SweepDesc& nx, bool ok, float sa, float sb) -> float {
    if (!(nx.use_c && nx.term2 && !nx.cent) || !ok) return 0.f;
    const float dl = sb - sa;
    if (!(fabsf(dl) <= FLIM)) s_exact = sweep_no + 1;
    return fast_exp2(fminf(fmaxf(dl, -FLIM), FLIM));
  };

  f32x4 dQa[MAXT][NC], dKa[MAXT][NC];
  float gbx[MAXT], gby[MAXT], gbz[MAXT], xt0[MAXT], xt1[MAXT], xt2[MAXT], dmu[MAXT], dnu[MAXT];
#pragma unroll
  for (int s = 0; s < MAXT; ++s) {
#pragma unroll
    for (int c = 0; c < NC; ++c) dQa[s][c] = dKa[s][c] = f32x4{0.f, 0.f, 0.f, 0.f};
    gbx[s] = gby[s] = gbz[s] = xt0[s] = xt1[s] = xt2[s] = dmu[s] = dnu[s] = 0.f;
  }
  float s_w = 0.f;  // sum W * cg (d w_dist, row-owned sweeps)

  uint64_t* xgu = a.xch + bh * 2 * (size_t)Np;
  uint64_t* xgv = xgu + Np;
  const uint32_t salt = a.salt << 12;
  uint32_t phase = 0;
  // placement words of the group (after all (b,h)'s exchange words): plain-store
  // publishing from the second exchange on if every member runs on its XCD
  uint64_t* xpl = a.xch + (size_t)BH * 4 * Np + bh * 32;
  bool local = false;

  auto write_rows = [&](f32x4 (&acc)[MAXT][NC], void* out, float scale) {  // gradients in the input type
    __syncthreads();
    if (!lead) {
#pragma unroll
      for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int r = 0; r < 4; ++r) spart[(size_t)wave * 16 * DP + (4 * g + r) * DP + c * 16 + (lane & 15)] = acc[0][c][r];
    }
    __syncthreads();
    if (lead) {
#pragma unroll
      for (int s = 0; s < MAXT; ++s) {
        const int rt = ts + nts * s;
        if (rt >= nr) continue;
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            float v = acc[s][c][r];
            for (unsigned m = tile_mask(rt) & ~(1u << wave); m; m &= m - 1u)
              v += spart[(size_t)__builtin_ctz(m) * 16 * DP + (4 * g + r) * DP + c * 16 + (lane & 15)];
            const int row = (t0 + rt) * 16 + 4 * g + r, col = c * 16 + (lane & 15);
            if (row < N && col < d)
              static_cast<T*>(out)[(bh * N + row) * d + col] = from_f32<T>((row < n && valid[row]) ? scale * v : 0.f);
          }
      }
    }
  };

  // Reduction of a per-(tile slot, lane) value over lane groups and parts into
  // `dst_fn(local row q, value)` for q < nr*16 (called by the owning threads).
  auto combine_rows = [&](const float (&val)[MAXT], auto dst_fn) {
#pragma unroll
    for (int s = 0; s < MAXT; ++s) {
      const float r = sum_groups(val[s]);
      if (lane < 16) sred[(wave * MAXT + s) * 16 + lane] = r;
    }
    __syncthreads();
    for (int q = tid; q < nr * 16; q += UNR_NT) {
      const int rt = q >> 4, l16 = q & 15;
      float v = 0.f;
      for (unsigned m = tile_mask(rt); m; m &= m - 1u) v += sred[(__builtin_ctz(m) * MAXT + slot_of(rt)) * 16 + l16];
      dst_fn(q, v);
    }
  };

  // One sweep.  ROW: resident rows i (streamed j), else resident columns j
  // (streamed i).  CENT: the centroid sweep of that orientation.  Index k as in
  // the header comment (CS_cent uses k = K).  USE_C (the recurrence term: all but
  // RS(-1) and CS_cent) and TERM2 (the mirror term: all but RS(K-1) and CS_cent) are
  // compile-time, so the element loop carries no test of them.
  // Streamed exponent terms STA / STB of a sweep (flags and k as the sweep's).  Filled
  // for the next sweep right after a sweep's combine (its main loop is done with them),
  // so the hist loads share the wait of the exchange and of the operand copy.
  // RES: the next sweep's history values, loaded at the start of a sweep (its main
  // loop issues no global loads, so they arrive under it instead of at the fill and
  // at the next sweep's start): the streamed terms' raw values (entries tid and
  // tid + UNR_NT; Np <= 1024 with resident operands) and the resident slots' terms.
  float pf0[2] = {0.f, 0.f}, pf1[2] = {0.f, 0.f};
  float pra[MAXT], prb[MAXT];
  bool pf_have = false;
  auto stream_terms = [&](const SweepDesc& nx, float f0, float f1, float& sa, float& sb) {
    sa = sb = NEG_BIG;
    if (nx.row) {  // streamed columns j: f0 = v^k_j, f1 = log nu_j
      if (nx.use_c) sa = (f0 * ik - f1) * LOG2E;  // s^{C,k}
      if (nx.term2 || nx.cent) sb = f0 * LOG2E;  // s^{R,k+1} or P
    } else if (nx.cent) {  // streamed rows i: f0 = log u_i, f1 = log Z_i
      sa = (f0 - f1) * LOG2E;  // P
    } else {  // f0 = u^k_i, f1 = log mu_i
      sa = (f0 * ik - f1) * LOG2E;  // s^{R,k}
      sb = f0 * LOG2E;             // s^{C,k}
    }
  };
  auto prefetch = [&](const SweepDesc& nx) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int ic = min(tid + u * UNR_NT, N - 1);  // clamped: the loads are unconditional
      if (nx.row) {
        pf0[u] = VnP(nx.k, ic);
        pf1[u] = pld(a.log_nu + bhN + ic);
      } else if (nx.cent) {
        pf0[u] = pld(a.log_u + bhN + ic);
        pf1[u] = pld(a.log_z + bhN + ic);
      } else {
        pf0[u] = UnP(nx.k, ic);
        pf1[u] = pld(a.log_mu + bhN + ic);
      }
    }
#pragma unroll
    for (int s = 0; s < MAXT; ++s) {
      const int rt = ts + nts * s;
      const int ri = (t0 + min(rt, nr - 1)) * 16 + (lane & 15);
      const bool ok = rt < nr && ri < n && valid[ri];
      float ra = NEG_BIG, rb = NEG_BIG;
      if (ok) {
        if (nx.row) {
          if (nx.use_c) ra = UnP(nx.k, ri) * LOG2E;
          if (nx.cent) rb = (pld(a.log_u + bhN + ri) - pld(a.log_z + bhN + ri)) * LOG2E;
          else if (nx.term2) rb = (UnP(nx.k + 1, ri) * ik - pld(a.log_mu + bhN + ri)) * LOG2E;
        } else if (nx.cent) {
          ra = VnP(K - 1, ri) * LOG2E;
        } else {
          ra = VnP(nx.k - 1, ri) * LOG2E;
          rb = (VnP(nx.k, ri) * ik - pld(a.log_nu + bhN + ri)) * LOG2E;
        }
      }
      pra[s] = ra;
      prb[s] = rb;
    }
  };
  auto fill_streamed = [&](const SweepDesc& nx) {
    if (RES && pf_have) {
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int i = tid + u * UNR_NT;
        if (i >= Np) continue;
        const bool ok = i < n && valid[i];
        float sa = NEG_BIG, sb = NEG_BIG;
        if (ok) stream_terms(nx, pf0[u], pf1[u], sa, sb);
        STA[i] = sa;
        STB[i] = sb;
        STG[i] = both_factor(nx, ok, sa, sb);
      }
      return;
    }
    for (int i = tid; i < Np; i += UNR_NT) {
      float sa = NEG_BIG, sb = NEG_BIG;
      if (i < n && valid[i]) {
        if (nx.row) {  // streamed columns j
          if (nx.use_c) sa = (Vn(nx.k, i) * ik - a.log_nu[bhN + i]) * LOG2E;  // s^{C,k}
          if (nx.term2 || nx.cent) sb = Vn(nx.k, i) * LOG2E;                  // s^{R,k+1} or P
        } else {       // streamed rows i
          if (nx.cent) sa = (a.log_u[bhN + i] - a.log_z[bhN + i]) * LOG2E;   // P
          else {
            sa = (Un(nx.k, i) * ik - a.log_mu[bhN + i]) * LOG2E;             // s^{R,k}
            sb = Un(nx.k, i) * LOG2E;                                         // s^{C,k}
          }
        }
      }
      STA[i] = sa;
      STB[i] = sb;
      STG[i] = both_factor(nx, i < n && valid[i], sa, sb);
    }
  };

  auto sweep = [&](auto row_tag, auto cent_tag, auto usec_tag, auto term2_tag, int k, SweepDesc next) -> bool {
    constexpr bool ROW = decltype(row_tag)::value;
    constexpr bool CENT = decltype(cent_tag)::value;
    constexpr bool use_c = decltype(usec_tag)::value;
    constexpr bool term2 = decltype(term2_tag)::value;
    const bool publish = ROW ? k >= 0 : (CENT || k >= 1);
    constexpr bool BOTH = use_c && term2 && !CENT;  // one exponential an element (see STG)
    ++sweep_no;
    __syncthreads();  // STA / STB / STG and the gathered vectors are complete
    const float* STC = ROW ? GLV : GLU;  // streamed recurrence coefficients
    const T* Sop = ROW ? kp : qp;  // GLOBAL: the streamed operand and its transpose in L2
    const T* Sot = ROW ? kt : qt;
    const T* Rop = ROW ? qp : kp;

    typename MQ::Frag bf[MAXT];
    typename M::Frag cbf[MAXT];
    float ra[MAXT], rb[MAXT], dd[MAXT], xr0[MAXT], xr1[MAXT], xr2[MAXT], Dr[MAXT], gr0[MAXT], gr1[MAXT], gr2[MAXT];
    float red[MAXT][4];  // per accumulator row of a lane: independent chains
    float cra[MAXT], crb[MAXT];  // ra / sc, rb / sc: the accumulator inits of the cost products
    float gam[MAXT];             // BOTH: row factor exp2(rb - ra) times dd
    bool row_out = false;        // BOTH: a row factor of this wave is out of range
    f32x4 gVa[MAXT][NC];
#pragma unroll
    for (int s = 0; s < MAXT; ++s) {
      const int rt = ts + nts * s;
      const int ri = (t0 + min(rt, nr - 1)) * 16 + (lane & 15);
      const bool ok = rt < nr && ri < n && valid[ri];
      if constexpr (RES) bf[s].v[0] = *reinterpret_cast<const bf16x8*>((ROW ? opq : opk) + res_off(ri, 8 * (lane >> 4)));
      else MQ::load(bf[s], Rop + (size_t)ri * DP, lane);
      if (CENT) M::load(cbf[s], (ROW ? gp : vp) + (size_t)ri * DP, lane);
      ra[s] = rb[s] = NEG_BIG;
      dd[s] = 0.f;
      if (RES && pf_have) {  // prefetched during the previous sweep (the same formulas)
        ra[s] = pra[s];
        rb[s] = prb[s];
        if (ok && ((ROW && term2) || (!ROW && !CENT))) dd[s] = ROW ? GLU[ri] : GLV[ri];
      } else if (ok) {
        if (ROW) {  // resident rows i
          if (use_c) ra[s] = Un(k, ri) * LOG2E;                                             // s^{C,k}
          if (CENT) rb[s] = (a.log_u[bhN + ri] - a.log_z[bhN + ri]) * LOG2E;                // P
          else if (term2) rb[s] = (Un(k + 1, ri) * ik - a.log_mu[bhN + ri]) * LOG2E;        // s^{R,k+1}
          if (term2) dd[s] = GLU[ri];
        } else {    // resident columns j
          if (CENT) ra[s] = Vn(K - 1, ri) * LOG2E;                                          // P
          else {
            ra[s] = Vn(k - 1, ri) * LOG2E;                                                  // s^{R,k}
            rb[s] = (Vn(k, ri) * ik - a.log_nu[bhN + ri]) * LOG2E;                          // s^{C,k}
            dd[s] = GLV[ri];
          }
        }
      }
      cra[s] = ra[s] * isc;
      crb[s] = rb[s] * isc;
      gam[s] = 0.f;
      if (BOTH && ok) {
        const float dl = rb[s] - ra[s];
        row_out |= !(fabsf(dl) <= FLIM);
        gam[s] = fast_exp2(fminf(fmaxf(dl, -FLIM), FLIM)) * dd[s];
      }
      xr0[s] = xs0[ri];
      xr1[s] = xs1[ri];
      xr2[s] = xs2[ri];
      Dr[s] = gr0[s] = gr1[s] = gr2[s] = 0.f;
      if (CENT && ROW) {
        Dr[s] = dcf[ri];
        gr0[s] = gx0[ri];
        gr1[s] = gx1[ri];
        gr2[s] = gx2[ri];
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) red[s][e] = 0.f;
#pragma unroll
      for (int c = 0; c < NC; ++c) gVa[s][c] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    if constexpr (RES) {  // the next sweep's history values, under this sweep's main loop
      if (next.valid) prefetch(next);
      pf_have = next.valid;
    }
    if (ts < nts) {
      // The streamed operands of a pair of tiles (Q or K fragments for the cost, the
      // transposed operand for dQ / dK) are the same for every resident slot, so they are
      // loaded once per pair: from LDS in the iteration itself (RES), or from L2 one pair
      // ahead (GLOBAL: the loads of pair sp + wstep are issued, unconditionally from a
      // clamped pair, before pair sp is computed).
      using V4 = typename VtQuad<T>::type;
      typename MQ::Frag afn[2];
      V4 vln[NC], vhn[NC];
      auto load_pair = [&](int sp_) {
        const int spc = min(sp_, n_pairs - 1);
        if constexpr (RES) {
          const T* so = ROW ? opk : opq;
#pragma unroll
          for (int hh = 0; hh < 2; ++hh)
            afn[hh].v[0] = *reinterpret_cast<const bf16x8*>(so + res_off((2 * spc + hh) * 16 + (lane & 15), 8 * (lane >> 4)));
#pragma unroll
          for (int c = 0; c < NC; ++c) {
            vln[c] = res_tr4(so, 32 * spc, c, lane);
            vhn[c] = res_tr4(so, 32 * spc + 16, c, lane);
          }
          return;
        }
#pragma unroll
        for (int hh = 0; hh < 2; ++hh)
          MQ::load(afn[hh], Sop + (size_t)((2 * spc + hh) * 16 + (lane & 15)) * DP, lane);
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          const T* vt_row = Sot + (size_t)(c * 16 + (lane & 15)) * Np + spc * 32;
          load_vt<T>(vt_row, lane, vln[c], vhn[c]);
        }
      };
      // resident operands come from LDS: loaded in the iteration itself (a register copy
      // of a prefetch would cost more than the LDS latency it hides)
      auto main_loop = [&](auto fast_tag) {
      // FAST (BOTH sweeps with factors in range): e2 = e1 * STG_j * exp2(rb - ra)
      constexpr bool FAST = decltype(fast_tag)::value;
      if (!RES) load_pair(wp0);
      for (int sp = wp0; sp < wp1; sp += wstep) {
        if (RES) load_pair(sp);
        typename MQ::Frag afc[2] = {afn[0], afn[1]};
        V4 vlc[NC], vhc[NC];
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          vlc[c] = vln[c];
          vhc[c] = vhn[c];
        }
        if (!RES) load_pair(sp + wstep);
#pragma unroll
        for (int s = 0; s < MAXT; ++s) {
          const int rt = ts + nts * s;
          if (rt >= nr) continue;
          const int ri = (t0 + rt) * 16 + (lane & 15);
          f32x4 wop[2], pop[2];
#pragma unroll
          for (int hh = 0; hh < 2; ++hh) {
            const int st = 2 * sp + hh;
            const int o = st * 16 + 4 * g;
            const typename MQ::Frag& af = afc[hh];
            const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
            f32x4 t = zero;
            if (CENT) {
              typename M::Frag cf;
              M::load(cf, (ROW ? vp : gp) + (size_t)(st * 16 + (lane & 15)) * DP, lane);
              t = M::qk(cf, cbf[s], zero);
            }
            // exponent arguments sc (q.k + ra / sc) + sa_j and sc (q.k + rb / sc) + sb_j: the
            // resident terms ride in the accumulator init, one product per term
            constexpr bool E1 = use_c || (CENT && !ROW), E2 = term2 || (CENT && ROW);
            const f32x4 x1 = E1 ? MQ::qk(af, bf[s], f32x4{cra[s], cra[s], cra[s], cra[s]}) : zero;
            const f32x4 x2 = (E2 && !FAST) ? MQ::qk(af, bf[s], f32x4{crb[s], crb[s], crb[s], crb[s]}) : zero;
            const f32x4 sa = *reinterpret_cast<const f32x4*>(STA + o);
            const f32x4 sb = *reinterpret_cast<const f32x4*>((FAST ? STG : STB) + o);  // FAST: column factors
            const f32x4 scf = use_c ? *reinterpret_cast<const f32x4*>(STC + o) : zero;
            const f32x4 sx0 = *reinterpret_cast<const f32x4*>(xs0 + o);
            const f32x4 sx1 = *reinterpret_cast<const f32x4*>(xs1 + o);
            const f32x4 sx2 = *reinterpret_cast<const f32x4*>(xs2 + o);
            f32x4 sg0 = zero, sg1 = zero, sg2 = zero, sD = zero;
            if (CENT && !ROW) {
              sg0 = *reinterpret_cast<const f32x4*>(gx0 + o);
              sg1 = *reinterpret_cast<const f32x4*>(gx1 + o);
              sg2 = *reinterpret_cast<const f32x4*>(gx2 + o);
              sD = *reinterpret_cast<const f32x4*>(dcf + o);
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const int sj = o + e;  // streamed index (< Np: padded bins read BIN_NONE)
              const int ii = ROW ? ri : sj, jj = ROW ? sj : ri;
              float bias = 0.f, cg = 0.f, dist = 1.f;
              const float dx = xr0[s] - sx0[e], dy = xr1[s] - sx1[e], dz = xr2[s] - sx2[e];
              if (geo) {
                dist = fmaxf(sqrtf(dx * dx + dy * dy + dz * dz), 1e-8f);
                cg = dist / (r0 + dist);
                bias = wd * cg;
              }
              int bin = -1;
              if (use_bins) {
                bin = bins_b[(size_t)ii * Np + jj];
                if (bin < 68) bias += s_pw[bin];
                else bin = -1;
              }
              const float bb = GEN ? bsc * bias : 0.f;
              const float e1 = E1 ? fast_exp2(__builtin_fmaf(x1[e], sc, GEN ? sa[e] + bb : sa[e])) : 0.f;
              const float e2 = (E2 && !FAST) ? fast_exp2(__builtin_fmaf(x2[e], sc, GEN ? sb[e] + bb : sb[e])) : 0.f;
              float W = 0.f;
              if (FAST) {
                // W = e1 scf_j + e2 dd_i = e1 (scf_j + STG_j exp2(rb_i - ra_i) dd_i)
                W = e1 * __builtin_fmaf(gam[s], sb[e], scf[e]);
                red[s][e] = __builtin_fmaf(-e1, scf[e], red[s][e]);
              } else {
                if (use_c) {
                  const float t1 = e1 * scf[e];  // scf holds kappa gl (scaled when gathered)
                  W = t1;
                  red[s][e] -= t1;
                }
                if (term2) W = __builtin_fmaf(e2, dd[s], W);
              }
              if (CENT) {
                const float P = ROW ? e2 : e1;
                float dT = t[e];
                if (ROW) dT += gr0[s] * sx0[e] + gr1[s] * sx1[e] + gr2[s] * sx2[e];
                else dT += sg0[e] * xr0[s] + sg1[e] * xr1[s] + sg2[e] * xr2[s];
                const float qv = P * (dT - (ROW ? Dr[s] : sD[e]));
                W -= qv;
                if (!ROW) {
                  red[s][e] += qv;
                  xt0[s] = __builtin_fmaf(P, sg0[e], xt0[s]);
                  xt1[s] = __builtin_fmaf(P, sg1[e], xt1[s]);
                  xt2[s] = __builtin_fmaf(P, sg2[e], xt2[s]);
                  pop[hh][e] = P;
                }
              }
              wop[hh][e] = W;
              if (geo) {
                const float om = 1.f - cg;
                const float f = W * om * om / dist;
                gbx[s] = __builtin_fmaf(f, dx, gbx[s]);
                gby[s] = __builtin_fmaf(f, dy, gby[s]);
                gbz[s] = __builtin_fmaf(f, dz, gbz[s]);
                if (ROW) s_w = __builtin_fmaf(W, cg, s_w);
              }
              if (ROW && bin >= 0 && W != 0.f) atomicAdd(&s_dpw[bin], W);
            }
          }
          // dQ += W K (dK += W^T Q): for bf16 inputs W is carried as a bf16 hi + lo pair
          // against the exact bf16 operand (two bf16 MFMAs), as the forward's P V
          const WOperand<T> wsp = w_operand<T>(wop[0], wop[1]);
#pragma unroll
          for (int c = 0; c < NC; ++c) {
            if (ROW) dQa[s][c] = pv_regs(wsp, vlc[c], vhc[c], dQa[s][c]);
            else dKa[s][c] = pv_regs(wsp, vlc[c], vhc[c], dKa[s][c]);
            if (CENT && !ROW)
              gVa[s][c] = M::pv(pop[0], pop[1], gt + (size_t)(c * 16 + (lane & 15)) * Np + sp * 32, lane, gVa[s][c]);
          }
        }
      }
      };
      if constexpr (BOTH) {
        if (s_exact != sweep_no && !__any(row_out)) main_loop(std::integral_constant<bool, true>{});
        else main_loop(std::integral_constant<bool, false>{});
      } else {
        main_loop(std::integral_constant<bool, false>{});
      }
    }
    // recurrence output (gl_u^k for RS, gl_v^{k-1} or g_v for CS) of my rows
    uint64_t* buf = ROW ? xgu : xgv;
    ++phase;
    const uint32_t tag = salt | phase;
    float redv[MAXT];
#pragma unroll
    for (int s = 0; s < MAXT; ++s) redv[s] = (red[s][0] + red[s][1]) + (red[s][2] + red[s][3]);
    // the marginal gradients accumulate in LDS (thread q owns row q in every sweep)
    // and are written once at the end
    combine_rows(redv, [&](int q, float v) {
      const int i = r_lo + q;
      if (i >= n) return;
      const bool ok = valid[i];
      if (publish) xch_put(buf + i, v, tag, local);
      if (!ok) return;
      if (ROW) {
        if (k >= 0) ldmu[q] += kappa * v;
      } else if (CENT || k >= 1) {
        ldnu[q] += kappa * v;
      } else if (a.dv_init) {
        a.dv_init[bhN + i] = v;
      }
    });
    // the next sweep's streamed terms, past the combine's barrier (no wave reads
    // STA / STB / STG any more): their loads share the exchange's wait
    if (next.valid) fill_streamed(next);
    if (publish) {
      // gathered as kappa gl: both readers (the streamed coefficients and the
      // resident dd) want the kappa multiple
      if (!gather_scaled(buf, n, Np, tag, ROW ? GLU : GLV, valid, a.err, &s_flag, kappa)) return false;
    } else {
      __syncthreads();
    }
    if (CENT && !ROW) write_rows(gVa, a.dv, 1.f);
    return true;
  };

  using TRUE_ = std::integral_constant<bool, true>;
  using FALSE_ = std::integral_constant<bool, false>;
  // (row, cent, use_c, term2)
  // (valid, row, cent, use_c, term2, k) of each sweep, for the fill that precedes it
  const SweepDesc cs_cent{true, false, true, false, false, K}, rs_cent{true, true, true, true, false, K - 1};
  auto rs_d = [&](int k) { return SweepDesc{true, true, false, true, true, k}; };
  auto cs_d = [&](int k) { return SweepDesc{true, false, false, true, true, k}; };
  const SweepDesc rs_last{true, true, false, false, true, -1}, none{false, false, false, false, false, 0};
  publish_placement(xpl, member, a.salt);
  fill_streamed(cs_cent);
  if (!sweep(FALSE_{}, TRUE_{}, FALSE_{}, FALSE_{}, K, rs_cent)) return;
  // every member published its placement before its words of the first exchange
  if (!read_placement(xpl, a.G, n_tiles, a.salt, a.err, &s_flag, &s_local)) return;
  local = s_local != 0;
  if (!sweep(TRUE_{}, TRUE_{}, TRUE_{}, FALSE_{}, K - 1, cs_d(K - 1))) return;
  for (int k = K - 1; k >= 0; --k) {
    if (k < K - 1 && !sweep(TRUE_{}, FALSE_{}, TRUE_{}, TRUE_{}, k, cs_d(k))) return;
    if (!sweep(FALSE_{}, FALSE_{}, TRUE_{}, TRUE_{}, k, k >= 1 ? rs_d(k - 1) : rs_last)) return;
  }
  if (!sweep(TRUE_{}, FALSE_{}, FALSE_{}, TRUE_{}, -1, none)) return;

  // ---- outputs of my stripe
  const float fs = -1.f / (sqrtf((float)d) * eps);
  write_rows(dQa, a.dq, fs);
  write_rows(dKa, a.dk, fs);
  // invalid rows of the stripe: zero marginal gradients
  for (int q = tid; q < nr * 16; q += UNR_NT) {
    const int i = r_lo + q;
    if (i >= N) continue;
    if (i < n && valid[i]) {
      a.dlog_mu[bhN + i] = ldmu[q];
      a.dlog_nu[bhN + i] = ldnu[q];
    } else {
      a.dlog_mu[bhN + i] = 0.f;
      a.dlog_nu[bhN + i] = 0.f;
      if (a.dv_init) a.dv_init[bhN + i] = 0.f;
    }
  }
  __syncthreads();
#pragma unroll
  for (int s = 0; s < MAXT; ++s) {
    const float v[6] = {sum_groups(gbx[s]), sum_groups(gby[s]), sum_groups(gbz[s]),
                        sum_groups(xt0[s]), sum_groups(xt1[s]), sum_groups(xt2[s])};
    if (lane < 16)
      for (int t = 0; t < 6; ++t) spart[((size_t)(wave * MAXT + s) * 16 + lane) * 6 + t] = v[t];
  }
  {
    const float sw = wave_sum(s_w);
    if (lane == 0) sscal[wave] = sw;
  }
  __syncthreads();
  const float gs = geo ? wd / (eps * r0) : 0.f;
  for (int q = tid; q < nr * 16; q += UNR_NT) {
    const int rt = q >> 4, l16 = q & 15;
    float v[6] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (unsigned m = tile_mask(rt); m; m &= m - 1u)
      for (int t = 0; t < 6; ++t)
        v[t] += spart[((size_t)(__builtin_ctz(m) * MAXT + slot_of(rt)) * 16 + l16) * 6 + t];
    const int i = r_lo + q;
    if (i < N) {
      const bool ok = i < n && valid[i];
      for (int t = 0; t < 3; ++t) a.dx_part[(bh * N + i) * 3 + t] = ok ? gs * v[t] + v[3 + t] : 0.f;
    }
  }
  if (tid < 68) a.dpw_part[(bh * a.G + member) * 68 + tid] = s_dpw[tid] / eps;
  if (tid == 0) {
    float sw = 0.f;
    for (int wv = 0; wv < NW; ++wv) sw += sscal[wv];
    a.dw_part[bh * a.G + member] = sw / eps;
  }
}

size_t unrolled_bwd_lds_bytes(int N, int DP, int elem, int ops) {
  const size_t Np = ((N + 31) / 32) * 32;
  size_t bytes = ((Np + 15) / 16) * 16;
  bytes += 12 * Np * 4;                              // coordinates, grad x_c, D, gathered vectors, STA, STB, STG
  bytes += (size_t)UNR_NW * UNR_MAXT_ANY * 16 * 4;   // recurrence partials
  bytes += 4 * (size_t)unr_region_floats(DP);       // part hand-over
  bytes += UNR_NW * 4;
  bytes += 2 * UNR_MAX_LOCAL * 4;                    // d log_mu, d log_nu of the stripe
  if (ops == UNR_OPS_RES) bytes += 2 * Np * DP * (size_t)elem;  // resident Q and K
  return bytes;
}

// Resident operands if they fit (bf16, DP = 32), else operands from L2.
int unrolled_operand_mode(int N, int DP, int elem, size_t limit) {
  if (elem == 2 && DP == 32 && unrolled_bwd_lds_bytes(N, DP, elem, UNR_OPS_RES) <= limit) return UNR_OPS_RES;
  return UNR_OPS_GLOBAL;
}

int unrolled_max_tiles(int DP) { return (DP <= 32 ? unr_maxt<32>() : unr_maxt<64>()) * UNR_NW; }

template <typename T, int DP>
static hipError_t launch_unr_prep_t(const UnrPrepArgs& p, hipStream_t stream) {
  const size_t Np = ((p.N + 31) / 32) * 32;
  const size_t total = (size_t)p.B * p.H * Np * DP;  // multiple of 1024
  hipLaunchKernelGGL((unrolled_prep_kernel<T, DP>), dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream, p);
  return hipGetLastError();
}

hipError_t launch_unrolled_prep(const UnrPrepArgs& p, bool bf16_in, int DP, hipStream_t stream) {
  if (bf16_in) {
    if (DP == 32) return launch_unr_prep_t<bf16, 32>(p, stream);
    if (DP == 64) return launch_unr_prep_t<bf16, 64>(p, stream);
  } else {
    if (DP == 32) return launch_unr_prep_t<float, 32>(p, stream);
    if (DP == 64) return launch_unr_prep_t<float, 64>(p, stream);
  }
  return hipErrorInvalidValue;
}

template <typename T, int DP, bool GEN, int OPS>
static hipError_t launch_unr_t(const UnrBwdArgs& a, size_t lds, hipStream_t stream, bool coop) {
  auto kern = unrolled_bwd_kernel<T, DP, GEN, OPS>;
  hipError_t e = set_lds_limit((const void*)kern, lds);
  if (e != hipSuccess) return e;
  dim3 grid(grid_blocks(a.B * a.H, a.G)), block(UNR_NT);
  UnrBwdArgs copy = a;
  if (coop) {
    void* args[] = {&copy};
    return hipLaunchCooperativeKernel((const void*)kern, grid, block, args, (unsigned)lds, stream);
  }
  hipLaunchKernelGGL(kern, grid, block, lds, stream, copy);
  return hipGetLastError();
}

template <typename T>
static hipError_t launch_unr_dt(const UnrBwdArgs& a, int DP, size_t lds, hipStream_t stream, bool coop, int ops) {
  const bool gen = (a.bins8 && a.pos_w) || (a.has_geo && a.w_dist);
  constexpr int G0 = UNR_OPS_GLOBAL, RS = UNR_OPS_RES;
  if constexpr (sizeof(T) == 2) {
    if (ops == RS && DP == 32)
      return gen ? launch_unr_t<T, 32, true, RS>(a, lds, stream, coop) : launch_unr_t<T, 32, false, RS>(a, lds, stream, coop);
  }
  if (ops != G0) return hipErrorInvalidValue;
  if (DP == 32)
    return gen ? launch_unr_t<T, 32, true, G0>(a, lds, stream, coop) : launch_unr_t<T, 32, false, G0>(a, lds, stream, coop);
  if (DP == 64)
    return gen ? launch_unr_t<T, 64, true, G0>(a, lds, stream, coop) : launch_unr_t<T, 64, false, G0>(a, lds, stream, coop);
  return hipErrorInvalidValue;
}

// ops: from unrolled_operand_mode(), with lds sized for it
hipError_t launch_unrolled_bwd(const UnrBwdArgs& a, bool bf16_in, int DP, size_t lds, hipStream_t stream, bool coop,
                               int ops) {
  return bf16_in ? launch_unr_dt<bf16>(a, DP, lds, stream, coop, ops)
                 : launch_unr_dt<float>(a, DP, lds, stream, coop, ops);
}

hipError_t launch_unrolled_finalize(const UnrBwdArgs& a, float* dx, float* dpw, float* dw, hipStream_t stream) {
  const int total = std::max(a.B * a.N * 3, a.H * 68);
  hipLaunchKernelGGL(unrolled_finalize_kernel, dim3((total + 255) / 256), dim3(256), 0, stream, a, dx, dpw, dw);
  return hipGetLastError();
}

}  // namespace dfl
