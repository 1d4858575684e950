// Unrolled backward of the balanced Sinkhorn transport on gfx950 (persistent
// per-(b,h) workgroup groups, fp32).
//
// Restates BalancedSinkhornFn.backward / BalancedSinkhornDualFn.backward of
// vv137/deepfold-linear (src/deepfold/model/kernels/flash_sinkhorn_transport.py:322-373
// and 448-516, kernels in balanced_sinkhorn_bwd.py and feature_transport_bwd.py):
// the exact gradient through K unrolled iterations of the forward
//   v^k_j = lm - LSE_i(L_ij + u^{k-1}_i)   (u^{-1} = 0)     column update
//   u^k_i = lm - LSE_j(L_ij + v^k_j)                          row update
//   P_ij  = exp(L_ij + u^{K-1}_i + v^{K-1}_j - lm)            (rows sum to 1)
//   xc_i = sum_j P_ij x_j,  hc_i = sum_j P_ij V_j,  L = -C/eps,
//   C_ij = (1 - w)(1 - q_i.k_j) + w d_ij/(r + d_ij)
// on the valid tokens of each sample (lm = -log n_valid).
//
// With s^{C,k}_ij = exp(L + u^{k-1}_i + v^k_j - lm) (columns sum to 1) and
// s^{R,k}_ij = exp(L + u^k_i + v^k_j - lm) (rows sum to 1, s^{R,K-1} = P):
//   D_i   = dxc_i.xc_i + dhc_i.hc_i,   W0_ij = -P_ij (dxc_i.x_j + dhc_i.V_j - D_i)
//   g_u   = 0 exactly (P is row-normalised), gl_v^{K-1}_j = -sum_i W0_ij
//   gl_u^{k-1}_i = -sum_j s^{C,k}_ij gl_v^k_j,   gl_v^{k}_j = -sum_i s^{R,k}_ij gl_u^k_i  (k < K-1)
//   eps dC = W0 + sum_k [ s^{C,k} diag(gl_v^k) + diag(gl_u^k) s^{R,k} ]
//   dQ = -(1-w)/eps (eps dC) K,  dK = -(1-w)/eps (eps dC)^T Q,  dV = P^T dhc,
//   dx_i += sum_j dC_ij w r/(r+d)^2 (x_i - x_j)/d  (both ends),  + P^T dxc,
//   d alpha = w(1-w) sum dC (Cgeo - Cfeat),  d r = -w sum dC d/(r+d)^2 * d|r|clamp/dr.
//
// Every gradient term is produced twice: once in a row-owned sweep (member's
// rows resident, all columns streamed), which accumulates dQ and the row ends of
// dx, and once in a column-owned sweep, which accumulates dK and the column ends.
// Sweep order (one exchange after each recurrence output):
//   CS(K-1): P, W0            -> gl_v^{K-1}, dV, P^T dxc
//   RS(k), k = K-1..0:  s^{C,k} gl_v^k (+ diag(gl_u^k) s^{R,k} for k < K-1, W0 for k = K-1)
//                             -> gl_u^{k-1}  (k >= 1)
//   CS(k), k = K-2..-1:  diag(gl_u^k) s^{R,k} (k >= 0) + s^{C,k+1} diag(gl_v^{k+1})
//                             -> gl_v^k  (k >= 0)
// so every sweep computes the cost tile once and at most two exponentials per
// element, and no cross-workgroup partial sums of N x d products are needed.
#include <type_traits>

#include "sinkhorn_bwd_kernel.h"

namespace dfl {

constexpr int BAL_NT = 512;
constexpr int BAL_NW = BAL_NT / WAVE;
// Resident tiles per wave: two at d <= 32; one at d = 64, where the accumulators
// of two tiles do not fit the register file.
template <int DP> constexpr int bal_maxt() { return DP <= 32 ? 2 : 1; }
constexpr int BAL_MAXT_ANY = 2;  // LDS sizing bound

__host__ __device__ inline int bal_wpt(int nr) { return nr >= BAL_NW ? 1 : BAL_NW / nr; }

// Prep: one thread per (b, h, i, c), c < DP.
template <int DP>
__global__ void __launch_bounds__(256) balanced_prep_kernel(BalPrepArgs p) {
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
  const size_t ro = ((size_t)bh * N + i) * d + c;  // (B,H,N,d) contiguous
  float qv = 0.f, kv = 0.f, vv = 0.f, gv = 0.f;
  if (ok && c < d) {
    qv = p.q[off];
    kv = p.k[off];
    if (p.gp) {
      vv = p.v[off];
      gv = p.ghc[ro];
    }
  }
  p.qp[row * DP + c] = qv;
  p.kp[row * DP + c] = kv;
  p.qt[((size_t)bh * DP + c) * Np + i] = qv;
  p.kt[((size_t)bh * DP + c) * Np + i] = kv;
  if (p.gp) {
    p.vp[row * DP + c] = vv;
    p.gp[row * DP + c] = gv;
    p.gt[((size_t)bh * DP + c) * Np + i] = gv;
  }
  if (c < 3) p.gxs[((size_t)bh * 3 + c) * Np + i] = (ok && p.gxc) ? p.gxc[((size_t)bh * N + i) * 3 + c] : 0.f;
  if (c < 3 && h == 0) p.xs[((size_t)b * 3 + c) * Np + i] = i < N ? p.x[((size_t)b * N + i) * 3 + c] : 0.f;
  if (c == 0) {
    float D = 0.f;
    if (ok) {
      if (p.gxc)
        for (int t = 0; t < 3; ++t) D += p.gxc[((size_t)bh * N + i) * 3 + t] * p.xc[((size_t)bh * N + i) * 3 + t];
      if (p.gp)
        for (int t = 0; t < d; ++t) D += p.ghc[((size_t)bh * N + i) * d + t] * p.hc[((size_t)bh * N + i) * d + t];
    }
    p.dcoef[(size_t)bh * Np + i] = D;
  }
}

// Finalize: dx = sum_h dx_part; d alpha, d r = sums of the workgroup partials.
__global__ void __launch_bounds__(256) balanced_finalize_kernel(BalBwdArgs a, float* dx, float* dalpha, float* dr) {
  const int e = blockIdx.x * 256 + threadIdx.x;
  const int nx = a.B * a.N * 3;
  if (e < nx) {
    const int b = e / (a.N * 3), r = e % (a.N * 3);
    dx[e] = ordered_sum(a.dx_part + (size_t)b * a.H * a.N * 3 + r, (size_t)a.N * 3, a.H, 0.f);
  } else if (e < nx + a.H) {
    const int h = e - nx;
    float sa = 0.f, sr = 0.f;
    for (int b = 0; b < a.B; ++b) {
      const float* p = a.ar_part + ((size_t)(b * a.H + h) * a.G) * 2;
      sa = ordered_sum(p, 2, a.G, sa);
      sr = ordered_sum(p + 1, 2, a.G, sr);
    }
    if (dalpha) dalpha[h] = sa;
    if (dr) dr[h] = sr;
  }
}

template <int DP>
__global__ void __launch_bounds__(BAL_NT) balanced_bwd_kernel(BalBwdArgs a) {
  using M = Mfma<float, DP>;
  constexpr int NC = DP / 16;
  constexpr int NW = BAL_NW;
  constexpr int MAXT = bal_maxt<DP>();
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ int s_flag, s_tmp, s_cnt;
  int grp, member;
  if (!group_of(a.B * a.H, a.G, grp, member)) return;
  const int b = grp / a.H, h = grp % a.H;
  const int N = a.N, d = a.d, K = a.K;
  const int Np = ((N + 31) / 32) * 32;
  const int BH = a.B * a.H;
  const size_t bh = (size_t)grp;
  const int tid = threadIdx.x, lane = tid & (WAVE - 1), wave = tid / WAVE, g = lane >> 4;
  if (tid == 0) { s_flag = 0; s_cnt = 0; }
  if (blockIdx.x == 0 && tid == 0)
    __hip_atomic_store(a.err.ws + 1, a.salt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

  // ---- LDS carve-up (must match balanced_bwd_lds_bytes)
  unsigned char* valid = smem;
  float* xs0 = reinterpret_cast<float*>(smem + ((Np + 15) / 16) * 16);
  float* xs1 = xs0 + Np;
  float* xs2 = xs1 + Np;
  float* gx0 = xs2 + Np;  // grad x_c (rows)
  float* gx1 = gx0 + Np;
  float* gx2 = gx1 + Np;
  float* dcf = gx2 + Np;  // D
  float* GLU = dcf + Np;  // gathered gl_u
  float* GLV = GLU + Np;  // gathered gl_v
  float* STA = GLV + Np;  // streamed exponent terms of the current sweep
  float* sred = STA + Np;                        // [NW][MAXT][16]
  float* spart = sred + NW * BAL_MAXT_ANY * 16;  // [NW][16*DP] part hand-over
  float* sscal = spart + NW * 16 * 64;   // [NW][2] (part region sized for DP = 64)

  const int n = mask_setup(a.mask ? a.mask + (size_t)b * N : nullptr, N, valid, &s_tmp);
  const int n_tiles = (n + 15) / 16;
  int t0, t1;
  stripe(n_tiles, member, a.G, t0, t1);
  const int nr = t1 - t0;
  // rows past the last valid tile belong to no stripe: zeroed here (row i by member i % G)
  for (int i = n_tiles * 16 + member; i < N; i += a.G) {
    for (int c = tid; c < d; c += BAL_NT) {
      a.dq[(bh * N + i) * d + c] = 0.f;
      a.dk[(bh * N + i) * d + c] = 0.f;
      if (a.dv) a.dv[(bh * N + i) * d + c] = 0.f;
    }
    if (tid < 3) a.dx_part[(bh * N + i) * 3 + tid] = 0.f;
  }
  if (n == 0 || nr <= 0) {
    if (tid < 2) a.ar_part[(bh * a.G + member) * 2 + tid] = 0.f;
    return;  // owns nothing; no other member waits on it
  }
  {
    int c = 0;
    for (int i = tid; i < n; i += BAL_NT) c += valid[i];
    atomicAdd(&s_cnt, c);
  }
  for (int i = tid; i < Np; i += BAL_NT) {
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
  __syncthreads();
  const float lm2 = -log2f((float)max(s_cnt, 1));  // log2 of the uniform marginal
  const float eps = a.eps[h];
  const float w = 1.f / (1.f + __expf(-a.alpha[h]));
  const float rh = a.r_h[h];
  const float rr = fmaxf(fabsf(rh), 0.1f);
  const float sc = LOG2E * (1.f - w) / eps;
  const float gsc = -LOG2E * w / eps;
  const int r_lo = t0 * 16;
  const float* hist = a.hist;
  auto Uh = [&](int k, int i) { return hist[((size_t)(2 * k + 1) * BH + bh) * N + i]; };
  auto Vh = [&](int k, int j) { return hist[((size_t)(2 * k) * BH + bh) * N + j]; };

  // wave -> (tile slot, part): wpt waves share a resident tile and split the streamed pairs
  const int wpt = bal_wpt(nr);
  const int nts = NW / wpt;
  const int ts = wave / wpt, part = wave % wpt;
  const int n_pairs = (n_tiles + 1) / 2;
  const float* qp = a.qp + bh * Np * DP;
  const float* kp = a.kp + bh * Np * DP;
  const float* qt = a.qt + bh * DP * Np;
  const float* kt = a.kt + bh * DP * Np;
  const float* vp = a.has_h ? a.vp + bh * Np * DP : nullptr;
  const float* gp = a.has_h ? a.gp + bh * Np * DP : nullptr;
  const float* gt = a.has_h ? a.gt + bh * DP * Np : nullptr;

  f32x4 dQa[MAXT][NC], dKa[MAXT][NC];
  // gb: sum f (x_res - x_str) with f = W (1 - cg)^2 / d, accumulated per element
  // (a split into x_res sum f - sum f x_str cancels badly where d is tiny)
  float gbx[MAXT], gby[MAXT], gbz[MAXT], xt0[MAXT], xt1[MAXT], xt2[MAXT];
#pragma unroll
  for (int s = 0; s < MAXT; ++s) {
#pragma unroll
    for (int c = 0; c < NC; ++c) dQa[s][c] = dKa[s][c] = f32x4{0.f, 0.f, 0.f, 0.f};
    gbx[s] = gby[s] = gbz[s] = xt0[s] = xt1[s] = xt2[s] = 0.f;
  }
  float s_al = 0.f, s_r = 0.f;

  uint64_t* xgu = a.xch + bh * 2 * (size_t)Np;
  uint64_t* xgv = xgu + Np;
  const uint32_t salt = a.salt << 12;
  uint32_t phase = 0;

  // Part hand-over of per-wave accumulators in the PV layout (row 4g + r, column
  // c*16 + l%16) and write-out: out[(row) * d + col] = scale * sum over parts.
  // With wpt > 1 every wave has at most one resident tile (slot 0).
  auto write_rows = [&](f32x4 (&acc)[MAXT][NC], float* out, float scale) {
    __syncthreads();
    if (wpt > 1 && part > 0 && ts < nr) {
#pragma unroll
      for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int r = 0; r < 4; ++r) spart[(size_t)wave * 16 * DP + (4 * g + r) * DP + c * 16 + (lane & 15)] = acc[0][c][r];
    }
    __syncthreads();
    if (part == 0) {
#pragma unroll
      for (int s = 0; s < MAXT; ++s) {
        const int rt = ts + nts * s;
        if (rt >= nr) continue;
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            float v = acc[s][c][r];
            for (int p = 1; p < wpt; ++p) v += spart[(size_t)(wave + p) * 16 * DP + (4 * g + r) * DP + c * 16 + (lane & 15)];
            const int row = (t0 + rt) * 16 + 4 * g + r, col = c * 16 + (lane & 15);
            if (row < N && col < d) out[(bh * N + row) * d + col] = (row < n && valid[row]) ? scale * v : 0.f;
          }
      }
    }
  };

  // One sweep.  ROW: resident rows i (streamed j), else resident columns j
  // (streamed i).  CENT: the centroid sweep of that orientation (k = K-1).
  auto sweep = [&](auto row_tag, auto cent_tag, int k) -> bool {
    constexpr bool ROW = decltype(row_tag)::value;
    constexpr bool CENT = decltype(cent_tag)::value;
    __syncthreads();  // readers of STA and of the gathered vectors are done
    for (int i = tid; i < Np; i += BAL_NT) {
      float val = NEG_BIG;
      if (i < n && valid[i]) val = ROW ? Vh(k, i) * LOG2E : (k >= 0 ? Uh(k, i) * LOG2E : 0.f) - lm2;
      STA[i] = val;
    }
    __syncthreads();
    const float* STC = ROW ? GLV : GLU;  // streamed coefficients (RS: gl_v^k, CS: gl_u^k)
    const bool use_c = ROW || (k >= 0 && k <= K - 2);
    const bool term2 = k <= K - 2;
    const bool publish = ROW ? k >= 1 : k >= 0;
    const bool hh_on = CENT && a.has_h;
    const float* Sop = ROW ? kp : qp;  // streamed operand rows
    const float* Sot = ROW ? kt : qt;  // streamed operand, transposed (product)
    const float* Rop = ROW ? qp : kp;  // resident operand rows

    // resident-side values of this wave's tiles
    typename M::Frag bf[MAXT], cbf[MAXT];
    float ab[MAXT], dl[MAXT], dd[MAXT], xr0[MAXT], xr1[MAXT], xr2[MAXT], Dr[MAXT], gr0[MAXT], gr1[MAXT], gr2[MAXT];
    float red[MAXT];
    f32x4 gVa[MAXT][NC];
#pragma unroll
    for (int s = 0; s < MAXT; ++s) {
      const int rt = ts + nts * s;
      const int ri = (t0 + min(rt, nr - 1)) * 16 + (lane & 15);  // in [0, Np)
      const bool ok = rt < nr && ri < n && valid[ri];
      M::load(bf[s], Rop + (size_t)ri * DP, lane);
      if (hh_on) M::load(cbf[s], (ROW ? gp : vp) + (size_t)ri * DP, lane);
      Dr[s] = gr0[s] = gr1[s] = gr2[s] = 0.f;
      if (CENT && ROW) {
        Dr[s] = dcf[ri];
        gr0[s] = gx0[ri];
        gr1[s] = gx1[ri];
        gr2[s] = gx2[ri];
      }
      if (ROW) {
        const float up = (k >= 1 && ok) ? Uh(k - 1, ri) : 0.f;
        ab[s] = ok ? up * LOG2E - lm2 : NEG_BIG;
        dl[s] = ok ? (Uh(k, ri) - up) * LOG2E : 0.f;
        dd[s] = term2 ? GLU[ri] : 0.f;
      } else {
        ab[s] = ok ? Vh(max(k, 0), ri) * LOG2E : NEG_BIG;
        dl[s] = (ok && k >= 0 && k <= K - 2) ? (Vh(k + 1, ri) - Vh(k, ri)) * LOG2E : 0.f;
        dd[s] = term2 ? GLV[ri] : 0.f;
      }
      xr0[s] = xs0[ri];
      xr1[s] = xs1[ri];
      xr2[s] = xs2[ri];
      red[s] = 0.f;
#pragma unroll
      for (int c = 0; c < NC; ++c) gVa[s][c] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    if (ts < nts) {
      for (int sp = part; sp < n_pairs; sp += wpt) {
#pragma unroll
        for (int s = 0; s < MAXT; ++s) {
          const int rt = ts + nts * s;
          if (rt >= nr) continue;
          f32x4 wop[2], pop[2];
#pragma unroll
          for (int hh = 0; hh < 2; ++hh) {
            // streamed tile st (< Np / 16; rows past n are zero and masked)
            const int st = 2 * sp + hh;
            const int o = st * 16 + 4 * g;
            typename M::Frag af;
            M::load(af, Sop + (size_t)(st * 16 + (lane & 15)) * DP, lane);
            const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
            f32x4 t = zero;
            if (hh_on) {
              typename M::Frag cf;
              M::load(cf, (ROW ? vp : gp) + (size_t)(st * 16 + (lane & 15)) * DP, lane);
              t = M::qk(cf, cbf[s], zero);
            }
            const f32x4 x = M::qk(af, bf[s], zero);
            const f32x4 sa = *reinterpret_cast<const f32x4*>(STA + o);
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
              const float dx = xr0[s] - sx0[e], dy = xr1[s] - sx1[e], dz = xr2[s] - sx2[e];
              const float dist = fmaxf(sqrtf(dx * dx + dy * dy + dz * dz), 1e-8f);
              const float cg = dist / (rr + dist);
              const float lg = __builtin_fmaf(x[e], sc, gsc * cg) + sa[e] + ab[s];
              const float e1 = fast_exp2(lg);
              const float e2 = (term2 || (CENT && ROW)) ? fast_exp2(lg + dl[s]) : 0.f;
              float W = 0.f;
              if (use_c) {
                const float t1 = e1 * scf[e];
                W = t1;
                red[s] -= t1;
              }
              if (term2) W = __builtin_fmaf(e2, dd[s], W);
              if (CENT) {
                const float P = ROW ? e2 : e1;
                float dT = t[e];
                if (ROW) dT += gr0[s] * sx0[e] + gr1[s] * sx1[e] + gr2[s] * sx2[e];
                else dT += sg0[e] * xr0[s] + sg1[e] * xr1[s] + sg2[e] * xr2[s];
                const float qv = P * (dT - (ROW ? Dr[s] : sD[e]));
                W -= qv;
                if (!ROW) {
                  red[s] += qv;
                  xt0[s] = __builtin_fmaf(P, sg0[e], xt0[s]);
                  xt1[s] = __builtin_fmaf(P, sg1[e], xt1[s]);
                  xt2[s] = __builtin_fmaf(P, sg2[e], xt2[s]);
                  pop[hh][e] = P;
                }
              }
              wop[hh][e] = W;
              const float om = 1.f - cg;
              const float f = W * om * om / dist;
              gbx[s] = __builtin_fmaf(f, dx, gbx[s]);
              gby[s] = __builtin_fmaf(f, dy, gby[s]);
              gbz[s] = __builtin_fmaf(f, dz, gbz[s]);
              if (ROW) {
                s_al = __builtin_fmaf(W, cg - 1.f + x[e], s_al);
                s_r = __builtin_fmaf(W, cg * om, s_r);
              }
            }
          }
#pragma unroll
          for (int c = 0; c < NC; ++c) {
            const float* vt_row = Sot + (size_t)(c * 16 + (lane & 15)) * Np + sp * 32;
            if (ROW) dQa[s][c] = M::pv(wop[0], wop[1], vt_row, lane, dQa[s][c]);
            else dKa[s][c] = M::pv(wop[0], wop[1], vt_row, lane, dKa[s][c]);
            if (CENT && !ROW && a.has_h)
              gVa[s][c] = M::pv(pop[0], pop[1], gt + (size_t)(c * 16 + (lane & 15)) * Np + sp * 32, lane, gVa[s][c]);
          }
        }
      }
    }
    // recurrence output: sum over lane groups, then over the parts of each tile
#pragma unroll
    for (int s = 0; s < MAXT; ++s) {
      const float r = sum_groups(red[s]);
      if (lane < 16) sred[(wave * MAXT + s) * 16 + lane] = r;
    }
    __syncthreads();
    if (publish) {
      ++phase;
      const uint32_t tag = salt | phase;
      uint64_t* buf = ROW ? xgu : xgv;
      for (int q = tid; q < nr * 16; q += BAL_NT) {
        const int rt = q >> 4, l16 = q & 15;
        const int s = rt / nts, tsl = rt % nts;
        float v = 0.f;
        for (int p = 0; p < wpt; ++p) v += sred[((tsl * wpt + p) * MAXT + s) * 16 + l16];
        const int i = r_lo + q;
        if (i < n) xch_put(buf + i, v, tag);
      }
      if (!gather_vector(buf, n, Np, tag, ROW ? GLU : GLV, valid, a.err, &s_flag)) return false;
    }
    if (CENT && !ROW) {
      if (a.dv) write_rows(gVa, a.dv, 1.f);
    }
    return true;
  };

  using TRUE_ = std::integral_constant<bool, true>;
  using FALSE_ = std::integral_constant<bool, false>;
  if (!sweep(FALSE_{}, TRUE_{}, K - 1)) return;
  if (!sweep(TRUE_{}, TRUE_{}, K - 1)) return;
  for (int k = K - 2; k >= 0; --k) {
    if (!sweep(FALSE_{}, FALSE_{}, k)) return;
    if (!sweep(TRUE_{}, FALSE_{}, k)) return;
  }
  if (!sweep(FALSE_{}, FALSE_{}, -1)) return;

  // ---- outputs of my stripe
  const float fs = -(1.f - w) / eps;
  write_rows(dQa, a.dq, fs);
  write_rows(dKa, a.dk, fs);
  // dx: (w / (eps r)) gb + P^T dxc, summed over lane groups and parts
  __syncthreads();
#pragma unroll
  for (int s = 0; s < MAXT; ++s) {
    const float v[6] = {sum_groups(gbx[s]), sum_groups(gby[s]), sum_groups(gbz[s]),
                        sum_groups(xt0[s]), sum_groups(xt1[s]), sum_groups(xt2[s])};
    if (lane < 16)
      for (int t = 0; t < 6; ++t) spart[((size_t)(wave * MAXT + s) * 16 + lane) * 6 + t] = v[t];
  }
  {
    const float sa_w = wave_sum(s_al), sr_w = wave_sum(s_r);
    if (lane == 0) {
      sscal[wave * 2] = sa_w;
      sscal[wave * 2 + 1] = sr_w;
    }
  }
  __syncthreads();
  const float gs = w / (eps * rr);
  for (int q = tid; q < nr * 16; q += BAL_NT) {
    const int rt = q >> 4, l16 = q & 15;
    const int s = rt / nts, tsl = rt % nts;
    float v[6] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int p = 0; p < wpt; ++p)
      for (int t = 0; t < 6; ++t) v[t] += spart[((size_t)((tsl * wpt + p) * MAXT + s) * 16 + l16) * 6 + t];
    const int i = r_lo + q;
    if (i < N) {
      const bool ok = i < n && valid[i];
      for (int t = 0; t < 3; ++t) a.dx_part[(bh * N + i) * 3 + t] = ok ? gs * v[t] + v[3 + t] : 0.f;
    }
  }
  if (tid == 0) {
    float sa_t = 0.f, sr_t = 0.f;
    for (int wv = 0; wv < NW; ++wv) {
      sa_t += sscal[wv * 2];
      sr_t += sscal[wv * 2 + 1];
    }
    const float dsign = fabsf(rh) >= 0.1f ? (rh > 0.f ? 1.f : (rh < 0.f ? -1.f : 0.f)) : 0.f;
    a.ar_part[(bh * a.G + member) * 2 + 0] = w * (1.f - w) / eps * sa_t;
    a.ar_part[(bh * a.G + member) * 2 + 1] = -(w / (eps * rr)) * sr_t * dsign;
  }
}

size_t balanced_bwd_lds_bytes(int N, int DP) {
  (void)DP;
  const size_t Np = ((N + 31) / 32) * 32;
  size_t bytes = ((Np + 15) / 16) * 16;
  bytes += 10 * Np * 4;                               // coordinates, grad x_c, D, gathered vectors, STA
  bytes += (size_t)BAL_NW * BAL_MAXT_ANY * 16 * 4;    // recurrence partials
  bytes += (size_t)BAL_NW * 16 * 64 * 4;              // part hand-over (>= the dx hand-over, NW*2*16*6)
  bytes += BAL_NW * 2 * 4;
  return bytes;
}

// Largest resident-tile count per member the kernel supports.
int balanced_max_tiles(int DP) { return (DP <= 32 ? bal_maxt<32>() : bal_maxt<64>()) * BAL_NW; }

hipError_t launch_balanced_prep(const BalPrepArgs& p, int DP, hipStream_t stream) {
  const int Np = ((p.N + 31) / 32) * 32;
  const size_t total = (size_t)p.B * p.H * Np * DP;
  const unsigned blocks = (unsigned)((total + 255) / 256);
  if (DP == 32) hipLaunchKernelGGL(balanced_prep_kernel<32>, dim3(blocks), dim3(256), 0, stream, p);
  else if (DP == 64) hipLaunchKernelGGL(balanced_prep_kernel<64>, dim3(blocks), dim3(256), 0, stream, p);
  else return hipErrorInvalidValue;
  return hipGetLastError();
}

template <int DP>
static hipError_t launch_bal_t(const BalBwdArgs& a, size_t lds, hipStream_t stream, bool coop) {
  auto kern = balanced_bwd_kernel<DP>;
  hipError_t e = set_lds_limit((const void*)kern, lds);
  if (e != hipSuccess) return e;
  dim3 grid(grid_blocks(a.B * a.H, a.G)), block(BAL_NT);
  BalBwdArgs copy = a;
  if (coop) {
    void* args[] = {&copy};
    return hipLaunchCooperativeKernel((const void*)kern, grid, block, args, (unsigned)lds, stream);
  }
  hipLaunchKernelGGL(kern, grid, block, lds, stream, copy);
  return hipGetLastError();
}

hipError_t launch_balanced_bwd(const BalBwdArgs& a, int DP, size_t lds, hipStream_t stream, bool coop) {
  if (DP == 32) return launch_bal_t<32>(a, lds, stream, coop);
  if (DP == 64) return launch_bal_t<64>(a, lds, stream, coop);
  return hipErrorInvalidValue;
}

hipError_t launch_balanced_finalize(const BalBwdArgs& a, float* dx, float* dalpha, float* dr, hipStream_t stream) {
  const int total = a.B * a.N * 3 + a.H;
  hipLaunchKernelGGL(balanced_finalize_kernel, dim3((total + 255) / 256), dim3(256), 0, stream, a, dx, dalpha, dr);
  return hipGetLastError();
}

}  // namespace dfl
