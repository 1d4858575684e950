// Argument blocks shared by the Sinkhorn kernels and the C-ABI layer.
#pragma once
#include <stdint.h>

#include "common.h"

namespace dfl {

// Workgroups launched for n_groups groups of G members: whole 8-XCD slots.
inline int grid_blocks(int n_groups, int G) { return 8 * ((n_groups + 7) / 8) * G; }

// Forward (flash_sinkhorn_attn.py:77-244 semantics).
struct SinkFwdArgs {
  const void* q;  // (B,H,N,d) bf16 or fp32, element strides sb/sh/sn, unit inner stride
  const void* k;
  const void* v;
  const void* g;  // gate logits, same layout (may be null: gate treated as +inf -> sigma = 1)
  long long sb, sh, sn;
  const float* x;       // (B,N,3) contiguous or null (zeros)
  const float* pos_w;   // (H,68) or null
  const int* bins;      // (B,N,N) int32 contiguous or null
  const float* eps;     // (H,)
  const float* w_dist;  // (H,) or null
  const float* log_mu;  // (B,H,N)
  const float* log_nu;  // (B,H,N)
  const float* u_init;  // (B,H,N) or null
  const float* v_init;  // (B,H,N) or null
  const float* mask;    // (B,N) or null
  int B, H, N, d;
  int K_iter;
  float lam, r0;
  // outputs (every position written; zeros where padded)
  float* o_flat;      // (B,N,H*d)
  float* x_centroid;  // (B,H,N,3)
  float* log_u;       // (B,H,N)
  float* log_v;       // (B,H,N)
  float* o_avg;       // (B,H,N,d)  saved for the backward
  float* log_z;       // (B,H,N)    LSE_j(u_i + L_ij + v_j)
  float* col_lse;     // (B,H,N)    LSE_i(L_ij + u_i) of the last column update
  // workspace
  uint64_t* xch;  // B*H*2*Np exchange words
  ErrRef err;     // error word (workspace) and host mailbox
  int G;          // workgroups per (b,h)
  uint32_t salt;  // 20-bit call salt for exchange tags
  // stream mode only (sinkhorn_pad_kernel output): zero-padded operand copies
  const void* qp;     // [B*H][Np][DP]
  const void* kp;     // [B*H][Np][DP]
  const void* vt;     // [B*H][DP][Np]
  const float* xs_p;  // [B][Np][3]
  // padded uint8 bins (bins8_kernel), row-major and transposed, [B][Np][Np] (null without bins)
  const uint8_t* bins8;
  const uint8_t* bins8t;
  // Balanced transport mode (flash_sinkhorn_transport.py:253-282, 289-320): column
  // update first, kappa = 1, uniform marginals -log(n_valid) per sample, cost
  // (1 - w_h)(1 - q.k) + w_h d/(r + d) with w_h = sigmoid(alpha_h), r = max(|r_h|, 0.1).
  // log_mu / log_nu / g / o_flat / col_lse are unused (may be null); v may be null.
  int balanced;
  const float* alpha;  // (H,)
  const float* r_h;    // (H,)
  float* hist;         // (K_iter, 2, B*H, N): v after the column update, u after the row update
                       // (both modes; null = not recorded)
};

// Backward (flash_sinkhorn_attn.py:246-667 semantics, plus analytic mode / CG).
struct SinkBwdArgs {
  const void* q;
  const void* k;
  const void* v;
  const void* g;
  long long sb, sh, sn;
  const float* x;
  const float* pos_w;
  const int* bins;
  const float* eps;
  const float* w_dist;
  const float* mask;
  const float* log_u;     // (B,H,N) forward outputs
  const float* log_v;
  const float* log_z;     // (B,H,N)
  const float* col_lse;   // (B,H,N)
  const float* o_avg;     // (B,H,N,d)
  const float* x_centroid;  // (B,H,N,3)
  const float* grad_o;    // (B,N,H*d) fp32
  const float* grad_xc;   // (B,H,N,3) fp32 or null
  int B, H, N, d;
  float lam, r0;
  int solver;   // 0 = fixed point (reference Gauss-Seidel), 1 = CG
  int iters;    // fixed-point sweeps or CG iterations
  int mode;     // 0 = reference signs, 1 = analytic adjoint
  float cg_rtol;  // CG early stop on ||r|| <= rtol ||b|| (0 = run all iterations)
  int geo_grad;   // compute d x_res / d w_dist cost terms (x given and requested)
  // outputs (every position written; zeros where padded)
  void* dq;         // (B,H,N,d) in the input type T
  void* dk;
  void* dv;
  void* dg;
  float* dlog_mu;   // (B,H,N)
  float* dlog_nu;
  float* dx_part;   // (B,H,N,3) per-head partials, summed over h by the finaliser
  float* dpw_part;  // (B*H*G, 68) per-workgroup partials
  float* dw_part;   // (B*H*G) per-workgroup partials
  // workspace
  uint64_t* xch;  // B*H*4*Np exchange words
  ErrRef err;
  // prepared by the prep kernel (per (b,h), Np rows, zero on invalid rows / padded columns):
  void* go_hi;    // [B*H][Np][DP]  T(gO), gO = sigma(G) * dO
  void* go_lo;    // [B*H][Np][DP]  T(gO - T(gO)) (bf16 inputs only)
  void* go_t;     // [B*H][DP][Np]  T(gO) transposed
  float* dcoef;   // [B*H][Np]      D_i = gO_i.O_avg_i + dxc_i.xc_i
  int G;
  uint32_t salt;
  int ch;         // streamed rows per LDS chunk in the heavy passes (multiple of 32)
  // stream mode only
  const void* qp;  // [B*H][Np][DP] zero-padded copies (sinkhorn_pad_kernel)
  const void* kp;
  float* vec_ws;   // per-workgroup vectors, BWD_STREAM_VECS * Np floats each
  const uint8_t* bins8;   // padded uint8 bins [B][Np][Np] and transposed (null without bins)
  const uint8_t* bins8t;
  // per-head bias computed once (bias_mat_kernel), [B*H][Np][Np] and transposed, or null
  const float* bias_mat;
  const float* bias_matT;
};

// Unrolled backward of the balanced transport (flash_sinkhorn_transport.py:322-373,
// 448-516).  fp32 operands; every prepared array is per (b,h) with Np rows, zero
// on masked rows, rows >= N and columns >= d.
struct BalBwdArgs {
  int B, H, N, d, K;
  const float* eps;    // (H,)
  const float* alpha;  // (H,)
  const float* r_h;    // (H,)
  const float* mask;   // (B,N) or null
  const float* hist;   // (K, 2, B*H, N) forward potentials (natural log)
  const float* qp;     // [B*H][Np][DP]
  const float* kp;
  const float* qt;     // [B*H][DP][Np]
  const float* kt;
  const float* vp;     // [B*H][Np][DP]  V            (h centroid only)
  const float* gp;     // [B*H][Np][DP]  grad h_c     (h centroid only)
  const float* gt;     // [B*H][DP][Np]  grad h_c transposed
  const float* dcoef;  // [B*H][Np]      D_i = dxc_i.xc_i + dhc_i.hc_i
  const float* gxs;    // [B*H][3][Np]   grad x_c, coordinate-major
  const float* xs;     // [B][3][Np]     coordinates, coordinate-major
  int has_h;           // grad h_c given
  float* dq;           // (B,H,N,d)
  float* dk;
  float* dv;           // (B,H,N,d) or null
  float* dx_part;      // (B,H,N,3) per-head partials
  float* ar_part;      // (B*H*G, 2) per-workgroup d alpha, d r partials
  uint64_t* xch;       // B*H*2*Np exchange words
  ErrRef err;
  int G;
  uint32_t salt;
};

// Unrolled backward of the UOT flash-Sinkhorn (the reference's GPU-path backward,
// sinkhorn_kernel.py:2085-2382): prepared fp32 operands as for the balanced one.
struct UnrBwdArgs {
  int B, H, N, d, K;
  const float* eps;      // (H,)
  float lam, r0;
  const float* mask;     // (B,N) or null
  const float* hist;     // (K, 2, B*H, N): v after the column update, u after the row update
  const float* log_mu;   // (B,H,N)
  const float* log_nu;
  const float* log_u;    // (B,H,N) forward outputs: final u and LSE_j(u + L + v)
  const float* log_z;
  const float* v_init;   // (B,H,N) or null (zeros)
  const uint8_t* bins8;  // padded uint8 bins [B][Np][Np] (bins8_kernel) or null
  const uint8_t* bins8t; // transposed copy (unused here)
  const float* pos_w;    // (H,68) or null
  const float* w_dist;   // (H,) or null
  int has_geo;           // geometry term present (x given and w_dist given)
  const void* qp;        // [B*H][Np][DP] copies in the input type, zero on masked rows / padding
  const void* kp;
  const void* qt;        // [B*H][DP][Np] in the input type
  const void* kt;
  const float* vp;       // V rows
  const float* gp;       // gO rows (gO = sigma(G) dO)
  const float* gt;       // gO transposed
  const float* dcoef;    // [B*H][Np] D_i = gO_i.O_i + dxc_i.xc_i
  const float* gxs;      // [B*H][3][Np] grad x_c
  const float* xs;       // [B][3][Np] coordinates
  void* dq;              // (B,H,N,d) in the input type
  void* dk;
  void* dv;
  float* dlog_mu;        // (B,H,N)
  float* dlog_nu;
  float* dv_init;        // (B,H,N) or null
  float* dx_part;        // (B,H,N,3)
  float* dpw_part;       // (B*H*G, 68)
  float* dw_part;        // (B*H*G)
  uint64_t* xch;
  ErrRef err;
  int G;
  uint32_t salt;
};

struct UnrPrepArgs {
  const void* q;  // (B,H,N,d) bf16 or fp32, element strides sb/sh/sn
  const void* k;
  const void* v;
  const void* g;  // gate logits or null
  long long sb, sh, sn;
  const float* x;        // (B,N,3) or null
  const float* mask;     // (B,N) or null
  const float* o_avg;    // (B,H,N,d) forward output
  const float* xc;       // (B,H,N,3) forward output
  const float* grad_o;   // (B,N,H*d) fp32
  const float* grad_xc;  // (B,H,N,3) or null
  int B, H, N, d;
  void* qp; void* kp;    // in the input type (the MFMA operands of the cost recompute and of dQ, dK)
  void* qt; void* kt;
  float* vp; float* gp; float* gt;
  float* dcoef; float* gxs; float* xs;
  void* dg;              // (B,H,N,d) in the input type, or null (no gate)
};

struct BalPrepArgs {
  const float* q;  // (B,H,N,d) fp32, element strides sb/sh/sn, unit inner stride
  const float* k;
  const float* v;  // or null
  long long sb, sh, sn;
  const float* x;      // (B,N,3)
  const float* mask;   // (B,N) or null
  const float* xc;     // (B,H,N,3) forward x centroid
  const float* hc;     // (B,H,N,d) forward h centroid (null without grad_hc)
  const float* gxc;    // (B,H,N,3) or null
  const float* ghc;    // (B,H,N,d) or null
  int B, H, N, d;
  float* qp; float* kp; float* qt; float* kt;
  float* vp; float* gp; float* gt;  // null without grad_hc
  float* dcoef; float* gxs; float* xs;
};

// Zero-padded operand copies for stream mode, written by sinkhorn_pad_kernel.
struct PadArgs {
  const void* q;
  const void* k;
  const void* v;
  long long sb, sh, sn;
  const float* x;     // (B,N,3) or null
  const float* mask;  // (B,N) or null
  int B, H, N, d;
  void* qp;     // [B*H][Np][DP]
  void* kp;     // [B*H][Np][DP]
  void* vt;     // [B*H][DP][Np] (null: not needed)
  float* xs_p;  // [B][Np][3] (null: not needed)
};

}  // namespace dfl
