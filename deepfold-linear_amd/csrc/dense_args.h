// Argument blocks of the dense (materialised-cost) Sinkhorn kernels and the C ABI.
#pragma once
#include <stdint.h>

namespace dfl {

// sinkhorn_solve forward.  All fp32, contiguous: C (B,H,N,N), log_mu / log_nu /
// inits (B,H,N), eps (H), mask (B,N) or null.  hist_* hold K+1 slices of (B,H,N):
// u_k, v_k (slice 0 = the initial potentials) and the LSEs r_k, c_k (k >= 1).
struct DenseSinkArgs {
  const float* C;
  const float* log_mu;
  const float* log_nu;
  const float* eps;
  const float* u_init;
  const float* v_init;
  const float* mask;
  int B, H, N, K;
  float lam;
  float* hist_u;
  float* hist_v;
  float* hist_r;
  float* hist_c;
  uint32_t* delta;  // 2 (K+1) words: max |u_k - u_{k-1}|, max |v_k - v_{k-1}| (float bits), or null
  float* log_u;     // outputs (masked)
  float* log_v;
};

// sinkhorn_solve backward through the K executed iterations.
struct DenseSinkBwdArgs {
  const float* C;
  const float* eps;
  const float* mask;
  const float* hist_u;
  const float* hist_v;
  const float* hist_r;
  const float* hist_c;
  int B, H, N, K;
  float lam;
  const float* grad_u;  // (B,H,N) or null
  const float* grad_v;
  float* dC;            // (B,H,N,N)
  float* dlog_mu;       // (B,H,N)
  float* dlog_nu;
  float* dlog_u_init;   // or null
  float* dlog_v_init;   // or null
  float* gv;            // workspace (B,H,N): g_v of the current iteration
  float* avec;          // workspace (B,H,N): -kappa g_u of the current iteration
};

// compute_transport_output forward / backward.  V, G, o_avg, goa (B,H,N,d) with d <= 64.
struct DenseTransportArgs {
  const float* V;
  const float* G;       // or null
  const float* log_u;
  const float* log_v;
  const float* C;
  const float* eps;
  const float* x_res;   // (B,N,3) or null
  const float* mask;    // (B,N) or null
  int B, H, N, d;
  float* o;             // (B,N,H*d)
  float* T_norm;        // (B,H,N,N)
  float* x_centroid;    // (B,H,N,3) or null
  float* o_avg;         // (B,H,N,d) saved for the backward
  // backward
  const float* grad_o;  // (B,N,H*d) or null
  const float* grad_T;  // (B,H,N,N) or null
  const float* grad_xc; // (B,H,N,3) or null
  float* dV;
  float* dG;            // or null
  float* dlog_u;
  float* dlog_v;
  float* dC;
  float* dx_res;        // (B,N,3) or null
  float* goa;           // workspace (B,H,N,d)
  float* dx_part;       // workspace (B,H,N,3), or null without x_res
};

}  // namespace dfl
