// Argument blocks of the TokenOTBlock steps either side of the balanced transport
// (src/deepfold/model/trunk_block.py:165-175 and :189-204): the fused sink
// projections and the gated coordinate update.
#pragma once
#include <cstddef>

namespace dfl {

// LN -> Q/K/V sink projections -> per-head L2 normalisation of Q and K.
struct ProjArgs {
  const void* h;                    // (M, C) of T (bf16 or fp32), row stride C
  const float* ln_w;                // (C) LayerNorm weight and bias
  const float* ln_b;
  const void* w[3];                 // (C, C) of T: nn.Linear weights (out, in) of q, k, v; w[2] may be null
  float* y[3];                      // forward outputs (M, C) fp32; y[0], y[1] normalised per head
  float* norm[2];                   // (M, H) norms of q and k before normalisation
  float* mean;                      // (M) LayerNorm statistics
  float* rstd;
  // backward
  const float* dy[3];               // (M, C) upstream gradients, null = zero
  float* du[3];                     // workspace: gradients of the pre-normalisation projections
  float* xa;                        // workspace (M, C): LayerNorm output (recomputed)
  float* xn;                        // workspace (M, C): normalised input before the affine map
  float* dxa;                       // workspace (M, C): gradient of the LayerNorm output
  float* dh;                        // (M, C) fp32 gradient of h
  float* dln_w;                     // (C)
  float* dln_b;
  float* dw[3];                     // (C, C) fp32
  float* part;                      // workspace: per-workgroup LayerNorm parameter partials
  int M, C, H;
};

// Up to three GEMMs per launch (blockIdx.z), each C[i][j] = sum_k A(i, k) B(j, k) in
// fp32 with the k range split into nseg segments of kseg, segment s reading A[z + s]
// and B[z + s] (one launch sums the three projections' products):
// A(i, k) = A[k * lda + i] when A is K-major, else A[i * lda + k]; B likewise.
struct GemmArgs {
  const float* A[3];
  const void* B[3];  // fp32 or bf16 (see the launcher)
  float* C[3];
  long long lda, ldb, ldc;
  int m, n, kseg, nseg;
};

// Sums of per-workgroup partial rows: out_s[c] = sum_r part[r][off_s + c], c < n_s.
struct SumSegs {
  const float* part;
  int rows, width, nseg;
  int off[5], n[5];
  float* out[5];
};

// x <- x + mask * sigmoid(w_gate . LN(h) + b_gate) * sum_h tanh(lambda_h) / H * (x_c,h - x)
struct CoordArgs {
  const void* h;        // (B*N, C) of T
  const float* ln_w;    // (C)
  const float* ln_b;
  const float* w_gate;  // (C)
  const float* b_gate;  // (1)
  const float* lam_raw; // (H)
  const float* xc;      // (B, H, N, 3)
  const float* x;       // (B, N, 3)
  const float* mask;    // (B, N) or null
  float* x_out;         // (B, N, 3)
  // backward
  const float* dx_out;  // (B, N, 3)
  float* dx;            // (B, N, 3)
  float* dxc;           // (B, H, N, 3)
  float* dh;            // (B*N, C) fp32
  float* dln_w;         // (C)
  float* dln_b;
  float* dw_gate;       // (C)
  float* db_gate;       // (1)
  float* dlam_raw;      // (H)
  float* part;          // workspace: per-workgroup partials, width 3C + H + 1
  int B, N, C, H;
};

}  // namespace dfl
