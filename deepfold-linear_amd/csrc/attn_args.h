// Argument block of the softmax-attention kernels (attention.hip) shared with the
// C-ABI layer.
#pragma once
#include <stdint.h>

namespace dfl {

enum AttnBias : int { ATTN_BIAS_NONE = 0, ATTN_BIAS_BINS = 1, ATTN_BIAS_DENSE = 2, ATTN_BIAS_WINDOW = 3 };

// Windowed attention geometry (flash_atom_attn.py: W_QUERY = 32, W_KEY = 128):
// window w = i / 32 holds queries [32w, 32w + 32) and keys [32w - 48, 32w + 80).
constexpr int ATTN_WQ = 32;
constexpr int ATTN_WK = 128;
constexpr int ATTN_WOFF = 48;

// O = softmax(scale Q K^T + bias, key mask) V, query-masked rows zero, optional
// sigmoid gate on the output.  Queries (B,H,Mq,d), keys/values (B,H,Nk,d).
struct AttnArgs {
  const void* q;  // element strides qsb/qsh/qsn, unit inner stride
  const void* k;
  const void* v;  // same strides as k
  const void* g;  // gate logits (B,H,Mq,d) with q's strides, or null
  long long qsb, qsh, qsn;
  long long ksb, ksh, ksn;
  const float* qmask;  // (B,Mq) or null
  const float* kmask;  // (B,Nk) or null
  int bias_mode;       // AttnBias
  const float* pos_w;  // (H,68)            ATTN_BIAS_BINS
  const int* bins;     // (B,Mq,Nk) int32   ATTN_BIAS_BINS
  const void* bias;    // (B,H,Mq,Nk) dense, or (ceil(Mq/32),H,32,128) window; element type of q
  int window;          // 1: windowed key ranges
  int B, H, Mq, Nk, d;
  float scale;
  // forward outputs
  void* o;     // (B,H,Mq,d) contiguous, element type of q (gated if g)
  float* lse;  // (B,H,Mq) natural-log row LSE of the scores (0 on masked rows)
  // backward inputs / outputs
  const void* dout;  // (B,H,Mq,d) contiguous, element type of q
  void* dq;          // (B,H,Mq,d) contiguous
  void* dk;          // (B,H,Nk,d) contiguous
  void* dv;
  void* dg;          // (B,H,Mq,d) or null
  void* dbias;       // same layout as bias, or null
  float* dpos_w;     // (H,68) or null
  // workspace
  void* do_w;        // [B*H][Mq][DP] element type of q: sigma(G) dO (or dO), zero on masked rows
  float* dcoef;      // [B*H][Mq]  D_i = sum_c dO_ic O_ic
  float* kv_part;    // [qsplit][B*H][Nk][2][DP] fp32 partial dK / dV (qsplit > 1)
  float* dpw_part;   // [B*H][ceil(Mq/64)][68] fp32 bins-gradient partials of the dQ pass
  void* dbias_rows;  // window bias, B > 1: [B][ceil(Mq/32)*H*32*128] per-batch-row gradients (type of q)
  int qsplit;        // query-range splits of the dK/dV pass
};

// Atom-to-token attention (per-token atom ranges).
struct A2TArgs {
  const void* q;   // (B,H,N,d) contiguous
  const void* k;   // (B,H,M,d) contiguous
  const void* v;
  const int* starts;  // (B,N)
  const int* counts;  // (B,N)
  const float* tmask; // (B,N) or null
  int B, H, N, M, d;
  float scale;
  void* o;            // (B,H,N,d)
  float* lse;         // (B,H,N)
  const void* dout;   // (B,H,N,d)
  void* dq;           // (B,H,N,d)
  float* dkv;         // (B,H,M,2,d) fp32 accumulators (zeroed by the backward launcher)
  void* dk;           // (B,H,M,d)
  void* dv;
};

}  // namespace dfl
