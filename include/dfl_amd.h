/*
 * deepfold_amd C ABI: MI355X (gfx950) kernels for DeepFold-Linear's flash-Sinkhorn
 * optimal-transport attention, its implicit-function-theorem backward, and the
 * neighbouring flash diffusion / atom-window / atom<->token cross attention.
 *
 * Conventions (every entry point):
 *  - Plain device pointers, explicit shapes and element strides, a dtype enum;
 *    no torch types.  Accumulation is fp32; Sinkhorn potentials and outputs are
 *    fp32, attention outputs and gradients use the element type of q.
 *  - The caller allocates every output; the kernels write every position of it
 *    (zeros at padded positions), so no initialisation is needed, except where
 *    an entry point says otherwise.  The caller also provides a workspace of
 *    dfl_*_workspace_size() bytes.  A workspace
 *    must be zero-filled once when it is first allocated; after that it may be
 *    reused by any number of calls without clearing.  Calls that share a
 *    workspace must not overlap in time.
 *  - Work is enqueued on `stream` (a hipStream_t; NULL = default stream).  The
 *    library never allocates device memory and never synchronises.
 *  - Return value: 0 = success, < 0 = argument error (see dfl_last_error()),
 *    > 0 = hipError_t of a failed launch.
 *  - Kernels that wait on other workgroups have bounded spins; if a wait ever
 *    expires the kernel exits (its outputs are then invalid) and records an
 *    error in the workspace, which dfl_workspace_error() reports (it
 *    synchronises `stream`), and in a pinned host word, which
 *    dfl_pending_error() reads without synchronising.
 *  - Exchange words are tagged with a 20-bit call salt chosen on the host per
 *    call.  When the salt wraps (every 2^20 calls), the first call on each
 *    workspace clears that workspace's exchange region with a fill kernel on its
 *    stream.  Because the salt is fixed at call time, the workspace entry points
 *    of the persistent kernels refuse a stream that is capturing a HIP graph
 *    (argument error); dfl_sinkhorn_fwd_noalloc is the capturable forward.
 */
#ifndef DFL_AMD_H
#define DFL_AMD_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

enum dfl_dtype { DFL_BF16 = 0, DFL_F32 = 1 };

/* Thread-local message for the last failed call on this thread. */
const char* dfl_last_error(void);

/* Library version string. */
const char* dfl_version(void);

/* Reports (and clears nothing) the error recorded by the most recent call that
 * used `workspace`: 0 = none, else the kernel's error code.  Synchronises `stream`. */
int dfl_workspace_error(const void* workspace, void* stream);

/* Error code of a kernel wait that expired in any launch since the last call to
 * this function (0 = none), read from pinned host memory that such a kernel writes:
 * no synchronisation, so it sees what completed kernels reported.  Clears it.
 * The reference has no counterpart: its ops fall back to the CPU on any exception
 * (flash_sinkhorn_attn.py:144, 751); here a failure is reported, never hidden. */
int dfl_pending_error(void);

/* Launch mode of the persistent kernels (the Sinkhorn forward and backwards), whose
 * workgroups wait on each other and so must all be resident at once.  No counterpart
 * in the reference, whose Triton launches are independent (sinkhorn_kernel.py:1991-2011).
 *  DFL_LAUNCH_AUTO (default): grids of at most one workgroup per CU are ordinary
 *    launches.  On an otherwise idle device all workgroups are resident.  If other
 *    kernels hold CUs (concurrent streams), a workgroup that cannot start leaves the
 *    others polling: their waits give up after about 2-4 s, the call's outputs are
 *    invalid, and error 2 is reported by dfl_pending_error() / dfl_workspace_error().
 *  DFL_LAUNCH_ORDINARY: always ordinary launches.
 *  DFL_LAUNCH_COOPERATIVE: cooperative launches, which the runtime makes resident as
 *    a whole even beside concurrent kernels, at about 12-16 us more per launch.
 * The process starts in COOPERATIVE if the environment sets DFL_AMD_COOP=1, ORDINARY
 * if it sets DFL_AMD_COOP=0, else AUTO.  Process-wide; returns 0 or an argument error. */
enum dfl_launch_mode { DFL_LAUNCH_AUTO = 0, DFL_LAUNCH_ORDINARY = 1, DFL_LAUNCH_COOPERATIVE = 2 };
int dfl_set_launch_mode(int mode);
int dfl_get_launch_mode(void);

/* For tests of the failure path only: the number of polls after which a
 * cross-workgroup wait gives up (0 restores the default of about 2-4 s).  A tiny
 * limit makes the persistent kernels' waits expire, so they report error 2 and exit
 * normally; with 1 the exchange waits give up at their first poll, whatever has
 * arrived.  No counterpart in the reference.  Process-wide; returns 0. */
int dfl_debug_set_spin_limit(unsigned limit);

/* ---------------------------------------------------------------------------
 * Flash-Sinkhorn forward.
 * Replaces FlashSinkhornAttn.forward (src/deepfold/model/kernels/flash_sinkhorn_attn.py:77-244)
 * and the Triton forward FlashSinkhornFunction.forward (sinkhorn_kernel.py:1921-2083):
 * K_iter log-domain UOT Sinkhorn iterations, then O_avg = T_norm V, x_c = T_norm x,
 * o = sigmoid(G) * O_avg permuted to (B, N, H*d).
 * q, k, v, g: (B,H,N,d) elements of `dtype` at q + b*stride_b + h*stride_h + n*stride_n + c.
 * g may be NULL (no gate: o = O_avg).  x_res (B,N,3), pos_weight (H,68), pos_bins (B,N,N)
 * int32, w_dist (H,), log_u_init/log_v_init (B,H,N) and mask (B,N) may be NULL.
 * Bins outside [0, 68) add no position bias.  NULL w_dist means no geometry term (the
 * kernels then carry no distance code; x_res is still the coordinate input of x_centroid).
 * Outputs o_flat (B,N,H*d), x_centroid (B,H,N,3), log_u, log_v (B,H,N); saved for the
 * backward: o_avg (B,H,N,d), log_z (B,H,N) = LSE_j(u_i + L_ij + v_j) and
 * col_lse (B,H,N) = LSE_i(L_ij + u_i) of the last column update.
 * storage selects where the kernels keep the cost:
 * DFL_STORAGE_REGISTER (3) computes each workgroup's block of logits once and keeps
 * it in registers for all iterations (each (b,h) split into a grid of plan blocks);
 * it serves the UOT forward with K_iter >= 1 while the blocks fit the register tiles
 * (at B*H = 16 up to N = 768; the balanced transport, K_iter = 0 and larger problems
 * are refused with an argument error);
 * RESIDENT keeps Q, K and the length-N vectors in LDS and recomputes the cost tile
 * on MFMA every sweep (fails with an argument error if they do not fit);
 * STREAM keeps only each workgroup's stripe in LDS and streams the rest through L2
 * (long sequences, e.g. N = 4096, d = 64);
 * DFL_STORAGE_AUTO (0) picks the resident layout with its logits held in registers
 * (each workgroup's stripe of plan rows and of plan columns, computed once) for the
 * UOT forward without hist where every stripe fits the register tiles (N <= 768 with
 * at most 3 tiles of 16 rows per stripe at N > 512, 4 below), else REGISTER where it
 * serves and the cost carries position bins or a geometry term, else RESIDENT where
 * it fits, else STREAM.  Results agree to rounding.
 * hist (K_iter,2,B,H,N) may be NULL; if given, the forward also writes v after the
 * column update and u after the row update of every iteration (natural log), which
 * dfl_sinkhorn_unrolled_bwd needs.
 */
enum dfl_storage { DFL_STORAGE_AUTO = 0, DFL_STORAGE_RESIDENT = 1, DFL_STORAGE_STREAM = 2, DFL_STORAGE_REGISTER = 3 };

typedef struct dfl_sinkhorn_fwd_params {
  int dtype;
  const void* q;
  const void* k;
  const void* v;
  const void* g;
  long long stride_b, stride_h, stride_n;
  const float* x_res;
  const float* pos_weight;
  const int* pos_bins;
  const float* eps;
  const float* w_dist;
  const float* log_mu;
  const float* log_nu;
  const float* log_u_init;
  const float* log_v_init;
  const float* mask;
  int B, H, N, d;
  int K_iter;
  float lam;
  float r_0;
  float* o_flat;
  float* x_centroid;
  float* log_u;
  float* log_v;
  float* o_avg;
  float* log_z;
  float* col_lse;
  int storage;
  float* hist;
} dfl_sinkhorn_fwd_params;

size_t dfl_sinkhorn_workspace_size(int B, int H, int N);
int dfl_sinkhorn_fwd(const dfl_sinkhorn_fwd_params* p, void* workspace, size_t workspace_bytes, void* stream);

/* Optional extension of the workspace for dfl_sinkhorn_bwd: a workspace of
 * dfl_sinkhorn_workspace_size(B, H, N) + dfl_sinkhorn_bias_workspace_size(B, H, N)
 * bytes lets a backward whose cost has position bins or a geometry term evaluate
 * that bias once per call (2 B H Np^2 floats, Np = N rounded up to 32) and read it
 * in every sweep instead of looking up bins and evaluating distances per element.
 * The results are the same; the forward ignores the extension.  No counterpart in
 * the reference, whose Triton backward recomputes the cost tile
 * (sinkhorn_kernel.py:1578-1760). */
size_t dfl_sinkhorn_bias_workspace_size(int B, int H, int N);

/* Allocation-free variant of dfl_sinkhorn_fwd.  It has no counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * params, outputs and kernels as dfl_sinkhorn_fwd, resident storage only (AUTO or
 * RESIDENT or REGISTER; a problem that needs stream storage is rejected).  Instead
 * of a workspace it uses a static device array of DFL_NOALLOC_SCRATCH_BYTES per GPU,
 * held until the process ends: it needs 256 + 8*B*H*(33*Np + 64) bytes (+ 2*B*Np*Np
 * with pos_bins), Np = N rounded up to 32, and rejects larger problems.  Every call on
 * one GPU shares that array, so calls that overlap in time on one GPU race.  It
 * calls no hipMalloc / hipFree and no allocating library routine.  Every call first
 * clears the array's header and exchange words with a fill kernel on `stream`, so a
 * HIP graph that captured the call can be replayed with new input values. */
#define DFL_NOALLOC_SCRATCH_BYTES (8u << 20)
int dfl_sinkhorn_fwd_noalloc(const dfl_sinkhorn_fwd_params* p, void* stream);

/* Error code (0 = none) recorded by the latest dfl_sinkhorn_fwd_noalloc call on the
 * current device, read from the static array's header; synchronises `stream`.  The
 * allocation-free forward reports an expired wait here, and also through
 * dfl_pending_error() once any other call has created the pinned host word. */
int dfl_noalloc_error(void* stream);

/* ---------------------------------------------------------------------------
 * Flash-Sinkhorn IFT backward.
 * Replaces FlashSinkhornAttn.backward (flash_sinkhorn_attn.py:246-667).  The linear
 * system (I - kappa^2 S_row^T S_col) z_v = g_v is solved either by the reference's
 * Gauss-Seidel fixed point (solver = DFL_IFT_FIXED_POINT, `iters` sweeps; the
 * reference uses iters = K_iter) or by conjugate gradient on its symmetric form
 * (solver = DFL_IFT_CG, `iters` CG steps).  mode = DFL_IFT_REFERENCE reproduces the
 * reference's signs; DFL_IFT_ANALYTIC gives the true implicit adjoint (the z_v*S_col
 * term of dC and d log_mu change sign).  Padded tokens (mask == 0) are excluded,
 * which equals evaluating each sample on its unpadded slice.
 * Inputs are the forward's inputs and saved outputs plus grad_o (B,N,H*d) fp32 and
 * grad_xc (B,H,N,3) fp32 (may be NULL).  Outputs (fully written): dq, dk, dv, dg
 * (B,H,N,d) in `dtype` (bf16 inputs get bf16 gradients, accumulated in fp32 and
 * rounded once), dlog_mu, dlog_nu (B,H,N) fp32; optional fp32 (NULL = not requested,
 * which also skips their per-element work): dx_res (B,N,3), dpos_weight (H,68), dw_dist (H,).
 * storage: as for the forward (the two calls choose independently).
 */
enum dfl_ift_solver { DFL_IFT_FIXED_POINT = 0, DFL_IFT_CG = 1 };
enum dfl_ift_mode { DFL_IFT_REFERENCE = 0, DFL_IFT_ANALYTIC = 1 };

typedef struct dfl_sinkhorn_bwd_params {
  int dtype;
  const void* q;
  const void* k;
  const void* v;
  const void* g;
  long long stride_b, stride_h, stride_n;
  const float* x_res;
  const float* pos_weight;
  const int* pos_bins;
  const float* eps;
  const float* w_dist;
  const float* mask;
  const float* log_u;
  const float* log_v;
  const float* log_z;
  const float* col_lse;
  const float* o_avg;
  const float* x_centroid;
  const float* grad_o;
  const float* grad_xc;
  int B, H, N, d;
  float lam;
  float r_0;
  int solver;
  int iters;
  int mode;
  float cg_rtol;
  void* dq; /* in `dtype` */
  void* dk;
  void* dv;
  void* dg;
  float* dlog_mu;
  float* dlog_nu;
  float* dx_res;
  float* dpos_weight;
  float* dw_dist;
  int storage;
} dfl_sinkhorn_bwd_params;

int dfl_sinkhorn_bwd(const dfl_sinkhorn_bwd_params* p, void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * Flash-Sinkhorn unrolled backward: the exact gradient through the K_iter executed
 * iterations, as the reference's GPU path computes it (FlashSinkhornFunction.backward,
 * sinkhorn_kernel.py:2085-2382; autograd through the dense iteration in its
 * tests/test_triton_fallback_consistency.py:312-430), instead of the implicit adjoint.
 * Inputs: the forward's inputs (q, k, v, g, strides, x_res, pos_weight, pos_bins, eps,
 * w_dist, log_mu, log_nu, log_v_init, mask, B, H, N, d, K_iter >= 1, lam, r_0) and
 * outputs (o_avg, x_centroid, log_u, log_z, and hist, which the forward must have
 * written), grad_o (B,N,H*d) fp32 and grad_xc (B,H,N,3) (may be NULL).  Outputs
 * (fully written): dq, dk, dv, dg (dg may be NULL without g) (B,H,N,d) in `dtype`;
 * fp32 dlog_mu, dlog_nu (B,H,N); optional fp32 (NULL = not requested): dlog_v_init
 * (B,H,N), dx_res (B,N,3), dpos_weight (H,68), dw_dist (H,).  Padded tokens are
 * excluded, as in dfl_sinkhorn_bwd.  Accumulation is fp32; with bf16 inputs the cost
 * recompute and the dq / dk products run on the bf16 MFMA (exact operands; the plan
 * weights as a bf16 hi + lo pair), the rest in fp32.  Workspace:
 * dfl_sinkhorn_unrolled_workspace_size(B, H, N, d) bytes; the forward's workspace
 * rules apply (a workspace that served the forward may serve this call if large enough).
 */
typedef struct dfl_sinkhorn_unrolled_bwd_params {
  int dtype;
  const void* q;
  const void* k;
  const void* v;
  const void* g;
  long long stride_b, stride_h, stride_n;
  const float* x_res;
  const float* pos_weight;
  const int* pos_bins;
  const float* eps;
  const float* w_dist;
  const float* log_mu;
  const float* log_nu;
  const float* log_v_init;
  const float* mask;
  int B, H, N, d;
  int K_iter;
  float lam;
  float r_0;
  const float* o_avg;
  const float* x_centroid;
  const float* log_u;
  const float* log_z;
  const float* hist;
  const float* grad_o;
  const float* grad_xc;
  void* dq; /* in `dtype` */
  void* dk;
  void* dv;
  void* dg;
  float* dlog_mu;
  float* dlog_nu;
  float* dlog_v_init;
  float* dx_res;
  float* dpos_weight;
  float* dw_dist;
} dfl_sinkhorn_unrolled_bwd_params;

size_t dfl_sinkhorn_unrolled_workspace_size(int B, int H, int N, int d);
int dfl_sinkhorn_unrolled_bwd(const dfl_sinkhorn_unrolled_bwd_params* p, void* workspace, size_t workspace_bytes,
                              void* stream);

/* ---------------------------------------------------------------------------
 * Softmax attention: O = softmax(scale * Q K^T + bias, key mask) V, rows of
 * masked queries zero, optional sigmoid gate O *= sigma(G).  One engine for
 *  - flash_diffusion_attn (flash_diffusion_attn.py:485-622): self attention with
 *    bias_mode = BINS (pos_weight[h, pos_bins]) or DENSE (pair bias (B,H,N,N));
 *  - flash_atom_attn (flash_atom_attn.py:262-354): window = 1, 32-query windows
 *    over keys [32w - 48, 32w + 80), optional bias_mode = WINDOW ((ceil(N/32),H,32,128));
 *  - token_to_atom_attn (cross_attn_kernel.py:555-696): cross attention Mq x Nk.
 * q, g: (B,H,Mq,d) and k, v: (B,H,Nk,d) elements of `dtype` with element strides
 * (unit inner stride); bias (dense / window) has the element type of q and is
 * contiguous.  q_mask (B,Mq), k_mask (B,Nk), pos_bins (B,Mq,Nk) int32 may be NULL.
 * Keys masked out contribute nothing; a query with no valid key gets a zero row.
 * Forward outputs: o (B,H,Mq,d) element type of q, contiguous; lse (B,H,Mq) fp32.
 * Backward inputs: grad_o (B,H,Mq,d) contiguous, plus the forward's o and lse;
 * outputs (element type of q, contiguous): dq, dk, dv; dg if g; dbias if a dense
 * or window bias is given (may be NULL; every entry is written, window entries
 * outside the sequence as zero).  The window bias is shared by the batch, so its
 * gradient is the sum over batch rows: with B > 1 each row's gradient goes to a
 * slab set of the workspace and the call sums them in row order (in fp32, rounded
 * once to the element type).  dpos_weight (H,68) fp32 for BINS (may be NULL).
 */
enum dfl_attn_bias { DFL_ATTN_BIAS_NONE = 0, DFL_ATTN_BIAS_BINS = 1, DFL_ATTN_BIAS_DENSE = 2, DFL_ATTN_BIAS_WINDOW = 3 };

typedef struct dfl_attn_params {
  int dtype;
  const void* q;
  const void* k;
  const void* v;
  const void* g;
  long long q_stride_b, q_stride_h, q_stride_n;
  long long k_stride_b, k_stride_h, k_stride_n;
  const float* q_mask;
  const float* k_mask;
  int bias_mode;
  const float* pos_weight;
  const int* pos_bins;
  const void* bias;
  int window;
  int B, H, Mq, Nk, d;
  float scale;
  void* o;
  float* lse;
  const void* grad_o;
  void* dq;
  void* dk;
  void* dv;
  void* dg;
  void* dbias;
  float* dpos_weight;
} dfl_attn_params;

/* Bytes of backward workspace (no zeroing needed); the forward uses none.  For
 * Mq == Nk and B > 1 it includes B * ceil(Mq/32) * H * 32 * 128 * 4 bytes for the
 * per-row window-bias gradients. */
size_t dfl_attn_workspace_size(int B, int H, int Mq, int Nk, int d);
int dfl_attn_fwd(const dfl_attn_params* p, void* stream);
int dfl_attn_bwd(const dfl_attn_params* p, void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * Atom-to-token attention (cross_attn_kernel.py:424-457, 496-552, 629-661):
 * token n attends to atoms [starts[n], starts[n] + counts[n]) (clipped to [0, M));
 * masked or empty tokens get zero rows.  q (B,H,N,d), k, v (B,H,M,d) contiguous,
 * element type `dtype`; starts, counts (B,N) int32; token_mask (B,N) or NULL.
 * Forward outputs o (B,H,N,d), lse (B,H,N) fp32.  Backward outputs dq (B,H,N,d),
 * dk, dv (B,H,M,d), element type `dtype`; the workspace holds fp32 accumulators.
 */
typedef struct dfl_a2t_params {
  int dtype;
  const void* q;
  const void* k;
  const void* v;
  const int* starts;
  const int* counts;
  const float* token_mask;
  int B, H, N, M, d;
  float scale;
  void* o;
  float* lse;
  const void* grad_o;
  void* dq;
  void* dk;
  void* dv;
} dfl_a2t_params;

size_t dfl_a2t_workspace_size(int B, int H, int M, int d);
int dfl_a2t_fwd(const dfl_a2t_params* p, void* stream);
int dfl_a2t_bwd(const dfl_a2t_params* p, void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * Dense, materialised-cost Sinkhorn (src/deepfold/model/sinkhorn.py).  fp32,
 * contiguous.  The caller allocates every output.
 *
 * dfl_dense_sinkhorn_fwd replaces sinkhorn_solve (sinkhorn.py:17-112): up to K
 * iterations u = kappa (log mu - LSE_j(-C/eps + v + cb)), v = kappa (log nu -
 * LSE_i(-C/eps + u + rb)) on C (B,H,N,N), masks as -1e9 biases, outputs log_u,
 * log_v (B,H,N) zero at padded positions.  threshold >= 0 enables the
 * reference's early stop (L-inf change < threshold, checked every check_every
 * iterations); each check synchronises `stream`, as the reference's .item() does.
 * history (4 (K+1) B H N floats) receives the potentials and LSEs of every
 * iteration for the backward; *iters_done (host memory) the iterations executed.
 * dfl_dense_sinkhorn_bwd is autograd through those iterations (the reference's
 * backward): outputs dC (B,H,N,N), dlog_mu, dlog_nu (B,H,N), and optionally the
 * initial potentials' gradients (NULL = not requested).
 */
typedef struct dfl_dense_sinkhorn_params {
  const float* C;
  const float* log_mu;
  const float* log_nu;
  const float* eps;
  const float* log_u_init;
  const float* log_v_init;
  const float* mask;
  int B, H, N;
  int K;
  float lam;
  float threshold;
  int check_every;
  float* log_u;
  float* log_v;
  float* history;
  int* iters_done;
} dfl_dense_sinkhorn_params;

typedef struct dfl_dense_sinkhorn_bwd_params {
  const float* C;
  const float* eps;
  const float* mask;
  const float* history;
  int B, H, N;
  int K_max;
  int K;
  float lam;
  const float* grad_log_u;
  const float* grad_log_v;
  float* dC;
  float* dlog_mu;
  float* dlog_nu;
  float* dlog_u_init;
  float* dlog_v_init;
} dfl_dense_sinkhorn_bwd_params;

size_t dfl_dense_sinkhorn_workspace_size(int B, int H, int N, int K);
int dfl_dense_sinkhorn_fwd(const dfl_dense_sinkhorn_params* p, void* workspace, size_t workspace_bytes, void* stream);
int dfl_dense_sinkhorn_bwd(const dfl_dense_sinkhorn_bwd_params* p, void* workspace, size_t workspace_bytes,
                           void* stream);

/* dfl_dense_transport_fwd replaces compute_transport_output (sinkhorn.py:115-198):
 * T_norm = exp(ls - max)/(sum + 1e-6) (rows of padded queries zero), O = T_norm V,
 * o = sigmoid(G) O permuted to (B,N,H*d) (G may be NULL: no gate), x_centroid =
 * T_norm x_res (x_res may be NULL).  d <= 64.  o_avg (B,H,N,d) is saved for the
 * backward.  dfl_dense_transport_bwd: gradients of those ops for grad_o, grad_T
 * (gradient of T_norm, may be NULL) and grad_xc (may be NULL): dV, dG (NULL if no
 * gate), dlog_u, dlog_v, dC and dx_res (NULL if no x_res). */
typedef struct dfl_dense_transport_params {
  const float* V;
  const float* G;
  const float* log_u;
  const float* log_v;
  const float* C;
  const float* eps;
  const float* x_res;
  const float* mask;
  int B, H, N, d;
  float* o;
  float* T_norm;
  float* x_centroid;
  float* o_avg;
  const float* grad_o;
  const float* grad_T;
  const float* grad_xc;
  float* dV;
  float* dG;
  float* dlog_u;
  float* dlog_v;
  float* dC;
  float* dx_res;
} dfl_dense_transport_params;

size_t dfl_dense_transport_workspace_size(int B, int H, int N, int d);
int dfl_dense_transport_fwd(const dfl_dense_transport_params* p, void* stream);
int dfl_dense_transport_bwd(const dfl_dense_transport_params* p, void* workspace, size_t workspace_bytes,
                            void* stream);

/* ---------------------------------------------------------------------------
 * Balanced Sinkhorn transport (the coordinate / feature centroid of TokenOTBlock).
 * Replaces BalancedSinkhornFn and BalancedSinkhornDualFn
 * (src/deepfold/model/kernels/flash_sinkhorn_transport.py:287-373, 403-516; CPU
 * form _sinkhorn_cpu :253-282).  Per (b,h), on the valid tokens of the sample:
 *   C_ij = (1 - w_h)(1 - q_i.k_j) + w_h d_ij / (r + d_ij),  w_h = sigmoid(alpha_h),
 *   r = max(|r_h|, 0.1), d_ij = max(|x_i - x_j|, 1e-8), L = -C / eps_h;
 *   K_iter iterations of  v = lm - LSE_i(L + u),  u = lm - LSE_j(L + v)  (column
 *   update first, u starts at 0, lm = -log n_valid);
 *   P = exp(u + L + v - lm) (rows sum to 1);  x_centroid = P x,  h_centroid = P V.
 * Inputs are fp32 (the reference casts to fp32 first).  q, k and v share the
 * element strides stride_b/h/n (unit inner stride); v has the head dim d and may be
 * NULL (coordinate centroid only, as balanced_sinkhorn_transport).  x_res (B,N,3)
 * contiguous is required; mask (B,N) may be NULL.  Padded tokens produce zero
 * outputs.  K_iter must be >= 1.
 * The forward writes x_centroid (B,H,N,3), h_centroid (B,H,N,d) (if v given),
 * log_u, log_v, log_z (B,H,N) and hist (K_iter,2,B,H,N): v after the column update
 * and u after the row update of every iteration, which the backward needs (the
 * reference saves the same history).
 * The backward (exact gradient of the K unrolled iterations) takes the forward's
 * inputs, its x_centroid / h_centroid / hist and grad_xc (B,H,N,3), grad_hc
 * (B,H,N,d) (either may be NULL), and writes dq, dk (B,H,N,d), dx_res (B,N,3),
 * dv (B,H,N,d) (may be NULL), dalpha_h and dr_h (H,).  eps receives no gradient,
 * as in the reference.  dfl_balanced_workspace_size(..., backward = 0) is the
 * forward's workspace (O(B*H*N) exchange words while a (b,h) fits in LDS);
 * backward = 1 gives the size that serves both directions (it adds O(B*H*N*d)
 * prepared operands).  The rules of dfl_sinkhorn_fwd's workspace apply.
 */
typedef struct dfl_balanced_fwd_params {
  int dtype; /* DFL_F32 */
  const void* q;
  const void* k;
  const void* v;
  long long stride_b, stride_h, stride_n;
  const float* x_res;
  const float* eps;
  const float* alpha_h;
  const float* r_h;
  const float* mask;
  int B, H, N, d;
  int K_iter;
  float* x_centroid;
  float* h_centroid;
  float* log_u;
  float* log_v;
  float* log_z;
  float* hist;
  int storage;
} dfl_balanced_fwd_params;

typedef struct dfl_balanced_bwd_params {
  int dtype; /* DFL_F32 */
  const void* q;
  const void* k;
  const void* v;
  long long stride_b, stride_h, stride_n;
  const float* x_res;
  const float* eps;
  const float* alpha_h;
  const float* r_h;
  const float* mask;
  int B, H, N, d;
  int K_iter;
  const float* x_centroid;
  const float* h_centroid;
  const float* hist;
  const float* grad_xc;
  const float* grad_hc;
  float* dq;
  float* dk;
  float* dv;
  float* dx_res;
  float* dalpha_h;
  float* dr_h;
} dfl_balanced_bwd_params;

size_t dfl_balanced_workspace_size(int B, int H, int N, int d, int backward);
int dfl_balanced_fwd(const dfl_balanced_fwd_params* p, void* workspace, size_t workspace_bytes, void* stream);
int dfl_balanced_bwd(const dfl_balanced_bwd_params* p, void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * Sink projections: the step before the balanced transport in TokenOTBlock.forward
 * (src/deepfold/model/trunk_block.py:165-175):
 *   h_s = LayerNorm(h) (biased variance, eps 1e-5);  u_p = h_s W_p^T for p = q, k, v;
 *   q_s, k_s = u / max(|u|, 1e-12) per head of C/H columns (F.normalize); v_s = u_v.
 * h is (M, C) rows of d_model in `dtype` (the weights share it; bf16 runs the
 * products on bf16 MFMA with fp32 accumulation, as autocast's bf16 Linear).  The
 * weights are nn.Linear (out, in) = (C, C) row-major; w_v may be NULL.  Outputs are
 * fp32 (M, C), i.e. (B, N, H, C/H): the (B, H, N, d) views the reference builds with
 * .view().permute() are these arrays with strides (N*C, C/H, C), which
 * dfl_balanced_fwd reads in place.  q_norm, k_norm (M, H) and ln_mean, ln_rstd (M)
 * are saved for the backward.  C must be a multiple of 64 with C/H in {16, 32, 64}
 * and at most 512 (fp32) or 1024 (bf16).
 * The backward takes the forward's inputs and saved values, the upstream gradients
 * dq_s, dk_s, dv_s (M, C) fp32 (any may be NULL: zero), and writes dh (M, C) fp32,
 * dln_weight, dln_bias (C) and dw_q, dw_k, dw_v (C, C) fp32 (dw_v NULL when w_v
 * is; any dw may be NULL).  Workspace: dfl_sink_proj_workspace_size(M, C) bytes,
 * no initialisation needed.
 */
typedef struct dfl_sink_proj_params {
  int dtype; /* DFL_F32 or DFL_BF16: h and the weights */
  const void* h;
  const float* ln_weight;
  const float* ln_bias;
  const void* w_q;
  const void* w_k;
  const void* w_v;
  int M, C, H;
  /* forward outputs; inputs of the backward */
  float* q_s;
  float* k_s;
  float* v_s;
  float* q_norm;
  float* k_norm;
  float* ln_mean;
  float* ln_rstd;
  /* backward */
  const float* dq_s;
  const float* dk_s;
  const float* dv_s;
  float* dh;
  float* dln_weight;
  float* dln_bias;
  float* dw_q;
  float* dw_k;
  float* dw_v;
} dfl_sink_proj_params;

size_t dfl_sink_proj_workspace_size(int M, int C);
int dfl_sink_proj_fwd(const dfl_sink_proj_params* p, void* stream);
int dfl_sink_proj_bwd(const dfl_sink_proj_params* p, void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * Gated coordinate update: the step after the balanced transport in
 * TokenOTBlock.forward (src/deepfold/model/trunk_block.py:189-204):
 *   gate = sigmoid(w_gate . LayerNorm(h) + b_gate)   (LayerNorm with its own weights)
 *   x_out = x_res + mask * gate * sum_h tanh(lambda_raw_h) / H * (x_centroid_h - x_res).
 * h is (B*N, C) in `dtype`; ln_weight, ln_bias, w_gate (C), b_gate (1), lambda_raw
 * (H), x_centroid (B,H,N,3), x_res (B,N,3) and mask (B,N) (may be NULL) are fp32.
 * The backward takes dx_out (B,N,3) and writes dx_res (B,N,3), dx_centroid
 * (B,H,N,3), dh (B*N, C) fp32, dln_weight, dln_bias, dw_gate (C), db_gate (1) and
 * dlambda_raw (H) (the parameter gradients may be NULL).  C must be a multiple of 64
 * and at most 1024; H at most 64.  Workspace: dfl_coord_update_workspace_size(C, H).
 */
typedef struct dfl_coord_update_params {
  int dtype; /* of h */
  const void* h;
  const float* ln_weight;
  const float* ln_bias;
  const float* w_gate;
  const float* b_gate;
  const float* lambda_raw;
  const float* x_centroid;
  const float* x_res;
  const float* mask;
  int B, N, C, H;
  float* x_out;
  /* backward */
  const float* dx_out;
  float* dx_res;
  float* dx_centroid;
  float* dh;
  float* dln_weight;
  float* dln_bias;
  float* dw_gate;
  float* db_gate;
  float* dlambda_raw;
} dfl_coord_update_params;

size_t dfl_coord_update_workspace_size(int C, int H);
int dfl_coord_update_fwd(const dfl_coord_update_params* p, void* stream);
int dfl_coord_update_bwd(const dfl_coord_update_params* p, void* workspace, size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* DFL_AMD_H */
