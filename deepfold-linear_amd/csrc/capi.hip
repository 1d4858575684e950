// C-ABI entry points (include/dfl_amd.h): argument checking, work split,
// workspace layout and launches.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <unordered_map>

#include "../../include/dfl_amd.h"
#include "attn_args.h"
#include "dense_args.h"
#include "sinkhorn_args.h"
#include "trunk_args.h"

namespace dfl {
size_t proj_fwd_lds_bytes(int C, bool bf16_in);
hipError_t launch_proj_fwd(const ProjArgs& a, bool bf16_in, hipStream_t s);
hipError_t launch_proj_bwd(const ProjArgs& a, bool bf16_in, hipStream_t s);
hipError_t launch_coord(const CoordArgs& a, bool bf16_in, bool bwd, hipStream_t s);
size_t sinkhorn_fwd_lds_bytes(int N, int DP, int elem, int G, bool stream);
hipError_t launch_sinkhorn_fwd(const SinkFwdArgs& a, bool bf16_in, int DP, size_t lds, hipStream_t stream,
                               bool coop);
hipError_t launch_sinkhorn_fwd_stream(const SinkFwdArgs& a, bool bf16_in, int DP, size_t lds, hipStream_t stream,
                                      bool coop);
hipError_t launch_sinkhorn_pad(const PadArgs& p, bool bf16_in, int DP, hipStream_t stream);
hipError_t launch_sinkhorn_fwd_reg(const SinkFwdArgs& a, bool bf16_in, int DP, size_t lds, hipStream_t stream,
                                   bool coop);
bool sinkhorn_fwd_reg_fits(int N, int G);
size_t sinkhorn_fwd_reg_lds_bytes(int N, int DP, int elem, int G);
hipError_t launch_sinkhorn_fwd_blk(const SinkFwdArgs& a, bool bf16_in, int DP, size_t lds, int L, hipStream_t stream,
                                   bool coop);
size_t sinkhorn_fwd_blk_lds_bytes(int N, int DP, int elem);
bool sinkhorn_fwd_blk_fits(int B, int H, int N, int L);
size_t sinkhorn_fwd_blk_xch_words(int B, int H, int N);
size_t sinkhorn_bwd_lds_bytes(int N, int DP, int elem, int G, int CH, bool stream);
hipError_t launch_sinkhorn_bwd(const SinkBwdArgs& a, bool bf16_in, int DP, size_t lds, hipStream_t stream,
                               bool coop);
hipError_t launch_sinkhorn_bwd_stream(const SinkBwdArgs& a, bool bf16_in, int DP, size_t lds, hipStream_t stream,
                                      bool coop);
hipError_t launch_sinkhorn_bwd_prep(const SinkBwdArgs& a, bool bf16_in, int DP, hipStream_t stream);
hipError_t launch_bias_mat(const SinkBwdArgs& a, float* mat, float* matT, hipStream_t stream);
hipError_t launch_sinkhorn_bwd_finalize(const SinkBwdArgs& a, float* dx, float* dpw, float* dw,
                                        hipStream_t stream);
hipError_t launch_attn_fwd(const AttnArgs& a, bool bf16_in, int DP, hipStream_t s);
hipError_t launch_attn_bwd(const AttnArgs& a, bool bf16_in, int DP, hipStream_t s);
hipError_t launch_a2t_fwd(const A2TArgs& a, bool bf16_in, hipStream_t s);
hipError_t launch_a2t_bwd(const A2TArgs& a, bool bf16_in, hipStream_t s);
hipError_t dense_sinkhorn_init(const DenseSinkArgs& a, hipStream_t s);
hipError_t dense_sinkhorn_iteration(const DenseSinkArgs& a, int k, hipStream_t s);
hipError_t dense_sinkhorn_finish(const DenseSinkArgs& a, int k, hipStream_t s);
hipError_t dense_sinkhorn_backward(const DenseSinkBwdArgs& a, hipStream_t s);
hipError_t dense_zero(float* p, size_t n, hipStream_t s);
hipError_t dense_transport_forward(const DenseTransportArgs& a, hipStream_t s);
hipError_t dense_transport_backward(const DenseTransportArgs& a, hipStream_t s);
hipError_t launch_bins8(const int* bins, int B, int N, uint8_t* b8, uint8_t* b8t, hipStream_t stream);
hipError_t launch_fill_u64(uint64_t* p, size_t n, hipStream_t stream);
size_t balanced_bwd_lds_bytes(int N, int DP);
int balanced_max_tiles(int DP);
hipError_t launch_balanced_prep(const BalPrepArgs& p, int DP, hipStream_t stream);
hipError_t launch_balanced_bwd(const BalBwdArgs& a, int DP, size_t lds, hipStream_t stream, bool coop);
hipError_t launch_balanced_finalize(const BalBwdArgs& a, float* dx, float* dalpha, float* dr, hipStream_t stream);
size_t unrolled_bwd_lds_bytes(int N, int DP, int elem, int ops);
int unrolled_operand_mode(int N, int DP, int elem, size_t limit);
int unrolled_max_tiles(int DP);
hipError_t launch_unrolled_prep(const UnrPrepArgs& p, bool bf16_in, int DP, hipStream_t stream);
hipError_t launch_unrolled_bwd(const UnrBwdArgs& a, bool bf16_in, int DP, size_t lds, hipStream_t stream, bool coop,
                               int ops);
hipError_t launch_unrolled_finalize(const UnrBwdArgs& a, float* dx, float* dpw, float* dw, hipStream_t stream);
}  // namespace dfl

// Scratch of dfl_sinkhorn_fwd_noalloc: exchange words, error word and bins copies.
// One copy per GPU, allocated with the code object and held until the process ends.
// Host code uses the device address from hipGetSymbolAddress, never this name.
static __device__ __align__(256) unsigned char scratch[DFL_NOALLOC_SCRATCH_BYTES];

namespace {

thread_local std::string g_err;

int fail(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
int fail(const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return -1;
}

int hip_fail(hipError_t e, const char* what) {
  g_err = std::string(what) + ": " + hipGetErrorString(e);
  return (int)e;
}

// Exchange tags carry a 20-bit call salt (common.h).  The counter behind it is
// 64-bit: its bits above the salt count the salt's wrap-arounds ("epochs").  A
// workspace first used in one epoch and used again in a later one could hold a
// word whose salt and phase match a current tag, so its exchange region and
// header are cleared (fill kernel, on the call's stream) at its first use in each
// new epoch.  A workspace never seen before is taken as zero-filled, as the ABI
// requires of a new workspace.
int cu_count();

// Launch mode of the persistent kernels, whose group members wait on each other and
// so must all be resident at once.  DFL_LAUNCH_AUTO launches a grid of at most one
// workgroup per CU (dfl::grid_blocks(n_groups, G) <= CU count, which group_size()
// arranges) as an ordinary launch: on an otherwise idle device every workgroup is
// resident at once.  If other kernels hold CUs when it starts, a member that cannot
// become resident leaves the others polling: their waits give up after about 2-4 s,
// the call's outputs are invalid, and the error (code 2) is raised by the next call
// (dfl_pending_error) or dfl_workspace_error.  DFL_LAUNCH_COOPERATIVE guarantees
// residency against concurrent kernels on other streams, at about 12-16 us more per
// launch on MI355X (measured: cfg2 layer 0.602 vs 0.572 ms); grids larger than the
// CU count are always cooperative (the runtime then checks that they fit).
// rocprofv3 ends with SIGSEGV in its exit-time teardown after any cooperative
// launch, even of a trivial kernel, so the committed profiles use ordinary launches.
// Process-wide launch mode (dfl_set_launch_mode); its start value comes from
// DFL_AMD_COOP ("1" cooperative, "0" ordinary), else DFL_LAUNCH_AUTO.
std::atomic<int> g_launch_mode{[] {
  const char* v = std::getenv("DFL_AMD_COOP");
  if (v && v[0] == '1' && v[1] == 0) return (int)DFL_LAUNCH_COOPERATIVE;
  if (v && v[0] == '0' && v[1] == 0) return (int)DFL_LAUNCH_ORDINARY;
  return (int)DFL_LAUNCH_AUTO;
}()};
bool coop_launch(int G, int n_groups) {
  const int mode = g_launch_mode.load(std::memory_order_relaxed);
  if (G <= 1 || mode == DFL_LAUNCH_ORDINARY) return false;
  if (mode == DFL_LAUNCH_COOPERATIVE) return true;
  return dfl::grid_blocks(n_groups, G) > cu_count();
}

// Polls a cross-workgroup wait makes before it gives up (dfl_debug_set_spin_limit).
std::atomic<uint32_t> g_spin_limit{dfl::SPIN_LIMIT};

// The persistent kernels tag their exchange words with a salt chosen on the host
// per call, so a graph that captured one call would replay that salt, and a replay
// would accept the words an earlier replay left in the workspace.  Such captures are
// refused; the allocation-free forward, which clears its scratch with a kernel on
// every call, is the entry point for graph capture.
int refuse_capture(void* stream, const char* what) {
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing((hipStream_t)stream, &st) != hipSuccess) {
    (void)hipGetLastError();
    return 0;  // not a capturing stream (a launch into an invalid capture fails on its own)
  }
  if (st != hipStreamCaptureStatusNone)
    return fail("%s cannot be captured into a HIP graph (its exchange tags are chosen on the host per call); "
                "dfl_sinkhorn_fwd_noalloc supports capture", what);
  return 0;
}

std::atomic<uint64_t> g_salt_counter{1};
std::mutex g_ws_mu;
struct WsState {
  uint64_t epoch;      // epoch of the last clear (or of the first use)
  size_t clean_bytes;  // bytes from the workspace start known free of older epochs' words
};
std::unordered_map<const void*, WsState> g_ws_state;

// Salt for a launch on `workspace` whose kernels read the first `xch_end` bytes
// (header + exchange words); clears what an earlier epoch may have left there.
// Returns 0 or a hipError_t of the clear launch.
// fixed: the record of a buffer the library owns (the allocation-free entry point's
// static array), used instead of a map entry so that nothing is allocated.
int acquire_salt(void* workspace, size_t xch_end, void* stream, uint32_t* salt_out, WsState* fixed = nullptr) {
  uint64_t c = g_salt_counter.fetch_add(1);
  if ((c & 0xfffffu) == 0) c = g_salt_counter.fetch_add(1);  // salt 0 is never used
  const uint64_t epoch = c >> 20;
  *salt_out = (uint32_t)(c & 0xfffffu);
  std::lock_guard<std::mutex> lock(g_ws_mu);
  WsState* st = fixed;
  if (!st) {
    auto it = g_ws_state.find(workspace);
    if (it == g_ws_state.end()) {
      g_ws_state.emplace(workspace, WsState{epoch, ~(size_t)0});
      return 0;
    }
    st = &it->second;
  }
  size_t from = 0;
  if (st->epoch != epoch) {
    *st = WsState{epoch, 0};
  } else if (st->clean_bytes >= xch_end) {
    return 0;
  } else {
    from = st->clean_bytes;
  }
  from &= ~(size_t)7;
  const size_t words = (xch_end - from + 7) / 8;
  hipError_t e = dfl::launch_fill_u64(reinterpret_cast<uint64_t*>(static_cast<unsigned char*>(workspace) + from),
                                      words, (hipStream_t)stream);
  if (e != hipSuccess) return (int)e;
  st->clean_bytes = from + words * 8;
  return 0;
}

// Pinned, device-mapped host word that a kernel writes when one of its waits
// expires (common.h: ErrRef); read and cleared by dfl_pending_error().  Allocated
// once per process; null if the allocation fails (errors then stay in the
// workspace word only).
uint32_t* g_mailbox_host = nullptr;
std::atomic<uint32_t*> g_mailbox_dev{nullptr};
std::once_flag g_mailbox_once;
uint32_t* mailbox() {
  std::call_once(g_mailbox_once, [] {
    void* h = nullptr;
    if (hipHostMalloc(&h, 256, hipHostMallocMapped | hipHostMallocPortable | hipHostMallocCoherent) != hipSuccess) {
      (void)hipGetLastError();
      return;
    }
    memset(h, 0, 256);
    void* d = nullptr;
    if (hipHostGetDevicePointer(&d, h, 0) != hipSuccess) {
      (void)hipGetLastError();
      d = h;  // unified addressing: the host address is valid on the device
    }
    g_mailbox_host = static_cast<uint32_t*>(h);
    g_mailbox_dev.store(static_cast<uint32_t*>(d));
  });
  return g_mailbox_dev.load();
}

// may_allocate = false (allocation-free entry point): the mailbox only if an
// earlier call already allocated it.
dfl::ErrRef err_ref(void* workspace, bool may_allocate = true) {
  dfl::ErrRef r;
  r.ws = static_cast<uint32_t*>(workspace);
  r.host = may_allocate ? mailbox() : g_mailbox_dev.load();
  r.spin_limit = g_spin_limit.load(std::memory_order_relaxed);
  return r;
}

constexpr size_t WS_HEADER = 256;  // error word + last salt, cache-line padded

struct WsHeader {
  uint32_t err;
  uint32_t pad[63];
};

int cu_count() {
  static int cached = -1;
  if (cached < 0) {
    int dev = 0;
    (void)hipGetDevice(&dev);
    int c = 0;
    if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c <= 0) c = 256;
    cached = c;
  }
  return cached;
}

size_t np32(int N) { return (size_t)((N + 31) / 32) * 32; }

// Exchange words: the register-storage forward's (its partial vectors, the largest
// use: dfl::sinkhorn_fwd_blk_xch_words), which also covers the resident / stream
// forward (u and v, 32 placement words per (b,h)) and the backward (four vectors).
size_t xch_words(int B, int H, int N) { return dfl::sinkhorn_fwd_blk_xch_words(B, H, N); }

int head_dim_pad(int d) { return d <= 32 ? 32 : (d <= 64 ? 64 : -1); }

// Workgroups per (b,h): as many as fit one per CU in the XCD-aligned grid
// (dfl::grid_blocks), at most one per 16-row tile.
int group_size(int B, int H, int N) {
  const int bh = B * H;
  int G = cu_count() / (8 * ((bh + 7) / 8));
  if (G < 1) G = 1;
  const int tiles = (N + 15) / 16;
  if (G > tiles) G = tiles;
  return G;
}

// Backward partials: dx (B,H,N,3), dpw (B*H*G,68), dw (B*H*G), rounded to 256 bytes.
size_t partials_bytes(int B, int H, int N, int G) {
  const size_t b = (size_t)B * H * N * 3 * 4 + (size_t)B * H * G * 69 * 4;
  return (b + 255) / 256 * 256;
}

// Prepared backward operands, sized for the widest case (d <= 64, fp32):
// go_hi, go_lo, go_t of B*H*Np*64 elements each, then D (B*H*Np floats).
size_t prep_operand_bytes(int B, int H, int N) { return (size_t)B * H * np32(N) * 64 * 4; }

// Stream-mode region (after the backward's prepared operands), sized for the
// widest case: padded Q, K and transposed V (prep_operand_bytes each), padded
// coordinates (B*Np*3 floats), then the backward's per-workgroup vectors.
constexpr int STREAM_VECS = 19;  // dfl::BWD_STREAM_VECS
constexpr size_t LDS_LIMIT = 160 * 1024;
// static LDS of the register-storage forward (its plan tables), beside the dynamic part
constexpr size_t BLK_STATIC_LDS = 9 * 1024;
size_t stream_region_bytes(int B, int H, int N, int G) {
  const size_t np = np32(N);
  size_t b = 3 * prep_operand_bytes(B, H, N);
  b += ((size_t)B * np * 3 * 4 + 255) / 256 * 256;
  b += (size_t)B * H * G * STREAM_VECS * np * 4;
  return (b + 255) / 256 * 256;
}
size_t stream_region_offset(int B, int H, int N, int G) {
  size_t off = WS_HEADER + xch_words(B, H, N) * 8 + partials_bytes(B, H, N, G);
  off += 3 * prep_operand_bytes(B, H, N) + (size_t)B * H * np32(N) * 4;
  return (off + 255) / 256 * 256;
}

// Padded uint8 bins (row-major and transposed, [B][Np][Np] each) at the end of a workspace.
size_t bins8_bytes(int B, int N) { return (2 * (size_t)B * np32(N) * np32(N) + 255) / 256 * 256; }
size_t sinkhorn_bins8_offset(int B, int H, int N) {
  const int G = group_size(B, H, N);
  return stream_region_offset(B, H, N, G) + stream_region_bytes(B, H, N, G);
}
// Converts the caller's int32 bins into the workspace copies; sets b8 / b8t (null without bins).
int prepare_bins8(const int* bins, int B, int N, void* ws, size_t off, const uint8_t** b8, const uint8_t** b8t,
                  void* stream) {
  *b8 = *b8t = nullptr;
  if (!bins) return 0;
  uint8_t* p = static_cast<unsigned char*>(ws) + off;
  const size_t per = (size_t)B * np32(N) * np32(N);
  hipError_t e = dfl::launch_bins8(bins, B, N, p, p + per, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "bins conversion launch");
  *b8 = p;
  *b8t = p + per;
  return 0;
}

struct StreamPtrs {
  void* qp;
  void* kp;
  void* vt;
  float* xs_p;
  float* vec;
};
StreamPtrs stream_ptrs(void* ws, int B, int H, int N, int G) {
  unsigned char* base = static_cast<unsigned char*>(ws) + stream_region_offset(B, H, N, G);
  const size_t opb = prep_operand_bytes(B, H, N);
  StreamPtrs p;
  p.qp = base;
  p.kp = base + opb;
  p.vt = base + 2 * opb;
  p.xs_p = reinterpret_cast<float*>(base + 3 * opb);
  p.vec = reinterpret_cast<float*>(base + 3 * opb + ((size_t)B * np32(N) * 3 * 4 + 255) / 256 * 256);
  return p;
}

// Query-range splits of the attention dK/dV pass: when keys are few (token-to-atom:
// 341 keys, 8192 queries), as many splits as keep the grid within one workgroup per
// CU, preferring a count that makes B*H*splits a multiple of 8, so that the key
// blocks of one (b,h, split) share an XCD and read its queries into one L2.
int attn_qsplit(int B, int H, int Mq, int Nk) {
  const int kv_blocks = ((Nk + 63) / 64) * B * H;
  if (kv_blocks >= cu_count()) return 1;
  const int max_s = (Mq + 63) / 64;
  int s = cu_count() / kv_blocks;
  if (s > max_s) s = max_s;
  if (s < 1) s = 1;
  for (int t = s; t >= (s + 1) / 2 && t > 1; --t)
    if ((B * H * t) % 8 == 0) return t;
  return s;
}

// Attention backward workspace: do_w, D, dK/dV partials, d pos_weight partials and,
// for square shapes with B > 1 (a window bias is possible), per-batch-row window-bias
// gradient slabs sized for 4-byte elements.
struct AttnWs {
  size_t do_w, dcoef, kv_part, dpw_part, dbias_rows, total;
};
AttnWs attn_ws_layout(int B, int H, int Mq, int Nk) {
  auto r256 = [](size_t x) { return (x + 255) / 256 * 256; };
  AttnWs w;
  const size_t rows = (size_t)B * H * Mq;
  const int qs = attn_qsplit(B, H, Mq, Nk);
  w.do_w = 0;
  w.dcoef = w.do_w + r256(rows * 64 * 4);
  w.kv_part = w.dcoef + r256(rows * 4);
  w.dpw_part = w.kv_part + (qs > 1 ? r256((size_t)qs * B * H * Nk * 2 * 64 * 4) : 0);
  w.dbias_rows = w.dpw_part + r256((size_t)B * H * ((Mq + 31) / 32) * 68 * 4);  // per 32- or 64-query block
  const size_t slab = (size_t)((Mq + 31) / 32) * H * 32 * 128;
  w.total = w.dbias_rows + (B > 1 && Mq == Nk ? r256((size_t)B * slab * 4) : 0);
  return w;
}

int check_attn(const dfl_attn_params* p, bool bwd) {
  if (!p) return fail("params is NULL");
  if (p->dtype != DFL_BF16 && p->dtype != DFL_F32) return fail("dtype must be DFL_BF16 or DFL_F32");
  if (p->B <= 0 || p->H <= 0 || p->Mq <= 0 || p->Nk <= 0 || p->d <= 0) return fail("B, H, Mq, Nk, d must be positive");
  if (head_dim_pad(p->d) < 0) return fail("head dim d=%d > 64 is not supported", p->d);
  if (!p->q || !p->k || !p->v || !p->o || !p->lse) return fail("q, k, v, o and lse are required");
  if (p->q_stride_n < p->d || p->k_stride_n < p->d) return fail("row strides must be >= d (unit inner stride)");
  if (p->bias_mode < DFL_ATTN_BIAS_NONE || p->bias_mode > DFL_ATTN_BIAS_WINDOW) return fail("unknown bias_mode");
  if (p->bias_mode == DFL_ATTN_BIAS_BINS && (!p->pos_weight || !p->pos_bins)) return fail("BINS needs pos_weight and pos_bins");
  if ((p->bias_mode == DFL_ATTN_BIAS_DENSE || p->bias_mode == DFL_ATTN_BIAS_WINDOW) && !p->bias) return fail("bias is NULL");
  if (p->window && p->Mq != p->Nk) return fail("windowed attention needs Mq == Nk");
  if (p->bias_mode == DFL_ATTN_BIAS_WINDOW && !p->window) return fail("a window bias needs window = 1");
  if (bwd && (!p->grad_o || !p->dq || !p->dk || !p->dv)) return fail("grad_o, dq, dk and dv are required");
  return 0;
}

dfl::AttnArgs attn_args(const dfl_attn_params* p) {
  dfl::AttnArgs a;
  memset(&a, 0, sizeof(a));
  a.q = p->q; a.k = p->k; a.v = p->v; a.g = p->g;
  a.qsb = p->q_stride_b; a.qsh = p->q_stride_h; a.qsn = p->q_stride_n;
  a.ksb = p->k_stride_b; a.ksh = p->k_stride_h; a.ksn = p->k_stride_n;
  a.qmask = p->q_mask; a.kmask = p->k_mask;
  a.bias_mode = p->bias_mode; a.pos_w = p->pos_weight; a.bins = p->pos_bins; a.bias = p->bias;
  a.window = p->window ? 1 : 0;
  a.B = p->B; a.H = p->H; a.Mq = p->Mq; a.Nk = p->Nk; a.d = p->d;
  a.scale = p->scale;
  a.o = p->o; a.lse = p->lse;
  a.dout = p->grad_o; a.dq = p->dq; a.dk = p->dk; a.dv = p->dv; a.dg = p->dg;
  a.dbias = p->dbias; a.dpos_w = p->dpos_weight;
  a.qsplit = 1;
  return a;
}

int check_a2t(const dfl_a2t_params* p, bool bwd) {
  if (!p) return fail("params is NULL");
  if (p->dtype != DFL_BF16 && p->dtype != DFL_F32) return fail("dtype must be DFL_BF16 or DFL_F32");
  if (p->B <= 0 || p->H <= 0 || p->N <= 0 || p->M <= 0 || p->d <= 0) return fail("B, H, N, M, d must be positive");
  if (p->d > 64) return fail("head dim d=%d > 64 is not supported", p->d);
  if (!p->q || !p->k || !p->v || !p->starts || !p->counts || !p->o || !p->lse) return fail("required input is NULL");
  if (bwd && (!p->grad_o || !p->dq || !p->dk || !p->dv)) return fail("grad_o, dq, dk and dv are required");
  return 0;
}

dfl::A2TArgs a2t_args(const dfl_a2t_params* p) {
  dfl::A2TArgs a;
  memset(&a, 0, sizeof(a));
  a.q = p->q; a.k = p->k; a.v = p->v; a.starts = p->starts; a.counts = p->counts; a.tmask = p->token_mask;
  a.B = p->B; a.H = p->H; a.N = p->N; a.M = p->M; a.d = p->d; a.scale = p->scale;
  a.o = p->o; a.lse = p->lse; a.dout = p->grad_o; a.dq = p->dq; a.dk = p->dk; a.dv = p->dv;
  return a;
}

// Argument checks of dfl_sinkhorn_fwd_params (all but the workspace) and the kernel
// argument block; 0 or a negative argument error.
int fwd_args(const dfl_sinkhorn_fwd_params* p, dfl::SinkFwdArgs& a) {
  if (!p) return fail("params is NULL");
  if (p->dtype != DFL_BF16 && p->dtype != DFL_F32) return fail("dtype must be DFL_BF16 or DFL_F32");
  if (p->B <= 0 || p->H <= 0 || p->N <= 0 || p->d <= 0) return fail("B, H, N, d must be positive");
  if (head_dim_pad(p->d) < 0) return fail("head dim d=%d > 64 is not supported", p->d);
  if (p->K_iter < 0 || p->K_iter > 2000) return fail("K_iter=%d outside [0, 2000]", p->K_iter);
  if (!p->q || !p->k || !p->v || !p->eps || !p->log_mu || !p->log_nu) return fail("required input is NULL");
  if (!p->o_flat || !p->x_centroid || !p->log_u || !p->log_v || !p->o_avg || !p->log_z || !p->col_lse)
    return fail("output pointer is NULL");
  if (p->stride_n < p->d) return fail("stride_n must be >= d (unit inner stride)");
  if (p->pos_bins && !p->pos_weight) return fail("pos_bins given without pos_weight");
  if (p->storage < DFL_STORAGE_AUTO || p->storage > DFL_STORAGE_REGISTER) return fail("unknown storage %d", p->storage);
  memset(&a, 0, sizeof(a));
  a.q = p->q; a.k = p->k; a.v = p->v; a.g = p->g;
  a.sb = p->stride_b; a.sh = p->stride_h; a.sn = p->stride_n;
  a.x = p->x_res; a.pos_w = p->pos_weight; a.bins = p->pos_bins;
  a.eps = p->eps; a.w_dist = p->w_dist; a.log_mu = p->log_mu; a.log_nu = p->log_nu;
  a.u_init = p->log_u_init; a.v_init = p->log_v_init; a.mask = p->mask;
  a.B = p->B; a.H = p->H; a.N = p->N; a.d = p->d;
  a.K_iter = p->K_iter; a.lam = p->lam; a.r0 = p->r_0;
  a.o_flat = p->o_flat; a.x_centroid = p->x_centroid; a.log_u = p->log_u; a.log_v = p->log_v;
  a.o_avg = p->o_avg; a.log_z = p->log_z; a.col_lse = p->col_lse;
  a.hist = p->hist;
  return 0;
}

// The allocation-free forward's per-device scratch (static array `scratch` at file
// scope below): its device address on each GPU, resolved once per device, and that
// buffer's salt-epoch record.
constexpr size_t NOALLOC_SCRATCH_BYTES = DFL_NOALLOC_SCRATCH_BYTES;
constexpr int MAX_DEVICES = 64;
struct ScratchSlot {
  unsigned char* ptr;
  WsState state;
};
std::mutex g_scratch_mu;
ScratchSlot g_scratch[MAX_DEVICES];

// Where a forward keeps its scratch: a caller's workspace (dfl_sinkhorn_fwd,
// dfl_balanced_fwd) or the library's static per-device array
// (dfl_sinkhorn_fwd_noalloc).  Layout: header, exchange words from WS_HEADER, the
// uint8 bins copies at bins_off; stream storage also uses the workspace's stream region.
struct FwdScratch {
  unsigned char* base;
  size_t bins_off;
  bool allow_stream;   // false: the buffer has no stream region
  WsState* fixed;      // salt-epoch record of a library-owned buffer (else the map)
  bool may_allocate;   // the host mailbox may be allocated by this call
  bool clear_always;   // clear header and exchange words with a fill kernel on every call
};

// Storage-mode choice, workspace pointers and launches of the persistent forward
// (shared by the UOT, the balanced and the allocation-free entry points).  a holds
// inputs and outputs.
int run_fwd(dfl::SinkFwdArgs& a, bool bf16, int DP, int storage, const FwdScratch& w, void* stream) {
  const int G = group_size(a.B, a.H, a.N);
  const int elem = bf16 ? 2 : 4;
  const int L = cu_count() / 8;
  const size_t lds_res = dfl::sinkhorn_fwd_lds_bytes(a.N, DP, elem, G, false);
  const size_t lds_blk = dfl::sinkhorn_fwd_blk_lds_bytes(a.N, DP, elem);
  // register storage: the UOT forward (not the balanced one) with at least one iteration,
  // whose member grids fit the register tiles and whose output pass fits resident LDS
  const bool blk_ok = !a.balanced && a.K_iter >= 1 && lds_blk + BLK_STATIC_LDS <= LDS_LIMIT &&
                      dfl::sinkhorn_fwd_blk_fits(a.B, a.H, a.N, L);
  if (storage == DFL_STORAGE_REGISTER && !blk_ok)
    return fail("register storage does not fit B=%d, H=%d, N=%d, d=%d%s (needs %zu bytes of LDS, limit %zu)", a.B, a.H,
                a.N, a.d, a.balanced ? " (balanced transport)" : (a.K_iter < 1 ? " with K_iter = 0" : ""), lds_blk,
                LDS_LIMIT);
  // AUTO takes register storage where it is the faster forward: with position bins or a
  // geometry term, whose per-element cost it computes once instead of every sweep
  const bool has_bias = (a.bins && a.pos_w) || (a.x && a.w_dist);
  const size_t lds_reg = dfl::sinkhorn_fwd_reg_lds_bytes(a.N, DP, elem, G);
  const bool reg_ok = !a.balanced && !a.hist && a.K_iter >= 1 && dfl::sinkhorn_fwd_reg_fits(a.N, G) &&
                      lds_reg <= LDS_LIMIT;
  const bool blk_mode =
      blk_ok && (storage == DFL_STORAGE_REGISTER || (storage == DFL_STORAGE_AUTO && has_bias && !reg_ok));
  const bool stream_mode =
      !blk_mode && (storage == DFL_STORAGE_STREAM || (storage == DFL_STORAGE_AUTO && lds_res > LDS_LIMIT));
  // resident layout with the logits in registers: the UOT forward without history whose
  // stripes and slots fit the register tiles
  const bool reg_mode = !blk_mode && !stream_mode && storage == DFL_STORAGE_AUTO && reg_ok;
  const size_t lds = blk_mode ? lds_blk
                              : (stream_mode ? dfl::sinkhorn_fwd_lds_bytes(a.N, DP, elem, G, true)
                                             : (reg_mode ? lds_reg : lds_res));
  if (stream_mode && !w.allow_stream)
    return fail("N=%d, d=%d needs stream storage (resident needs %zu bytes of LDS, limit %zu), which the "
                "allocation-free forward does not provide", a.N, a.d, lds_res, LDS_LIMIT);
  if (lds > LDS_LIMIT)
    return fail("N=%d, d=%d, %s storage needs %zu bytes of LDS per workgroup (limit %zu)", a.N, a.d,
                stream_mode ? "stream" : "resident", lds, LDS_LIMIT);
  unsigned char* ws = w.base;
  void* workspace = ws;
  a.err = err_ref(ws, w.may_allocate);
  a.xch = reinterpret_cast<uint64_t*>(ws + WS_HEADER);
  a.G = G;
  // the exchange words this launch uses: the register-storage layout, or u and v of
  // every (b,h) then 32 placement words per (b,h)
  const size_t xch_end = WS_HEADER + (blk_mode ? dfl::sinkhorn_fwd_blk_xch_words(a.B, a.H, a.N)
                                               : (size_t)a.B * a.H * (2 * np32(a.N) + 32)) * 8;
  if (w.clear_always) {
    // every call starts from zeroed words, so a replay of a captured call (same salt)
    // never meets an earlier replay's words
    hipError_t e = dfl::launch_fill_u64(reinterpret_cast<uint64_t*>(ws), xch_end / 8, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "scratch clear launch");
    uint64_t c = g_salt_counter.fetch_add(1);
    if ((c & 0xfffffu) == 0) c = g_salt_counter.fetch_add(1);
    a.salt = (uint32_t)(c & 0xfffffu);
  } else {
    if (int rc = refuse_capture(stream, "dfl_sinkhorn_fwd")) return rc;
    if (int rc = acquire_salt(ws, xch_end, stream, &a.salt, w.fixed))
      return hip_fail((hipError_t)rc, "workspace clear launch");
  }
  if (a.bins)
    if (int rc = prepare_bins8(a.bins, a.B, a.N, workspace, w.bins_off, &a.bins8, &a.bins8t, stream)) return rc;
  hipError_t e;
  if (blk_mode) {
    e = dfl::launch_sinkhorn_fwd_blk(a, bf16, DP, lds, L, (hipStream_t)stream, coop_launch(L, 8));
  } else if (stream_mode) {
    const bool coop = coop_launch(G, a.B * a.H);
    const StreamPtrs sp = stream_ptrs(workspace, a.B, a.H, a.N, G);
    dfl::PadArgs pa;
    memset(&pa, 0, sizeof(pa));
    pa.q = a.q; pa.k = a.k; pa.v = a.v;
    pa.sb = a.sb; pa.sh = a.sh; pa.sn = a.sn;
    pa.x = a.x; pa.mask = a.mask;
    pa.B = a.B; pa.H = a.H; pa.N = a.N; pa.d = a.d;
    pa.qp = sp.qp; pa.kp = sp.kp; pa.vt = a.v ? sp.vt : nullptr; pa.xs_p = sp.xs_p;
    e = dfl::launch_sinkhorn_pad(pa, bf16, DP, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "sinkhorn pad launch");
    a.qp = sp.qp; a.kp = sp.kp; a.vt = sp.vt; a.xs_p = sp.xs_p;
    e = dfl::launch_sinkhorn_fwd_stream(a, bf16, DP, lds, (hipStream_t)stream, coop);
  } else if (reg_mode) {
    e = dfl::launch_sinkhorn_fwd_reg(a, bf16, DP, lds, (hipStream_t)stream, coop_launch(G, a.B * a.H));
  } else {
    e = dfl::launch_sinkhorn_fwd(a, bf16, DP, lds, (hipStream_t)stream, coop_launch(G, a.B * a.H));
  }
  if (e != hipSuccess) return hip_fail(e, "sinkhorn forward launch");
  return 0;
}

// Balanced transport workspace: the forward's (header, exchange words, stream
// region), or the backward's prepared operands and partials if larger.
struct BalWs {
  size_t qp, kp, qt, kt, vp, gp, gt, dcoef, gxs, xs, dx_part, ar_part, total;
};
BalWs bal_ws_layout(int B, int H, int N, int d) {
  auto r256 = [](size_t x) { return (x + 255) / 256 * 256; };
  const size_t np = np32(N);
  const int DP = head_dim_pad(d) < 0 ? 64 : head_dim_pad(d);
  const int G = group_size(B, H, N);
  const size_t op = r256((size_t)B * H * np * DP * 4);
  BalWs w;
  w.qp = r256(WS_HEADER + xch_words(B, H, N) * 8);
  w.kp = w.qp + op;
  w.qt = w.kp + op;
  w.kt = w.qt + op;
  w.vp = w.kt + op;
  w.gp = w.vp + op;
  w.gt = w.gp + op;
  w.dcoef = w.gt + op;
  w.gxs = w.dcoef + r256((size_t)B * H * np * 4);
  w.xs = w.gxs + r256((size_t)B * H * 3 * np * 4);
  w.dx_part = w.xs + r256((size_t)B * 3 * np * 4);
  w.ar_part = w.dx_part + r256((size_t)B * H * N * 3 * 4);
  w.total = w.ar_part + r256((size_t)B * H * G * 2 * 4);
  return w;
}

// Forward workspace: the header and exchange words when (b,h) stays resident in
// LDS, else the whole stream-mode layout of the UOT forward.
size_t bal_fwd_need(int B, int H, int N, int d, int storage) {
  const int DP = head_dim_pad(d) < 0 ? 64 : head_dim_pad(d);
  const size_t lds_res = dfl::sinkhorn_fwd_lds_bytes(N, DP, 4, group_size(B, H, N), false);
  const bool stream_mode = storage == DFL_STORAGE_STREAM || (storage == DFL_STORAGE_AUTO && lds_res > LDS_LIMIT);
  if (stream_mode) return dfl_sinkhorn_workspace_size(B, H, N);
  return WS_HEADER + xch_words(B, H, N) * 8;
}

// Unrolled UOT backward workspace: header, exchange words, fp32 operand copies
// (Q, K, V, gO rows; Q, K, gO transposed), vectors and partials.
struct UnrWs {
  size_t qp, kp, qt, kt, vp, gp, gt, dcoef, gxs, xs, dx_part, dpw_part, dw_part, total;
};
UnrWs unr_ws_layout(int B, int H, int N, int d) {
  auto r256 = [](size_t x) { return (x + 255) / 256 * 256; };
  const size_t np = np32(N);
  const int DP = head_dim_pad(d) < 0 ? 64 : head_dim_pad(d);
  const int G = group_size(B, H, N);
  const size_t op = r256((size_t)B * H * np * DP * 4);
  UnrWs w;
  w.qp = r256(WS_HEADER + xch_words(B, H, N) * 8);
  w.kp = w.qp + op;
  w.qt = w.kp + op;
  w.kt = w.qt + op;
  w.vp = w.kt + op;
  w.gp = w.vp + op;
  w.gt = w.gp + op;
  w.dcoef = w.gt + op;
  w.gxs = w.dcoef + r256((size_t)B * H * np * 4);
  w.xs = w.gxs + r256((size_t)B * H * 3 * np * 4);
  w.dx_part = w.xs + r256((size_t)B * 3 * np * 4);
  w.dpw_part = w.dx_part + r256((size_t)B * H * N * 3 * 4);
  w.dw_part = w.dpw_part + r256((size_t)B * H * G * 68 * 4);
  w.total = w.dw_part + r256((size_t)B * H * G * 4) + bins8_bytes(B, N);  // bins copies last
  return w;
}

int check_balanced(int dtype, const void* q, const void* k, const float* x, const float* eps, const float* alpha,
                   const float* r, int B, int H, int N, int d, int K_iter, long long sn) {
  if (dtype != DFL_F32) return fail("balanced transport computes in fp32: dtype must be DFL_F32");
  if (B <= 0 || H <= 0 || N <= 0 || d <= 0) return fail("B, H, N, d must be positive");
  if (head_dim_pad(d) < 0) return fail("head dim d=%d > 64 is not supported", d);
  if (K_iter < 1 || K_iter > 1000) return fail("K_iter=%d outside [1, 1000]", K_iter);
  if (!q || !k || !x || !eps || !alpha || !r) return fail("required input is NULL");
  if (sn < d) return fail("stride_n must be >= d (unit inner stride)");
  return 0;
}

}  // namespace

extern "C" {

const char* dfl_last_error(void) { return g_err.c_str(); }

const char* dfl_version(void) { return "deepfold_amd 0.1.0 (gfx950)"; }

size_t dfl_sinkhorn_workspace_size(int B, int H, int N) {
  if (B <= 0 || H <= 0 || N <= 0) return 0;
  const int G = group_size(B, H, N);
  return stream_region_offset(B, H, N, G) + stream_region_bytes(B, H, N, G) + bins8_bytes(B, N);
}

// The backward's precomputed bias: [B*H][Np][Np] floats and the transposed copy, after
// the regular workspace (rounded up to 256 bytes).
static size_t bias_mat_offset(int B, int H, int N) { return (dfl_sinkhorn_workspace_size(B, H, N) + 255) / 256 * 256; }
size_t dfl_sinkhorn_bias_workspace_size(int B, int H, int N) {
  if (B <= 0 || H <= 0 || N <= 0) return 0;
  const size_t np = np32(N);
  return 2 * (size_t)B * H * np * np * 4 + (bias_mat_offset(B, H, N) - dfl_sinkhorn_workspace_size(B, H, N));
}

int dfl_pending_error(void) {
  if (!g_mailbox_host) return 0;
  const uint32_t w = __atomic_exchange_n(g_mailbox_host, 0u, __ATOMIC_ACQ_REL);
  if (w == 0) return 0;
  const int code = (int)(w & 0xfffu);
  g_err = "a kernel launched earlier reported error code " + std::to_string(code) +
          " (a cross-workgroup wait expired; its outputs are invalid)";
  return code;
}

int dfl_set_launch_mode(int mode) {
  if (mode != DFL_LAUNCH_AUTO && mode != DFL_LAUNCH_ORDINARY && mode != DFL_LAUNCH_COOPERATIVE)
    return fail("unknown launch mode %d", mode);
  g_launch_mode.store(mode);
  return 0;
}

int dfl_get_launch_mode(void) { return g_launch_mode.load(); }

int dfl_debug_set_spin_limit(unsigned limit) {
  g_spin_limit.store(limit == 0 ? dfl::SPIN_LIMIT : (uint32_t)limit);
  return 0;
}

int dfl_workspace_error(const void* workspace, void* stream) {
  if (!workspace) return fail("workspace is NULL");
  uint32_t words[2] = {0, 0};
  hipError_t e = hipMemcpyAsync(words, workspace, 8, hipMemcpyDeviceToHost, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "dfl_workspace_error copy");
  e = hipStreamSynchronize((hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "dfl_workspace_error sync");
  // word 0: (salt << 12) | code of the call that raised it; word 1: salt of the
  // latest call that ran on this workspace (written by its first workgroup).
  if ((words[0] >> 12) == words[1]) return (int)(words[0] & 0xfffu);
  return 0;
}

int dfl_sinkhorn_fwd(const dfl_sinkhorn_fwd_params* p, void* workspace, size_t workspace_bytes, void* stream) {
  dfl::SinkFwdArgs a;
  if (int rc = fwd_args(p, a)) return rc;
  const size_t need = dfl_sinkhorn_workspace_size(p->B, p->H, p->N);
  if (!workspace || workspace_bytes < need) return fail("workspace too small: need %zu bytes", need);
  const FwdScratch w{static_cast<unsigned char*>(workspace), sinkhorn_bins8_offset(p->B, p->H, p->N), true, nullptr,
                     true, false};
  return run_fwd(a, p->dtype == DFL_BF16, head_dim_pad(p->d), p->storage, w, stream);
}

int dfl_sinkhorn_fwd_noalloc(const dfl_sinkhorn_fwd_params* p, void* stream) {
  dfl::SinkFwdArgs a;
  if (int rc = fwd_args(p, a)) return rc;
  if (p->storage == DFL_STORAGE_STREAM)
    return fail("the allocation-free forward runs resident storage only (storage=DFL_STORAGE_STREAM given)");
  // layout in the static array: header, exchange words (as many as the register-storage
  // forward uses, the most of any storage), then the uint8 bins copies
  const size_t xch_end = WS_HEADER + dfl::sinkhorn_fwd_blk_xch_words(p->B, p->H, p->N) * 8;
  const size_t bins_off = (xch_end + 255) / 256 * 256;
  const size_t need = bins_off + (p->pos_bins ? bins8_bytes(p->B, p->N) : 0);
  if (need > NOALLOC_SCRATCH_BYTES)
    return fail("B=%d, H=%d, N=%d%s needs %zu bytes of scratch; the allocation-free forward holds %zu", p->B, p->H,
                p->N, p->pos_bins ? " with pos_bins" : "", need, NOALLOC_SCRATCH_BYTES);
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  if (dev < 0 || dev >= MAX_DEVICES) return fail("device %d outside [0, %d)", dev, MAX_DEVICES);
  ScratchSlot* slot = nullptr;
  {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    slot = &g_scratch[dev];
    if (!slot->ptr) {
      // The array's address on this device (each GPU holds its own copy); the host-side
      // name of the array is not a device address and is never passed to a kernel.
      void* ptr = nullptr;
      e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
      if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
      slot->ptr = static_cast<unsigned char*>(ptr);
      slot->state = WsState{~(uint64_t)0, 0};  // first use clears the exchange region
    }
  }
  const FwdScratch w{slot->ptr, bins_off, false, &slot->state, false, true};
  return run_fwd(a, p->dtype == DFL_BF16, head_dim_pad(p->d), p->storage, w, stream);
}

int dfl_noalloc_error(void* stream) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  if (dev < 0 || dev >= MAX_DEVICES) return fail("device %d outside [0, %d)", dev, MAX_DEVICES);
  unsigned char* base = nullptr;
  {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    base = g_scratch[dev].ptr;
  }
  if (!base) return 0;  // no allocation-free call has run on this device
  return dfl_workspace_error(base, stream);
}

int dfl_sinkhorn_bwd(const dfl_sinkhorn_bwd_params* p, void* workspace, size_t workspace_bytes, void* stream) {
  if (!p) return fail("params is NULL");
  if (p->dtype != DFL_BF16 && p->dtype != DFL_F32) return fail("dtype must be DFL_BF16 or DFL_F32");
  if (p->B <= 0 || p->H <= 0 || p->N <= 0 || p->d <= 0) return fail("B, H, N, d must be positive");
  const int DP = head_dim_pad(p->d);
  if (DP < 0) return fail("head dim d=%d > 64 is not supported", p->d);
  if (p->solver != DFL_IFT_FIXED_POINT && p->solver != DFL_IFT_CG) return fail("unknown solver %d", p->solver);
  if (p->mode != DFL_IFT_REFERENCE && p->mode != DFL_IFT_ANALYTIC) return fail("unknown mode %d", p->mode);
  if (p->iters < 0 || p->iters > 1000) return fail("iters=%d outside [0, 1000]", p->iters);
  if (!p->q || !p->k || !p->v || !p->eps || !p->log_u || !p->log_v || !p->log_z || !p->col_lse || !p->o_avg ||
      !p->x_centroid || !p->grad_o)
    return fail("required input is NULL");
  if (!p->dq || !p->dk || !p->dv || !p->dg || !p->dlog_mu || !p->dlog_nu) return fail("output pointer is NULL");
  if (p->stride_n < p->d) return fail("stride_n must be >= d (unit inner stride)");
  if (p->pos_bins && !p->pos_weight) return fail("pos_bins given without pos_weight");
  const size_t need = dfl_sinkhorn_workspace_size(p->B, p->H, p->N);
  if (!workspace || workspace_bytes < need) return fail("workspace too small: need %zu bytes", need);
  if (p->storage < DFL_STORAGE_AUTO || p->storage > DFL_STORAGE_STREAM) return fail("unknown storage %d", p->storage);
  const int G = group_size(p->B, p->H, p->N);
  const int elem = p->dtype == DFL_BF16 ? 2 : 4;
  int CH = ((p->N + 31) / 32) * 32 < 256 ? ((p->N + 31) / 32) * 32 : 256;  // streamed rows per LDS chunk
  const size_t lds_res = dfl::sinkhorn_bwd_lds_bytes(p->N, DP, elem, G, CH, false);
  const bool stream_mode = p->storage == DFL_STORAGE_STREAM || (p->storage == DFL_STORAGE_AUTO && lds_res > LDS_LIMIT);
  size_t lds = lds_res;
  if (stream_mode) {
    // the largest chunk (multiple of 32 rows) whose staging fits next to the stripes
    for (; CH > 32 && dfl::sinkhorn_bwd_lds_bytes(p->N, DP, elem, G, CH, true) > LDS_LIMIT; CH -= 32) {
    }
    lds = dfl::sinkhorn_bwd_lds_bytes(p->N, DP, elem, G, CH, true);
  }
  if (lds > LDS_LIMIT)
    return fail("N=%d, d=%d, %s storage needs %zu bytes of LDS per workgroup (limit %zu)", p->N, p->d,
                stream_mode ? "stream" : "resident", lds, LDS_LIMIT);

  dfl::SinkBwdArgs a;
  memset(&a, 0, sizeof(a));
  a.q = p->q; a.k = p->k; a.v = p->v; a.g = p->g;
  a.sb = p->stride_b; a.sh = p->stride_h; a.sn = p->stride_n;
  a.x = p->x_res; a.pos_w = p->pos_weight; a.bins = p->pos_bins;
  a.eps = p->eps; a.w_dist = p->w_dist; a.mask = p->mask;
  a.log_u = p->log_u; a.log_v = p->log_v; a.log_z = p->log_z; a.col_lse = p->col_lse;
  a.o_avg = p->o_avg; a.x_centroid = p->x_centroid; a.grad_o = p->grad_o; a.grad_xc = p->grad_xc;
  a.B = p->B; a.H = p->H; a.N = p->N; a.d = p->d;
  a.lam = p->lam; a.r0 = p->r_0;
  a.solver = p->solver; a.iters = p->iters; a.mode = p->mode; a.cg_rtol = p->cg_rtol;
  a.geo_grad = (p->x_res && (p->dx_res || p->dw_dist)) ? 1 : 0;
  a.dq = p->dq; a.dk = p->dk; a.dv = p->dv; a.dg = p->dg;
  a.dlog_mu = p->dlog_mu; a.dlog_nu = p->dlog_nu;
  unsigned char* ws = static_cast<unsigned char*>(workspace);
  a.err = err_ref(ws);
  a.xch = reinterpret_cast<uint64_t*>(ws + WS_HEADER);
  unsigned char* cur = ws + WS_HEADER + xch_words(p->B, p->H, p->N) * 8;
  float* parts = reinterpret_cast<float*>(cur);
  a.dx_part = parts;
  a.dpw_part = parts + (size_t)p->B * p->H * p->N * 3;
  a.dw_part = a.dpw_part + (size_t)p->B * p->H * G * 68;
  cur += partials_bytes(p->B, p->H, p->N, G);
  const size_t opb = prep_operand_bytes(p->B, p->H, p->N);
  a.go_hi = cur;
  a.go_lo = cur + opb;
  a.go_t = cur + 2 * opb;
  a.dcoef = reinterpret_cast<float*>(cur + 3 * opb);
  a.G = G;
  if (int rc = refuse_capture(stream, "dfl_sinkhorn_bwd")) return rc;
  if (int rc = acquire_salt(ws, WS_HEADER + xch_words(p->B, p->H, p->N) * 8, stream, &a.salt))
    return hip_fail((hipError_t)rc, "workspace clear launch");
  a.ch = CH;
  if (p->pos_bins)
    if (int rc = prepare_bins8(p->pos_bins, p->B, p->N, workspace, sinkhorn_bins8_offset(p->B, p->H, p->N),
                               &a.bins8, &a.bins8t, stream))
      return rc;
  // a workspace with room for the bias matrices: the per-element bins lookups and
  // distances are evaluated once here instead of in every sweep
  const bool has_bias = (p->pos_bins && p->pos_weight) || (p->x_res && p->w_dist);
  if (has_bias && workspace_bytes >= need + dfl_sinkhorn_bias_workspace_size(p->B, p->H, p->N)) {
    float* mat = reinterpret_cast<float*>(ws + bias_mat_offset(p->B, p->H, p->N));
    float* matT = mat + (size_t)p->B * p->H * np32(p->N) * np32(p->N);
    hipError_t e = dfl::launch_bias_mat(a, mat, matT, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "bias matrix launch");
    a.bias_mat = mat;
    a.bias_matT = matT;
  }
  const bool coop = coop_launch(G, a.B * a.H);
  hipError_t e = dfl::launch_sinkhorn_bwd_prep(a, p->dtype == DFL_BF16, DP, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "sinkhorn backward prep launch");
  if (stream_mode) {
    const StreamPtrs sp = stream_ptrs(workspace, p->B, p->H, p->N, G);
    dfl::PadArgs pa;
    memset(&pa, 0, sizeof(pa));
    pa.q = p->q; pa.k = p->k; pa.v = p->v;
    pa.sb = p->stride_b; pa.sh = p->stride_h; pa.sn = p->stride_n;
    pa.mask = p->mask;
    pa.B = p->B; pa.H = p->H; pa.N = p->N; pa.d = p->d;
    pa.qp = sp.qp; pa.kp = sp.kp;  // V^T and coordinates are not needed by the backward
    e = dfl::launch_sinkhorn_pad(pa, p->dtype == DFL_BF16, DP, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "sinkhorn pad launch");
    a.qp = sp.qp; a.kp = sp.kp; a.vec_ws = sp.vec;
    e = dfl::launch_sinkhorn_bwd_stream(a, p->dtype == DFL_BF16, DP, lds, (hipStream_t)stream, coop);
  } else {
    e = dfl::launch_sinkhorn_bwd(a, p->dtype == DFL_BF16, DP, lds, (hipStream_t)stream, coop);
  }
  if (e != hipSuccess) return hip_fail(e, "sinkhorn backward launch");
  if (p->dx_res || p->dpos_weight || p->dw_dist) {  // the partial sums feed only these
    e = dfl::launch_sinkhorn_bwd_finalize(a, p->dx_res, p->dpos_weight, p->dw_dist, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "sinkhorn backward finalize launch");
  }
  return 0;
}

size_t dfl_attn_workspace_size(int B, int H, int Mq, int Nk, int d) {
  (void)d;
  if (B <= 0 || H <= 0 || Mq <= 0 || Nk <= 0) return 0;
  return attn_ws_layout(B, H, Mq, Nk).total;
}

int dfl_attn_fwd(const dfl_attn_params* p, void* stream) {
  if (int rc = check_attn(p, false)) return rc;
  const dfl::AttnArgs a = attn_args(p);
  hipError_t e = dfl::launch_attn_fwd(a, p->dtype == DFL_BF16, head_dim_pad(p->d), (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "attention forward launch");
  return 0;
}

int dfl_attn_bwd(const dfl_attn_params* p, void* workspace, size_t workspace_bytes, void* stream) {
  if (int rc = check_attn(p, true)) return rc;
  const AttnWs w = attn_ws_layout(p->B, p->H, p->Mq, p->Nk);
  if (!workspace || workspace_bytes < w.total) return fail("workspace too small: need %zu bytes", w.total);
  dfl::AttnArgs a = attn_args(p);
  unsigned char* ws = static_cast<unsigned char*>(workspace);
  a.do_w = ws + w.do_w;
  a.dcoef = reinterpret_cast<float*>(ws + w.dcoef);
  a.kv_part = reinterpret_cast<float*>(ws + w.kv_part);
  a.dpw_part = reinterpret_cast<float*>(ws + w.dpw_part);
  // the window bias is shared by the batch: with B > 1 its gradient sums per-row slabs
  a.dbias_rows = (p->bias_mode == DFL_ATTN_BIAS_WINDOW && p->dbias && p->B > 1) ? ws + w.dbias_rows : nullptr;
  a.qsplit = attn_qsplit(p->B, p->H, p->Mq, p->Nk);
  if (a.bias_mode != dfl::ATTN_BIAS_DENSE && a.bias_mode != dfl::ATTN_BIAS_WINDOW) a.dbias = nullptr;
  if (!a.g) a.dg = nullptr;
  hipError_t e = dfl::launch_attn_bwd(a, p->dtype == DFL_BF16, head_dim_pad(p->d), (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "attention backward launch");
  return 0;
}

size_t dfl_a2t_workspace_size(int B, int H, int M, int d) {
  if (B <= 0 || H <= 0 || M <= 0 || d <= 0) return 0;
  return ((size_t)B * H * M * 2 * d * 4 + 255) / 256 * 256;
}

int dfl_a2t_fwd(const dfl_a2t_params* p, void* stream) {
  if (int rc = check_a2t(p, false)) return rc;
  hipError_t e = dfl::launch_a2t_fwd(a2t_args(p), p->dtype == DFL_BF16, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "atom-to-token forward launch");
  return 0;
}

int dfl_a2t_bwd(const dfl_a2t_params* p, void* workspace, size_t workspace_bytes, void* stream) {
  if (int rc = check_a2t(p, true)) return rc;
  const size_t need = dfl_a2t_workspace_size(p->B, p->H, p->M, p->d);
  if (!workspace || workspace_bytes < need) return fail("workspace too small: need %zu bytes", need);
  dfl::A2TArgs a = a2t_args(p);
  a.dkv = static_cast<float*>(workspace);
  hipError_t e = dfl::launch_a2t_bwd(a, p->dtype == DFL_BF16, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "atom-to-token backward launch");
  return 0;
}

// ---------------------------------------------------------------------------
// Dense (materialised-cost) Sinkhorn
size_t dfl_dense_sinkhorn_workspace_size(int B, int H, int N, int K) {
  if (B <= 0 || H <= 0 || N <= 0 || K < 0) return 0;
  const size_t bhn = (size_t)B * H * N;
  return ((size_t)2 * (K + 1) * 4 + 255) / 256 * 256 + (2 * bhn * 4 + 255) / 256 * 256;
}

int dfl_dense_sinkhorn_fwd(const dfl_dense_sinkhorn_params* p, void* workspace, size_t workspace_bytes,
                           void* stream) {
  if (!p) return fail("params is NULL");
  if (p->B <= 0 || p->H <= 0 || p->N <= 0) return fail("B, H, N must be positive");
  if (p->K < 0 || p->K > 100000) return fail("K=%d outside [0, 100000]", p->K);
  if (!p->C || !p->log_mu || !p->log_nu || !p->eps || !p->log_u || !p->log_v || !p->history)
    return fail("required pointer is NULL");
  if (p->threshold >= 0.f && p->check_every <= 0) return fail("check_every must be positive");
  const size_t need = dfl_dense_sinkhorn_workspace_size(p->B, p->H, p->N, p->K);
  if (!workspace || workspace_bytes < need) return fail("workspace too small: need %zu bytes", need);
  const size_t bhn = (size_t)p->B * p->H * p->N;
  dfl::DenseSinkArgs a;
  memset(&a, 0, sizeof(a));
  a.C = p->C; a.log_mu = p->log_mu; a.log_nu = p->log_nu; a.eps = p->eps;
  a.u_init = p->log_u_init; a.v_init = p->log_v_init; a.mask = p->mask;
  a.B = p->B; a.H = p->H; a.N = p->N; a.K = p->K; a.lam = p->lam;
  const size_t slices = (size_t)(p->K + 1) * bhn;
  a.hist_u = p->history;
  a.hist_v = p->history + slices;
  a.hist_r = p->history + 2 * slices;
  a.hist_c = p->history + 3 * slices;
  const bool early = p->threshold >= 0.f;
  a.delta = early ? static_cast<uint32_t*>(workspace) : nullptr;
  a.log_u = p->log_u; a.log_v = p->log_v;
  hipStream_t s = (hipStream_t)stream;
  hipError_t e = dfl::dense_sinkhorn_init(a, s);
  if (e != hipSuccess) return hip_fail(e, "dense sinkhorn init launch");
  int done = 0;
  for (int k = 1; k <= p->K; ++k) {
    e = dfl::dense_sinkhorn_iteration(a, k, s);
    if (e != hipSuccess) return hip_fail(e, "dense sinkhorn iteration launch");
    done = k;
    if (early && k % p->check_every == 0) {
      uint32_t words[2] = {0, 0};
      e = hipMemcpyAsync(words, a.delta + 2 * k, sizeof(words), hipMemcpyDeviceToHost, s);
      if (e != hipSuccess) return hip_fail(e, "dense sinkhorn change copy");
      e = hipStreamSynchronize(s);
      if (e != hipSuccess) return hip_fail(e, "dense sinkhorn change sync");
      float du, dv;
      memcpy(&du, &words[0], 4);
      memcpy(&dv, &words[1], 4);
      if ((du > dv ? du : dv) < p->threshold) break;
    }
  }
  e = dfl::dense_sinkhorn_finish(a, done, s);
  if (e != hipSuccess) return hip_fail(e, "dense sinkhorn finish launch");
  if (p->iters_done) *p->iters_done = done;
  return 0;
}

int dfl_dense_sinkhorn_bwd(const dfl_dense_sinkhorn_bwd_params* p, void* workspace, size_t workspace_bytes,
                           void* stream) {
  if (!p) return fail("params is NULL");
  if (p->B <= 0 || p->H <= 0 || p->N <= 0) return fail("B, H, N must be positive");
  if (p->K < 0 || p->K > p->K_max) return fail("K=%d outside [0, K_max=%d]", p->K, p->K_max);
  if (!p->C || !p->eps || !p->history || !p->dC || !p->dlog_mu || !p->dlog_nu) return fail("required pointer is NULL");
  const size_t need = dfl_dense_sinkhorn_workspace_size(p->B, p->H, p->N, p->K_max);
  if (!workspace || workspace_bytes < need) return fail("workspace too small: need %zu bytes", need);
  const size_t bhn = (size_t)p->B * p->H * p->N;
  dfl::DenseSinkBwdArgs a;
  memset(&a, 0, sizeof(a));
  a.C = p->C; a.eps = p->eps; a.mask = p->mask;
  const size_t slices = (size_t)(p->K_max + 1) * bhn;
  a.hist_u = p->history;
  a.hist_v = p->history + slices;
  a.hist_r = p->history + 2 * slices;
  a.hist_c = p->history + 3 * slices;
  a.B = p->B; a.H = p->H; a.N = p->N; a.K = p->K; a.lam = p->lam;
  a.grad_u = p->grad_log_u; a.grad_v = p->grad_log_v;
  a.dC = p->dC; a.dlog_mu = p->dlog_mu; a.dlog_nu = p->dlog_nu;
  a.dlog_u_init = p->dlog_u_init; a.dlog_v_init = p->dlog_v_init;
  unsigned char* ws = static_cast<unsigned char*>(workspace);
  float* vecs = reinterpret_cast<float*>(ws + ((size_t)2 * (p->K_max + 1) * 4 + 255) / 256 * 256);
  a.gv = vecs;
  a.avec = vecs + bhn;
  hipStream_t s = (hipStream_t)stream;
  hipError_t e;
  if (p->K == 0) {  // outputs are the (masked) initial potentials: dC, d log mu, d log nu vanish
    e = dfl::dense_zero(p->dC, bhn * p->N, s);
    if (e == hipSuccess) e = dfl::dense_zero(p->dlog_mu, bhn, s);
    if (e == hipSuccess) e = dfl::dense_zero(p->dlog_nu, bhn, s);
    if (e != hipSuccess) return hip_fail(e, "dense sinkhorn backward zero launch");
  }
  e = dfl::dense_sinkhorn_backward(a, s);
  if (e != hipSuccess) return hip_fail(e, "dense sinkhorn backward launch");
  return 0;
}

size_t dfl_dense_transport_workspace_size(int B, int H, int N, int d) {
  if (B <= 0 || H <= 0 || N <= 0 || d <= 0) return 0;
  const size_t bhn = (size_t)B * H * N;
  return (bhn * d * 4 + 255) / 256 * 256 + (bhn * 3 * 4 + 255) / 256 * 256;
}

static int check_transport(const dfl_dense_transport_params* p) {
  if (!p) return fail("params is NULL");
  if (p->B <= 0 || p->H <= 0 || p->N <= 0 || p->d <= 0) return fail("B, H, N, d must be positive");
  if (p->d > 64) return fail("head dim d=%d > 64 is not supported", p->d);
  if (!p->V || !p->log_u || !p->log_v || !p->C || !p->eps) return fail("required input is NULL");
  return 0;
}

static dfl::DenseTransportArgs transport_args(const dfl_dense_transport_params* p) {
  dfl::DenseTransportArgs a;
  memset(&a, 0, sizeof(a));
  a.V = p->V; a.G = p->G; a.log_u = p->log_u; a.log_v = p->log_v; a.C = p->C; a.eps = p->eps;
  a.x_res = p->x_res; a.mask = p->mask;
  a.B = p->B; a.H = p->H; a.N = p->N; a.d = p->d;
  a.o = p->o; a.T_norm = p->T_norm; a.x_centroid = p->x_res ? p->x_centroid : nullptr; a.o_avg = p->o_avg;
  a.grad_o = p->grad_o; a.grad_T = p->grad_T; a.grad_xc = p->grad_xc;
  a.dV = p->dV; a.dG = p->G ? p->dG : nullptr; a.dlog_u = p->dlog_u; a.dlog_v = p->dlog_v; a.dC = p->dC;
  a.dx_res = p->x_res ? p->dx_res : nullptr;
  return a;
}

int dfl_dense_transport_fwd(const dfl_dense_transport_params* p, void* stream) {
  if (int rc = check_transport(p)) return rc;
  if (!p->o || !p->T_norm || !p->o_avg) return fail("o, T_norm and o_avg are required");
  if (p->x_res && !p->x_centroid) return fail("x_centroid is required with x_res");
  hipError_t e = dfl::dense_transport_forward(transport_args(p), (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "dense transport forward launch");
  return 0;
}

int dfl_dense_transport_bwd(const dfl_dense_transport_params* p, void* workspace, size_t workspace_bytes,
                            void* stream) {
  if (int rc = check_transport(p)) return rc;
  if (!p->T_norm || !p->o_avg || !p->dV || !p->dlog_u || !p->dlog_v || !p->dC)
    return fail("T_norm, o_avg, dV, dlog_u, dlog_v and dC are required");
  const size_t need = dfl_dense_transport_workspace_size(p->B, p->H, p->N, p->d);
  if (!workspace || workspace_bytes < need) return fail("workspace too small: need %zu bytes", need);
  dfl::DenseTransportArgs a = transport_args(p);
  const size_t bhn = (size_t)p->B * p->H * p->N;
  unsigned char* ws = static_cast<unsigned char*>(workspace);
  a.goa = reinterpret_cast<float*>(ws);
  a.dx_part = p->x_res ? reinterpret_cast<float*>(ws + (bhn * p->d * 4 + 255) / 256 * 256) : nullptr;
  hipError_t e = dfl::dense_transport_backward(a, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "dense transport backward launch");
  return 0;
}

size_t dfl_balanced_workspace_size(int B, int H, int N, int d, int backward) {
  if (B <= 0 || H <= 0 || N <= 0 || d <= 0) return 0;
  const size_t f = bal_fwd_need(B, H, N, d, DFL_STORAGE_AUTO);
  if (!backward) return f;
  const size_t b = bal_ws_layout(B, H, N, d).total;
  return f > b ? f : b;
}

int dfl_balanced_fwd(const dfl_balanced_fwd_params* p, void* workspace, size_t workspace_bytes, void* stream) {
  if (!p) return fail("params is NULL");
  if (int rc = check_balanced(p->dtype, p->q, p->k, p->x_res, p->eps, p->alpha_h, p->r_h, p->B, p->H, p->N, p->d,
                              p->K_iter, p->stride_n))
    return rc;
  if (!p->x_centroid || !p->log_u || !p->log_v || !p->log_z || !p->hist) return fail("output pointer is NULL");
  if (p->h_centroid && !p->v) return fail("h_centroid needs v");
  if (p->storage < DFL_STORAGE_AUTO || p->storage > DFL_STORAGE_STREAM) return fail("unknown storage %d", p->storage);
  const size_t need = bal_fwd_need(p->B, p->H, p->N, p->d, p->storage);
  if (!workspace || workspace_bytes < need) return fail("workspace too small: need %zu bytes", need);
  dfl::SinkFwdArgs a;
  memset(&a, 0, sizeof(a));
  a.q = p->q; a.k = p->k; a.v = p->h_centroid ? p->v : nullptr;
  a.sb = p->stride_b; a.sh = p->stride_h; a.sn = p->stride_n;
  a.x = p->x_res; a.eps = p->eps; a.mask = p->mask;
  a.B = p->B; a.H = p->H; a.N = p->N; a.d = p->d;
  a.K_iter = p->K_iter; a.lam = 1.f; a.r0 = 1.f;
  a.x_centroid = p->x_centroid; a.o_avg = p->h_centroid;
  a.log_u = p->log_u; a.log_v = p->log_v; a.log_z = p->log_z;
  a.balanced = 1; a.alpha = p->alpha_h; a.r_h = p->r_h; a.hist = p->hist;
  const FwdScratch w{static_cast<unsigned char*>(workspace), 0, true, nullptr, true, false};  // no bins
  return run_fwd(a, false, head_dim_pad(p->d), p->storage, w, stream);
}

int dfl_balanced_bwd(const dfl_balanced_bwd_params* p, void* workspace, size_t workspace_bytes, void* stream) {
  if (!p) return fail("params is NULL");
  if (int rc = check_balanced(p->dtype, p->q, p->k, p->x_res, p->eps, p->alpha_h, p->r_h, p->B, p->H, p->N, p->d,
                              p->K_iter, p->stride_n))
    return rc;
  if (!p->x_centroid || !p->hist) return fail("x_centroid and hist are required");
  if (p->grad_hc && (!p->v || !p->h_centroid)) return fail("grad_hc needs v and h_centroid");
  if (!p->dq || !p->dk || !p->dx_res || !p->dalpha_h || !p->dr_h) return fail("output pointer is NULL");
  const size_t need = bal_ws_layout(p->B, p->H, p->N, p->d).total;
  if (!workspace || workspace_bytes < need) return fail("workspace too small: need %zu bytes", need);
  const int DP = head_dim_pad(p->d);
  const int G = group_size(p->B, p->H, p->N);
  const int max_nr = ((p->N + 15) / 16 + G - 1) / G;
  if (max_nr > dfl::balanced_max_tiles(DP))
    return fail("balanced backward: N=%d over %d workgroups per (b,h) exceeds %d tiles of 16 rows each", p->N, G,
                dfl::balanced_max_tiles(DP));
  const size_t lds = dfl::balanced_bwd_lds_bytes(p->N, DP);
  if (lds > LDS_LIMIT)
    return fail("balanced backward: N=%d needs %zu bytes of LDS per workgroup (limit %zu)", p->N, lds, LDS_LIMIT);
  unsigned char* ws = static_cast<unsigned char*>(workspace);
  const BalWs L = bal_ws_layout(p->B, p->H, p->N, p->d);
  auto F = [&](size_t off) { return reinterpret_cast<float*>(ws + off); };
  const bool has_h = p->grad_hc != nullptr;
  dfl::BalPrepArgs pr;
  memset(&pr, 0, sizeof(pr));
  pr.q = static_cast<const float*>(p->q); pr.k = static_cast<const float*>(p->k);
  pr.v = static_cast<const float*>(p->v);
  pr.sb = p->stride_b; pr.sh = p->stride_h; pr.sn = p->stride_n;
  pr.x = p->x_res; pr.mask = p->mask; pr.xc = p->x_centroid; pr.hc = p->h_centroid;
  pr.gxc = p->grad_xc; pr.ghc = p->grad_hc;
  pr.B = p->B; pr.H = p->H; pr.N = p->N; pr.d = p->d;
  pr.qp = F(L.qp); pr.kp = F(L.kp); pr.qt = F(L.qt); pr.kt = F(L.kt);
  pr.vp = has_h ? F(L.vp) : nullptr; pr.gp = has_h ? F(L.gp) : nullptr; pr.gt = has_h ? F(L.gt) : nullptr;
  pr.dcoef = F(L.dcoef); pr.gxs = F(L.gxs); pr.xs = F(L.xs);
  hipError_t e = dfl::launch_balanced_prep(pr, DP, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "balanced backward prep launch");
  dfl::BalBwdArgs a;
  memset(&a, 0, sizeof(a));
  a.B = p->B; a.H = p->H; a.N = p->N; a.d = p->d; a.K = p->K_iter;
  a.eps = p->eps; a.alpha = p->alpha_h; a.r_h = p->r_h; a.mask = p->mask; a.hist = p->hist;
  a.qp = pr.qp; a.kp = pr.kp; a.qt = pr.qt; a.kt = pr.kt; a.vp = pr.vp; a.gp = pr.gp; a.gt = pr.gt;
  a.dcoef = pr.dcoef; a.gxs = pr.gxs; a.xs = pr.xs; a.has_h = has_h ? 1 : 0;
  a.dq = p->dq; a.dk = p->dk; a.dv = p->dv; a.dx_part = F(L.dx_part); a.ar_part = F(L.ar_part);
  a.err = err_ref(ws);
  a.xch = reinterpret_cast<uint64_t*>(ws + WS_HEADER);
  a.G = G;
  if (int rc = refuse_capture(stream, "dfl_balanced_bwd")) return rc;
  if (int rc = acquire_salt(ws, WS_HEADER + xch_words(p->B, p->H, p->N) * 8, stream, &a.salt))
    return hip_fail((hipError_t)rc, "workspace clear launch");
  e = dfl::launch_balanced_bwd(a, DP, lds, (hipStream_t)stream, coop_launch(G, a.B * a.H));
  if (e != hipSuccess) return hip_fail(e, "balanced backward launch");
  e = dfl::launch_balanced_finalize(a, p->dx_res, p->dalpha_h, p->dr_h, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "balanced backward finalize launch");
  return 0;
}

size_t dfl_sinkhorn_unrolled_workspace_size(int B, int H, int N, int d) {
  if (B <= 0 || H <= 0 || N <= 0 || d <= 0) return 0;
  return unr_ws_layout(B, H, N, d).total;
}

int dfl_sinkhorn_unrolled_bwd(const dfl_sinkhorn_unrolled_bwd_params* p, void* workspace, size_t workspace_bytes,
                              void* stream) {
  if (!p) return fail("params is NULL");
  if (p->dtype != DFL_BF16 && p->dtype != DFL_F32) return fail("dtype must be DFL_BF16 or DFL_F32");
  if (p->B <= 0 || p->H <= 0 || p->N <= 0 || p->d <= 0) return fail("B, H, N, d must be positive");
  const int DP = head_dim_pad(p->d);
  if (DP < 0) return fail("head dim d=%d > 64 is not supported", p->d);
  if (p->K_iter < 1 || p->K_iter > 1000) return fail("K_iter=%d outside [1, 1000]", p->K_iter);
  if (!p->q || !p->k || !p->v || !p->eps || !p->log_mu || !p->log_nu || !p->o_avg || !p->x_centroid || !p->log_u ||
      !p->log_z || !p->hist || !p->grad_o)
    return fail("required input is NULL");
  if (!p->dq || !p->dk || !p->dv || !p->dlog_mu || !p->dlog_nu || (p->g && !p->dg))
    return fail("output pointer is NULL");
  if (p->stride_n < p->d) return fail("stride_n must be >= d (unit inner stride)");
  if (p->pos_bins && !p->pos_weight) return fail("pos_bins given without pos_weight");
  const UnrWs L = unr_ws_layout(p->B, p->H, p->N, p->d);
  if (!workspace || workspace_bytes < L.total) return fail("workspace too small: need %zu bytes", L.total);
  const int G = group_size(p->B, p->H, p->N);
  const int max_nr = ((p->N + 15) / 16 + G - 1) / G;
  if (max_nr > dfl::unrolled_max_tiles(DP))
    return fail("unrolled backward: N=%d over %d workgroups per (b,h) exceeds %d tiles of 16 rows each", p->N, G,
                dfl::unrolled_max_tiles(DP));
  const int elem = p->dtype == DFL_BF16 ? 2 : 4;
  const int ops = dfl::unrolled_operand_mode(p->N, DP, elem, LDS_LIMIT);
  const size_t lds = dfl::unrolled_bwd_lds_bytes(p->N, DP, elem, ops);
  if (lds > LDS_LIMIT)
    return fail("unrolled backward: N=%d needs %zu bytes of LDS per workgroup (limit %zu)", p->N, lds, LDS_LIMIT);
  unsigned char* ws = static_cast<unsigned char*>(workspace);
  auto F = [&](size_t off) { return reinterpret_cast<float*>(ws + off); };
  dfl::UnrPrepArgs pr;
  memset(&pr, 0, sizeof(pr));
  pr.q = p->q; pr.k = p->k; pr.v = p->v; pr.g = p->g;
  pr.sb = p->stride_b; pr.sh = p->stride_h; pr.sn = p->stride_n;
  pr.x = p->x_res; pr.mask = p->mask; pr.o_avg = p->o_avg; pr.xc = p->x_centroid;
  pr.grad_o = p->grad_o; pr.grad_xc = p->grad_xc;
  pr.B = p->B; pr.H = p->H; pr.N = p->N; pr.d = p->d;
  pr.qp = F(L.qp); pr.kp = F(L.kp); pr.qt = F(L.qt); pr.kt = F(L.kt);
  pr.vp = F(L.vp); pr.gp = F(L.gp); pr.gt = F(L.gt);
  pr.dcoef = F(L.dcoef); pr.gxs = F(L.gxs); pr.xs = F(L.xs); pr.dg = p->dg;
  hipError_t e = dfl::launch_unrolled_prep(pr, p->dtype == DFL_BF16, DP, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "unrolled backward prep launch");
  dfl::UnrBwdArgs a;
  memset(&a, 0, sizeof(a));
  a.B = p->B; a.H = p->H; a.N = p->N; a.d = p->d; a.K = p->K_iter;
  a.eps = p->eps; a.lam = p->lam; a.r0 = p->r_0; a.mask = p->mask; a.hist = p->hist;
  a.log_mu = p->log_mu; a.log_nu = p->log_nu; a.log_u = p->log_u; a.log_z = p->log_z; a.v_init = p->log_v_init;
  if (int rc = prepare_bins8(p->pos_bins, p->B, p->N, workspace, L.total - bins8_bytes(p->B, p->N), &a.bins8,
                             &a.bins8t, stream))
    return rc;
  a.pos_w = p->pos_weight; a.w_dist = p->w_dist;
  a.has_geo = (p->x_res && p->w_dist) ? 1 : 0;
  a.qp = pr.qp; a.kp = pr.kp; a.qt = pr.qt; a.kt = pr.kt; a.vp = pr.vp; a.gp = pr.gp; a.gt = pr.gt;
  a.dcoef = pr.dcoef; a.gxs = pr.gxs; a.xs = pr.xs;
  a.dq = p->dq; a.dk = p->dk; a.dv = p->dv; a.dlog_mu = p->dlog_mu; a.dlog_nu = p->dlog_nu;
  a.dv_init = p->dlog_v_init;
  a.dx_part = F(L.dx_part); a.dpw_part = F(L.dpw_part); a.dw_part = F(L.dw_part);
  a.err = err_ref(ws);
  a.xch = reinterpret_cast<uint64_t*>(ws + WS_HEADER);
  a.G = G;
  if (int rc = refuse_capture(stream, "dfl_sinkhorn_unrolled_bwd")) return rc;
  if (int rc = acquire_salt(ws, WS_HEADER + xch_words(p->B, p->H, p->N) * 8, stream, &a.salt))
    return hip_fail((hipError_t)rc, "workspace clear launch");
  e = dfl::launch_unrolled_bwd(a, p->dtype == DFL_BF16, DP, lds, (hipStream_t)stream, coop_launch(G, a.B * a.H),
                               ops);
  if (e != hipSuccess) return hip_fail(e, "unrolled backward launch");
  e = dfl::launch_unrolled_finalize(a, p->x_res ? p->dx_res : nullptr, p->dpos_weight, p->dw_dist,
                                    (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "unrolled backward finalize launch");
  return 0;
}

// ---------------------------------------------------------------------------
// TokenOTBlock steps either side of the balanced transport.

static size_t r256z(size_t x) { return (x + 255) / 256 * 256; }
static constexpr int TRUNK_PARTS = 64;  // partial rows written by the per-token kernels

static int check_proj(const dfl_sink_proj_params* p) {
  if (!p) return fail("params is NULL");
  if (p->dtype != DFL_F32 && p->dtype != DFL_BF16) return fail("dtype must be DFL_F32 or DFL_BF16");
  if (p->M <= 0 || p->C <= 0 || p->H <= 0) return fail("M, C, H must be positive");
  if (p->C % 64 != 0 || p->C > 1024 || p->C % p->H != 0)
    return fail("C=%d must be a multiple of 64 and of H=%d, at most 1024", p->C, p->H);
  const int dh = p->C / p->H;
  if (dh != 16 && dh != 32 && dh != 64) return fail("head dim C/H=%d must be 16, 32 or 64", dh);
  if (dfl::proj_fwd_lds_bytes(p->C, p->dtype == DFL_BF16) + 1024 > LDS_LIMIT)
    return fail("C=%d too large for the %s projection (LDS)", p->C, p->dtype == DFL_BF16 ? "bf16" : "fp32");
  if (!p->h || !p->ln_weight || !p->ln_bias || !p->w_q || !p->w_k) return fail("required input is NULL");
  return 0;
}

static dfl::ProjArgs proj_args(const dfl_sink_proj_params* p) {
  dfl::ProjArgs a;
  memset(&a, 0, sizeof(a));
  a.h = p->h; a.ln_w = p->ln_weight; a.ln_b = p->ln_bias;
  a.w[0] = p->w_q; a.w[1] = p->w_k; a.w[2] = p->w_v;
  a.y[0] = p->q_s; a.y[1] = p->k_s; a.y[2] = p->v_s;
  a.norm[0] = p->q_norm; a.norm[1] = p->k_norm;
  a.mean = p->ln_mean; a.rstd = p->ln_rstd;
  a.M = p->M; a.C = p->C; a.H = p->H;
  return a;
}

size_t dfl_sink_proj_workspace_size(int M, int C) {
  if (M <= 0 || C <= 0) return 0;
  const size_t mc = r256z((size_t)M * C * 4);
  return 6 * mc + r256z((size_t)TRUNK_PARTS * 2 * C * 4);  // du x3, xa, xn, dxa; LayerNorm partials
}

int dfl_sink_proj_fwd(const dfl_sink_proj_params* p, void* stream) {
  if (int rc = check_proj(p)) return rc;
  if (!p->q_s || !p->k_s || (p->w_v && !p->v_s) || !p->q_norm || !p->k_norm || !p->ln_mean || !p->ln_rstd)
    return fail("output pointer is NULL");
  hipError_t e = dfl::launch_proj_fwd(proj_args(p), p->dtype == DFL_BF16, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "sink projection launch");
  return 0;
}

int dfl_sink_proj_bwd(const dfl_sink_proj_params* p, void* workspace, size_t workspace_bytes, void* stream) {
  if (int rc = check_proj(p)) return rc;
  if (!p->q_s || !p->k_s || !p->q_norm || !p->k_norm || !p->ln_mean || !p->ln_rstd)
    return fail("saved forward value is NULL");
  if (!p->dh) return fail("dh is NULL");
  if (p->dw_v && !p->w_v) return fail("dw_v needs w_v");
  const size_t need = dfl_sink_proj_workspace_size(p->M, p->C);
  if (!workspace || workspace_bytes < need) return fail("workspace too small: need %zu bytes", need);
  dfl::ProjArgs a = proj_args(p);
  unsigned char* ws = static_cast<unsigned char*>(workspace);
  const size_t mc = r256z((size_t)p->M * p->C * 4);
  for (int i = 0; i < 3; ++i) a.du[i] = reinterpret_cast<float*>(ws + i * mc);
  a.xa = reinterpret_cast<float*>(ws + 3 * mc);
  a.xn = reinterpret_cast<float*>(ws + 4 * mc);
  a.dxa = reinterpret_cast<float*>(ws + 5 * mc);
  a.part = reinterpret_cast<float*>(ws + 6 * mc);
  a.dy[0] = p->dq_s; a.dy[1] = p->dk_s; a.dy[2] = p->w_v ? p->dv_s : nullptr;
  a.dh = p->dh; a.dln_w = p->dln_weight; a.dln_b = p->dln_bias;
  a.dw[0] = p->dw_q; a.dw[1] = p->dw_k; a.dw[2] = p->dw_v;
  hipError_t e = dfl::launch_proj_bwd(a, p->dtype == DFL_BF16, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "sink projection backward launch");
  return 0;
}

static int check_coord(const dfl_coord_update_params* p) {
  if (!p) return fail("params is NULL");
  if (p->dtype != DFL_F32 && p->dtype != DFL_BF16) return fail("dtype must be DFL_F32 or DFL_BF16");
  if (p->B <= 0 || p->N <= 0 || p->C <= 0 || p->H <= 0) return fail("B, N, C, H must be positive");
  if (p->C % 64 != 0 || p->C > 1024) return fail("C=%d must be a multiple of 64 and at most 1024", p->C);
  if (p->H > 64) return fail("H=%d > 64 is not supported", p->H);
  if (!p->h || !p->ln_weight || !p->ln_bias || !p->w_gate || !p->b_gate || !p->lambda_raw || !p->x_centroid ||
      !p->x_res)
    return fail("required input is NULL");
  return 0;
}

static dfl::CoordArgs coord_args(const dfl_coord_update_params* p) {
  dfl::CoordArgs a;
  memset(&a, 0, sizeof(a));
  a.h = p->h; a.ln_w = p->ln_weight; a.ln_b = p->ln_bias; a.w_gate = p->w_gate; a.b_gate = p->b_gate;
  a.lam_raw = p->lambda_raw; a.xc = p->x_centroid; a.x = p->x_res; a.mask = p->mask; a.x_out = p->x_out;
  a.B = p->B; a.N = p->N; a.C = p->C; a.H = p->H;
  return a;
}

size_t dfl_coord_update_workspace_size(int C, int H) {
  if (C <= 0 || H <= 0) return 0;
  return r256z((size_t)TRUNK_PARTS * (3 * C + H + 1) * 4);
}

int dfl_coord_update_fwd(const dfl_coord_update_params* p, void* stream) {
  if (int rc = check_coord(p)) return rc;
  if (!p->x_out) return fail("x_out is NULL");
  hipError_t e = dfl::launch_coord(coord_args(p), p->dtype == DFL_BF16, false, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "coordinate update launch");
  return 0;
}

int dfl_coord_update_bwd(const dfl_coord_update_params* p, void* workspace, size_t workspace_bytes, void* stream) {
  if (int rc = check_coord(p)) return rc;
  if (!p->dx_out || !p->dx_res || !p->dx_centroid || !p->dh) return fail("gradient pointer is NULL");
  const size_t need = dfl_coord_update_workspace_size(p->C, p->H);
  if (!workspace || workspace_bytes < need) return fail("workspace too small: need %zu bytes", need);
  dfl::CoordArgs a = coord_args(p);
  a.dx_out = p->dx_out; a.dx = p->dx_res; a.dxc = p->dx_centroid; a.dh = p->dh;
  a.dln_w = p->dln_weight; a.dln_b = p->dln_bias; a.dw_gate = p->dw_gate; a.db_gate = p->db_gate;
  a.dlam_raw = p->dlambda_raw;
  a.part = static_cast<float*>(workspace);
  hipError_t e = dfl::launch_coord(a, p->dtype == DFL_BF16, true, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "coordinate update backward launch");
  return 0;
}

}  // extern "C"
