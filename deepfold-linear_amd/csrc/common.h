// Shared device-side building blocks for the deepfold_amd HIP kernels (gfx950).
//
//  * MFMA fragment traits for bf16 (v_mfma_f32_16x16x32_bf16) and fp32
//    (v_mfma_f32_16x16x4_f32) tiles with one unified LDS fragment layout.
//  * Tagged device-scope exchange: 64-bit words {tag, float} written and polled
//    with relaxed agent-scope atomics.  Each word carries its own round tag, so no
//    fences are needed (agent-scope acquire/release fences cost ~8 us each on
//    MI355X because they write back / invalidate the whole L2).
//  * Error flag + bounded spins so every wave of a persistent kernel terminates.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <map>
#include <mutex>
#include <utility>

namespace dfl {

// Raises a kernel's dynamic-LDS limit once per (kernel, device) and size: the
// attribute call costs host time that would otherwise sit in front of every launch.
inline hipError_t set_lds_limit(const void* kern, size_t lds) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  static std::mutex mu;
  static std::map<std::pair<const void*, int>, size_t> done;
  std::lock_guard<std::mutex> lock(mu);
  const auto key = std::make_pair(kern, dev);
  const auto it = done.find(key);
  if (it != done.end() && it->second >= lds) return hipSuccess;
  e = hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (e == hipSuccess) done[key] = lds;
  return e;
}

typedef __bf16 bf16;
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;

constexpr float LOG2E = 1.4426950408889634f;
constexpr float LN2 = 0.6931471805599453f;
constexpr float NEG_BIG = -1.0e30f;  // masked logit (log2 units); exp2 -> 0

constexpr int WAVE = 64;

// ---------------------------------------------------------------------------
// conversions
__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(bf16 x) { return (float)x; }
template <typename T> __device__ __forceinline__ T from_f32(float x);
template <> __device__ __forceinline__ float from_f32<float>(float x) { return x; }
template <> __device__ __forceinline__ bf16 from_f32<bf16>(float x) { return (bf16)x; }

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float fast_log2(float x) { return __builtin_amdgcn_logf(x); }

// ---------------------------------------------------------------------------
// MFMA traits.
//
// A 16x16 output tile D[m][n] lives in 4 fp32 registers per lane:
//   lane l holds D[4*(l/16) + r][l % 16], r = 0..3.
// QK-type products D = A * B^T with A rows (m) and B rows (n) taken from LDS
// arrays stored row-major [row][DP] (DP = padded head dim, multiple of 32 for
// bf16 and of 4 for fp32).  Both operands use the same k permutation: lane
// group g = l/16 owns the contiguous column run [g*DP/4, (g+1)*DP/4) of its row
// (row = l % 16), which is loaded with one vector read.
//
// PV-type products O[i][c] += sum_j P[i][j] V[j][c] consume P straight from the
// QK-type accumulator layout of two consecutive 16-row streamed tiles; V comes
// from an LDS array stored transposed [c][j].
template <typename T, int DP> struct Mfma;

template <int DP> struct Mfma<bf16, DP> {
  static_assert(DP % 32 == 0, "bf16 head dim must be padded to 32");
  static constexpr int KSTEPS = DP / 32;
  static constexpr int RUN = DP / 4;  // elements per lane per row
  struct Frag { bf16x8 v[KSTEPS]; };
  __device__ static __forceinline__ void load(Frag& f, const bf16* row_base, int lane) {
    // row_base points at row (l%16) of the tile already
    const bf16* p = row_base + (lane >> 4) * RUN;
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) f.v[s] = *reinterpret_cast<const bf16x8*>(p + 8 * s);
  }
  // run: the RUN elements this lane owns, in column order
  __device__ static __forceinline__ void from_run(Frag& f, const bf16* run) {
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s)
#pragma unroll
      for (int e = 0; e < 8; ++e) f.v[s][e] = run[8 * s + e];
  }
  __device__ static __forceinline__ f32x4 qk(const Frag& a, const Frag& b, f32x4 c) {
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.v[s], b.v[s], c, 0, 0, 0);
    return c;
  }
  // P: two tiles of accumulator values p0 (streamed rows 0..15), p1 (16..31).
  // vt_row: LDS pointer to row (c0 + l%16) of the transposed V array, at column j0.
  __device__ static __forceinline__ f32x4 pv(const f32x4& p0, const f32x4& p1, const bf16* vt_row, int lane,
                                             f32x4 acc) {
    const int g = lane >> 4;
    bf16x8 a, b;
    a[0] = (bf16)p0[0]; a[1] = (bf16)p0[1]; a[2] = (bf16)p0[2]; a[3] = (bf16)p0[3];
    a[4] = (bf16)p1[0]; a[5] = (bf16)p1[1]; a[6] = (bf16)p1[2]; a[7] = (bf16)p1[3];
    bf16x4 lo = *reinterpret_cast<const bf16x4*>(vt_row + 4 * g);
    bf16x4 hi = *reinterpret_cast<const bf16x4*>(vt_row + 16 + 4 * g);
    b[0] = lo[0]; b[1] = lo[1]; b[2] = lo[2]; b[3] = lo[3];
    b[4] = hi[0]; b[5] = hi[1]; b[6] = hi[2]; b[7] = hi[3];
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc, 0, 0, 0);
  }
  // Same product with P carried as a hi + lo pair of bf16 values (~16-bit
  // mantissa): two MFMAs against the same V operand.
  __device__ static __forceinline__ f32x4 pv_split(const f32x4& p0, const f32x4& p1, const bf16* vt_row, int lane,
                                                   f32x4 acc) {
    const int g = lane >> 4;
    bf16x8 ah, al, b;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const bf16 h0 = (bf16)p0[r], h1 = (bf16)p1[r];
      ah[r] = h0; ah[4 + r] = h1;
      al[r] = (bf16)(p0[r] - (float)h0); al[4 + r] = (bf16)(p1[r] - (float)h1);
    }
    bf16x4 lo = *reinterpret_cast<const bf16x4*>(vt_row + 4 * g);
    bf16x4 hi = *reinterpret_cast<const bf16x4*>(vt_row + 16 + 4 * g);
    b[0] = lo[0]; b[1] = lo[1]; b[2] = lo[2]; b[3] = lo[3];
    b[4] = hi[0]; b[5] = hi[1]; b[6] = hi[2]; b[7] = hi[3];
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, b, acc, 0, 0, 0);
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, b, acc, 0, 0, 0);
  }
  // Transposed PV product: D[c][i] += sum_j S^T[c][j] P[j][i] with P from the
  // QK-type accumulator layout (lane <-> resident index i = l%16, streamed j) and
  // S^T from an LDS array stored [c][j]; the result keeps lane <-> i, so
  // per-resident-row scalars need no lane exchange.  st_row: row (c0 + l%16) at j0.
  __device__ static __forceinline__ f32x4 pvt(const f32x4& p0, const f32x4& p1, const bf16* st_row, int lane,
                                              f32x4 acc) {
    const int g = lane >> 4;
    bf16x8 a, b;
    b[0] = (bf16)p0[0]; b[1] = (bf16)p0[1]; b[2] = (bf16)p0[2]; b[3] = (bf16)p0[3];
    b[4] = (bf16)p1[0]; b[5] = (bf16)p1[1]; b[6] = (bf16)p1[2]; b[7] = (bf16)p1[3];
    const bf16x4 lo = *reinterpret_cast<const bf16x4*>(st_row + 4 * g);
    const bf16x4 hi = *reinterpret_cast<const bf16x4*>(st_row + 16 + 4 * g);
    a[0] = lo[0]; a[1] = lo[1]; a[2] = lo[2]; a[3] = lo[3];
    a[4] = hi[0]; a[5] = hi[1]; a[6] = hi[2]; a[7] = hi[3];
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc, 0, 0, 0);
  }
  static constexpr bool SPLIT = true;
};

template <int DP> struct Mfma<float, DP> {
  static_assert(DP % 4 == 0, "fp32 head dim must be padded to 4");
  static constexpr int KSTEPS = DP / 4;
  static constexpr int RUN = DP / 4;
  struct Frag { float v[KSTEPS]; };
  __device__ static __forceinline__ void load(Frag& f, const float* row_base, int lane) {
    const float* p = row_base + (lane >> 4) * RUN;
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) f.v[s] = p[s];
  }
  __device__ static __forceinline__ void from_run(Frag& f, const float* run) {
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) f.v[s] = run[s];
  }
  __device__ static __forceinline__ f32x4 qk(const Frag& a, const Frag& b, f32x4 c) {
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) c = __builtin_amdgcn_mfma_f32_16x16x4f32(a.v[s], b.v[s], c, 0, 0, 0);
    return c;
  }
  __device__ static __forceinline__ f32x4 pv(const f32x4& p0, const f32x4& p1, const float* vt_row, int lane,
                                             f32x4 acc) {
    const int g = lane >> 4;
    const f32x4 lo = *reinterpret_cast<const f32x4*>(vt_row + 4 * g);
    const f32x4 hi = *reinterpret_cast<const f32x4*>(vt_row + 16 + 4 * g);
#pragma unroll
    for (int r = 0; r < 4; ++r) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(p0[r], lo[r], acc, 0, 0, 0);
#pragma unroll
    for (int r = 0; r < 4; ++r) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(p1[r], hi[r], acc, 0, 0, 0);
    return acc;
  }
  __device__ static __forceinline__ f32x4 pv_split(const f32x4& p0, const f32x4& p1, const float* vt_row, int lane,
                                                   f32x4 acc) {
    return pv(p0, p1, vt_row, lane, acc);
  }
  __device__ static __forceinline__ f32x4 pvt(const f32x4& p0, const f32x4& p1, const float* st_row, int lane,
                                              f32x4 acc) {
    const int g = lane >> 4;
    const f32x4 lo = *reinterpret_cast<const f32x4*>(st_row + 4 * g);
    const f32x4 hi = *reinterpret_cast<const f32x4*>(st_row + 16 + 4 * g);
#pragma unroll
    for (int r = 0; r < 4; ++r) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(lo[r], p0[r], acc, 0, 0, 0);
#pragma unroll
    for (int r = 0; r < 4; ++r) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(hi[r], p1[r], acc, 0, 0, 0);
    return acc;
  }
  static constexpr bool SPLIT = false;  // fp32 operands are exact already
};

// ---------------------------------------------------------------------------
// Lane reductions across the 4 lane groups (l/16) of a wave that hold the same
// accumulator column.  gfx950's v_permlane16/32_swap exchange 16-lane rows inside
// the VALU: with x as both operands, the two results hold x[l] and x[l ^ 16]
// (resp. x[l ^ 32]) in some order, so their sum / max is the pair reduction with
// no LDS round trip (a __shfl_xor compiles to ds_bpermute).
__device__ __forceinline__ float xor16_pair(float x, bool mx) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  const float a = __uint_as_float(r[0]), b = __uint_as_float(r[1]);
  return mx ? fmaxf(a, b) : a + b;
}
__device__ __forceinline__ float xor32_pair(float x, bool mx) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  const float a = __uint_as_float(r[0]), b = __uint_as_float(r[1]);
  return mx ? fmaxf(a, b) : a + b;
}
__device__ __forceinline__ float sum_groups(float x) { return xor32_pair(xor16_pair(x, false), false); }
// Sum over the 64 lanes of a wave, in every lane (DPP within 16-lane rows, then the
// row swaps); a fixed order, so equal inputs give bit-equal sums in every wave.
__device__ __forceinline__ float wave_sum(float x) {
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0xb1, 0xf, 0xf, false));   // quad_perm 1,0,3,2
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x4e, 0xf, 0xf, false));   // quad_perm 2,3,0,1
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x141, 0xf, 0xf, false));  // row_half_mirror
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x140, 0xf, 0xf, false));  // row_mirror
  return sum_groups(x);
}
__device__ __forceinline__ float max_groups(float x) { return xor32_pair(xor16_pair(x, true), true); }

// Unsigned maximum over the 64 lanes of a wave; every lane must be active.
// Four DPP steps reduce each 16-lane row, four readlanes combine the rows.  (An
// atomicMax on one LDS word from every lane compiles to a 64-step readlane loop
// per wave, which measured ~2 us for a 512-thread block.)
__device__ __forceinline__ unsigned wave_max_u32(unsigned x) {
  x = max(x, (unsigned)__builtin_amdgcn_update_dpp(0, (int)x, 0xb1, 0xf, 0xf, false));   // quad_perm 1,0,3,2
  x = max(x, (unsigned)__builtin_amdgcn_update_dpp(0, (int)x, 0x4e, 0xf, 0xf, false));   // quad_perm 2,3,0,1
  x = max(x, (unsigned)__builtin_amdgcn_update_dpp(0, (int)x, 0x141, 0xf, 0xf, false));  // row_half_mirror
  x = max(x, (unsigned)__builtin_amdgcn_update_dpp(0, (int)x, 0x140, 0xf, 0xf, false));  // row_mirror
  const unsigned r0 = __builtin_amdgcn_readlane(x, 0), r1 = __builtin_amdgcn_readlane(x, 16);
  const unsigned r2 = __builtin_amdgcn_readlane(x, 32), r3 = __builtin_amdgcn_readlane(x, 48);
  return max(max(r0, r1), max(r2, r3));
}

// *s = max(*s, x) over the whole block (LDS word); one atomic per wave.
// Called by every thread of the block (full waves).
__device__ __forceinline__ void block_atomic_max_u32(unsigned* s, unsigned x) {
  const unsigned w = wave_max_u32(x);
  if ((threadIdx.x & (WAVE - 1)) == 0) atomicMax(s, w);
}

// s + sum_{k < n} p[k * stride] in the order k = 0, 1, ...: loads in batches of 8 in
// flight, then the adds (the order of a plain loop, without one memory latency per term).
__device__ __forceinline__ float ordered_sum(const float* p, size_t stride, int n, float s) {
  for (int k0 = 0; k0 < n; k0 += 8) {
    float v[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = k0 + k < n ? p[(size_t)(k0 + k) * stride] : 0.f;
#pragma unroll
    for (int k = 0; k < 8; ++k)
      if (k0 + k < n) s += v[k];
  }
  return s;
}

// ---------------------------------------------------------------------------
// Error flag and tagged exchange.
constexpr uint32_t SPIN_LIMIT = 1u << 22;  // ~2-4 s of polling

// Where a kernel reports an expired wait: the workspace's error word, which holds
// (salt << 12) | code for the call that raised it (a word carrying another call's
// salt is stale and ignored), and, when the library has one, a word of pinned,
// device-mapped host memory that the host reads at its next call without a
// synchronisation (only a kernel that gives up writes it).
struct ErrRef {
  uint32_t* ws;         // workspace error word (word 1 of the header holds the latest salt)
  uint32_t* host;       // mapped host mailbox, or null
  uint32_t spin_limit;  // polls before a wait gives up: SPIN_LIMIT, lowered only by tests
                        // of the failure path (dfl_debug_set_spin_limit)
};
__device__ __forceinline__ void raise_error(ErrRef err, uint32_t salt, uint32_t code) {
  const uint32_t w = (salt << 12) | (code & 0xfffu);
  __hip_atomic_store(err.ws, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (err.host) __hip_atomic_store(err.host, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ bool error_raised(ErrRef err, uint32_t salt) {
  const uint32_t e = __hip_atomic_load(err.ws, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return (e >> 12) == salt && (e & 0xfffu) != 0u;
}

__device__ __forceinline__ void xch_put(uint64_t* word, float v, uint32_t tag) {
  const uint64_t w = ((uint64_t)__float_as_uint(v) << 32) | (uint64_t)tag;
  __hip_atomic_store(word, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Publishing for a group whose members all run on one XCD: a plain store lands in
// that XCD's L2, where the members' agent-scope polls read it, without the
// write-through to memory of an agent-scope store (one exchange round measured
// 0.98 us instead of 1.43 us on MI355X).  A store of this kind is not visible to
// polls from another XCD, so it is used only after every member of the group has
// confirmed its placement (xcc_placed, group_placement).
// One aligned 64-bit vector store with no cache-scope bits (a workgroup-scope
// atomic store would carry sc0), so value and tag stay one single-copy-atomic word.
__device__ __forceinline__ void xch_put_local(uint64_t* word, float v, uint32_t tag) {
  const uint64_t w = ((uint64_t)__float_as_uint(v) << 32) | (uint64_t)tag;
  asm volatile("global_store_dwordx2 %0, %1, off" ::"v"(word), "v"(w) : "memory");
}
__device__ __forceinline__ void xch_put(uint64_t* word, float v, uint32_t tag, bool local) {
  if (local) xch_put_local(word, v, tag);
  else xch_put(word, v, tag);
}

// Workgroup barrier that orders LDS accesses only: it waits for the thread's LDS
// operations (lgkmcnt) but not for its global stores, as __syncthreads() does.
// Used where a barrier follows the publishing of exchange words, whose
// completion no thread of the workgroup waits for; never where threads of the
// workgroup pass data through global memory.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// True when this workgroup runs on the XCD that the round-robin dispatch order
// assigns to it (workgroup id mod 8), read from the hardware XCC id register.
__device__ __forceinline__ bool xcc_placed() {
  unsigned v;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
  return (v & 0xfu) == (blockIdx.x & 7u);
}

}  // namespace dfl
