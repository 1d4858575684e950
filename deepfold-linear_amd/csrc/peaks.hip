// Issue-rate and exchange probes behind the forward's roofline figures (a separate
// library, libdfl_peaks.so, loaded only by bench.py --workload peaks; nothing in the
// product calls it).  Every probe runs one 512-thread workgroup per CU (the dynamic
// LDS request keeps a second one off the CU), i.e. two waves per SIMD as in the
// Sinkhorn kernels, on `blocks` workgroups.
//   mode 0  exp2:  24 independent chains x = exp2(-x) per thread (v_exp_f32)
//   mode 1  fma:   24 independent chains y = y * a + 0.25 (v_fma_f32)
//   mode 2  mfma:  6 independent v_mfma_f32_16x16x32_bf16 accumulators per wave
//   mode 3  sweep: the fixed-shift sweep's per-element mix, s += exp2(x * a + w)
//   mode 4  exchange: groups of 16 workgroups on one XCD (workgroup id % 8 = XCD),
//           each member publishes 48 tagged 64-bit words per round and polls the
//           group's 768 words with the Sinkhorn kernels' poll (poll_vector)
// Rates are taken from HIP events around the launch; clk is clock64() of workgroup 0
// between the probe's first and last round.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "sinkhorn_engine.h"

namespace dfl {
namespace {

constexpr int PNT = 512;
constexpr int PROBE_LDS = 96 * 1024;

template <int MODE>
__global__ void __launch_bounds__(PNT) peak_kernel(float* out, int iters, float a, long long* clk) {
  const int lane = threadIdx.x & 63;
  float x[24], s[24];
#pragma unroll
  for (int k = 0; k < 24; ++k) {
    x[k] = 1e-3f * (float)(threadIdx.x + k);
    s[k] = 0.f;
  }
  bf16x8 A, B;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    A[e] = (bf16)(1e-2f * (float)(lane + e));
    B[e] = (bf16)(2e-2f * (float)e);
  }
  f32x4 c[6];
#pragma unroll
  for (int k = 0; k < 6; ++k) c[k] = f32x4{0.f, 0.f, 0.f, 0.f};
  const long long t0 = clock64();
  for (int it = 0; it < iters; ++it) {
    if constexpr (MODE == 0) {
#pragma unroll
      for (int k = 0; k < 24; ++k) x[k] = __builtin_amdgcn_exp2f(-x[k]);
    } else if constexpr (MODE == 1) {
#pragma unroll
      for (int k = 0; k < 24; ++k) x[k] = __builtin_fmaf(x[k], a, 0.25f);
    } else if constexpr (MODE == 2) {
#pragma unroll
      for (int k = 0; k < 6; ++k) c[k] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, B, c[k], 0, 0, 0);
    } else {
      // a slowly varying scale keeps the exponentials inside the loop; x stays fixed
      // and small, s grows linearly
      const float ai = a + (float)it * 1e-7f;
#pragma unroll
      for (int k = 0; k < 24; ++k) s[k] += __builtin_amdgcn_exp2f(__builtin_fmaf(x[k], ai, -0.5f));
    }
  }
  const long long t1 = clock64();
  float r = 0.f;
#pragma unroll
  for (int k = 0; k < 24; ++k) r += x[k] + s[k];
#pragma unroll
  for (int k = 0; k < 6; ++k) r += c[k][0] + c[k][1] + c[k][2] + c[k][3];
  out[(size_t)blockIdx.x * PNT + threadIdx.x] = r;
  if (blockIdx.x == 0 && threadIdx.x == 0) *clk = t1 - t0;
}

constexpr int XG = 16, XNP = 768, XPER = XNP / XG;

// buf: 2 (round parity) x groups x XNP words, zero or older-salt words on entry.
__global__ void __launch_bounds__(PNT) peak_exchange(uint64_t* buf, uint32_t* errw, int groups, int rounds,
                                                     uint32_t salt, float* out, long long* clk) {
  __shared__ int s_flag;
  int grp, member;
  if (!group_of(groups, XG, grp, member)) return;
  if (threadIdx.x == 0) s_flag = 0;
  __syncthreads();
  const ErrRef err{errw, nullptr, SPIN_LIMIT};
  const bool local = xcc_placed();
  float acc = 0.f;
  const long long t0 = clock64();
  for (int r = 0; r < rounds; ++r) {
    const uint32_t tag = (salt << 12) | (uint32_t)(r + 1);
    uint64_t* words = buf + ((size_t)(r & 1) * groups + grp) * XNP;
    if (threadIdx.x < XPER) xch_put(words + member * XPER + threadIdx.x, (float)(r + threadIdx.x), tag, local);
    const bool ok = poll_vector<PNT>(words, XNP, tag, err, [&](int off, uint64_t w) {
      acc += __uint_as_float((uint32_t)(w >> 32));
    });
    if (!ok) s_flag = 1;
    __syncthreads();
    if (s_flag) break;
  }
  const long long t1 = clock64();
  out[(size_t)blockIdx.x * PNT + threadIdx.x] = acc;
  if (blockIdx.x == 0 && threadIdx.x == 0) *clk = t1 - t0;
}

template <typename K>
hipError_t lds_limit(K kern) {
  return hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, PROBE_LDS);
}

}  // namespace
}  // namespace dfl

// mode 0..3: issue-rate probes on `blocks` workgroups for `iters` iterations;
// mode 4: exchange probe, `blocks` = 16 * groups workgroups (groups <= 16 and a
// multiple of 8, one group per XCD slot), `iters` rounds (<= 4000).
// Writes the launch's event time (ms) and workgroup 0's clock64() span; returns a
// hipError_t, or 1000 + 2 if an exchange wait expired.
extern "C" int dfl_peak_run(int mode, int blocks, int iters, float* out_ms, long long* out_clk) {
  using namespace dfl;
  if (blocks <= 0 || iters <= 0 || mode < 0 || mode > 4) return (int)hipErrorInvalidValue;
  if (mode == 4 && (blocks % (8 * XG) != 0 || blocks / XG > 16 || iters > 4000)) return (int)hipErrorInvalidValue;
  float* out = nullptr;
  long long* clk = nullptr;
  uint64_t* buf = nullptr;
  uint32_t* errw = nullptr;
  const int groups = blocks / XG;
  hipError_t e = hipMalloc(&out, (size_t)blocks * PNT * sizeof(float));
  if (e == hipSuccess) e = hipMalloc(&clk, sizeof(long long));
  if (e == hipSuccess && mode == 4) e = hipMalloc(&buf, 2 * (size_t)groups * XNP * sizeof(uint64_t));
  if (e == hipSuccess && mode == 4) e = hipMalloc(&errw, sizeof(uint32_t));
  if (e == hipSuccess && mode == 4) e = hipMemset(buf, 0, 2 * (size_t)groups * XNP * sizeof(uint64_t));
  if (e == hipSuccess && mode == 4) e = hipMemset(errw, 0, sizeof(uint32_t));
  hipEvent_t a = nullptr, b = nullptr;
  if (e == hipSuccess) e = hipEventCreate(&a);
  if (e == hipSuccess) e = hipEventCreate(&b);
  if (e == hipSuccess) {
    switch (mode) {
      case 0: e = lds_limit(peak_kernel<0>); break;
      case 1: e = lds_limit(peak_kernel<1>); break;
      case 2: e = lds_limit(peak_kernel<2>); break;
      case 3: e = lds_limit(peak_kernel<3>); break;
      default: e = lds_limit(peak_exchange); break;
    }
  }
  if (e == hipSuccess) e = hipEventRecord(a, 0);
  if (e == hipSuccess) {
    const float coef = 0.999f;
    switch (mode) {
      case 0: hipLaunchKernelGGL(peak_kernel<0>, dim3(blocks), dim3(PNT), PROBE_LDS, 0, out, iters, coef, clk); break;
      case 1: hipLaunchKernelGGL(peak_kernel<1>, dim3(blocks), dim3(PNT), PROBE_LDS, 0, out, iters, coef, clk); break;
      case 2: hipLaunchKernelGGL(peak_kernel<2>, dim3(blocks), dim3(PNT), PROBE_LDS, 0, out, iters, coef, clk); break;
      case 3: hipLaunchKernelGGL(peak_kernel<3>, dim3(blocks), dim3(PNT), PROBE_LDS, 0, out, iters, coef, clk); break;
      default: {
        static uint32_t salt = 0;
        salt = (salt % 0xffffeu) + 1u;
        uint32_t s = salt;
        int g = groups, r = iters;
        void* args[] = {&buf, &errw, &g, &r, &s, &out, &clk};
        e = hipLaunchCooperativeKernel((const void*)peak_exchange, dim3(blocks), dim3(PNT), args, PROBE_LDS, 0);
      }
    }
    if (e == hipSuccess) e = hipGetLastError();
  }
  if (e == hipSuccess) e = hipEventRecord(b, 0);
  if (e == hipSuccess) e = hipEventSynchronize(b);
  if (e == hipSuccess) e = hipEventElapsedTime(out_ms, a, b);
  if (e == hipSuccess) e = hipMemcpy(out_clk, clk, sizeof(long long), hipMemcpyDeviceToHost);
  uint32_t ew = 0;
  if (e == hipSuccess && mode == 4) e = hipMemcpy(&ew, errw, sizeof(uint32_t), hipMemcpyDeviceToHost);
  if (a) (void)hipEventDestroy(a);
  if (b) (void)hipEventDestroy(b);
  if (out) (void)hipFree(out);
  if (clk) (void)hipFree(clk);
  if (buf) (void)hipFree(buf);
  if (errw) (void)hipFree(errw);
  if (e != hipSuccess) return (int)e;
  return (ew & 0xfffu) ? 1000 + (int)(ew & 0xfffu) : 0;
}
