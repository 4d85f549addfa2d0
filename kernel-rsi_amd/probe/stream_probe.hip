// Streaming-bandwidth probe for hw.py: the HBM rate a plain streaming kernel reaches at a
// given mix of read and written bytes on this GPU. These are the achievable ceilings that the
// bandwidth-bound kernels (RMSNorm, GEGLU) are compared with, beside the 8 TB/s published peak.
// This is not part of the kernel library; it is built into its own libkrsi_probe.so.
//
// out_w[i] = sum_r in_r[i] (+ w) over n 16-byte chunks per array: 128-bit loads and stores,
// a grid-stride loop with `unroll` chunks in flight per thread, optional non-temporal
// stores. Every index is below n by construction.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <bool NT>
__device__ __forceinline__ void put(u32x4* p, u32x4 v) {
  if (NT)
    __builtin_nontemporal_store(v, p);
  else
    *p = v;
}

template <int R, int W, int UNR, bool NT>
__global__ __launch_bounds__(256) void stream_kernel(const u32x4* __restrict__ a0, const u32x4* __restrict__ a1,
                                                     const u32x4* __restrict__ a2, u32x4* __restrict__ o0,
                                                     u32x4* __restrict__ o1, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  for (; i + (UNR - 1) * stride < n; i += UNR * stride) {
    u32x4 v[UNR];
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      u32x4 t = {(uint32_t)u, 1u, 2u, 3u};
      if (R > 0) t = a0[i + u * stride];
      if (R > 1) t += a1[i + u * stride];
      if (R > 2) t += a2[i + u * stride];
      v[u] = t;
    }
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      if (W > 0) put<NT>(o0 + i + u * stride, v[u]);
      if (W > 1) put<NT>(o1 + i + u * stride, v[u] + 1u);
      // Read-only mixes: a store no input can trigger keeps the loads alive.
      if (W == 0 && v[u][0] == 0x9e3779b9u && v[u][1] == 0x7f4a7c15u) o0[0] = v[u];
    }
  }
  for (; i < n; i += stride) {
    u32x4 t = {0u, 1u, 2u, 3u};
    if (R > 0) t = a0[i];
    if (R > 1) t += a1[i];
    if (R > 2) t += a2[i];
    if (W > 0) o0[i] = t;
    if (W > 1) o1[i] = t + 1u;
    if (W == 0 && t[0] == 0x9e3779b9u && t[1] == 0x7f4a7c15u) o0[0] = t;
  }
}

template <int R, int W>
int launch(int unroll, int nt, int blocks, const void* const* in, void* const* out, int64_t n, hipStream_t st) {
  const u32x4* a0 = (const u32x4*)in[0];
  const u32x4* a1 = R > 1 ? (const u32x4*)in[1] : nullptr;
  const u32x4* a2 = R > 2 ? (const u32x4*)in[2] : nullptr;
  u32x4* o0 = (u32x4*)out[0];
  u32x4* o1 = W > 1 ? (u32x4*)out[1] : nullptr;
#define KRSI_PROBE_CASE(U)                                                                                      \
  if (unroll == U) {                                                                                            \
    if (nt)                                                                                                     \
      hipLaunchKernelGGL((stream_kernel<R, W, U, true>), dim3(blocks), dim3(256), 0, st, a0, a1, a2, o0, o1, n);  \
    else                                                                                                        \
      hipLaunchKernelGGL((stream_kernel<R, W, U, false>), dim3(blocks), dim3(256), 0, st, a0, a1, a2, o0, o1, n); \
    return hipGetLastError() == hipSuccess ? 0 : 2;                                                             \
  }
  KRSI_PROBE_CASE(1) KRSI_PROBE_CASE(2) KRSI_PROBE_CASE(4) KRSI_PROBE_CASE(8)
#undef KRSI_PROBE_CASE
  return 1;
}

}  // namespace

extern "C" {

// reads in 1..3 and writes in 0..2 (reads + writes >= 1; a read-only mix still needs out[0]);
// in[0..reads-1] and out[0..max(writes,1)-1] hold n 16-byte chunks each. Returns 0, 1 for an
// unsupported mix or unroll (nothing launched), 2 if the launch was rejected.
int krsi_probe_stream(int reads, int writes, int unroll, int nontemporal, int blocks, const void* const* in,
                      void* const* out, int64_t n, void* stream) {
  if (n <= 0 || blocks <= 0 || !in || !out) return 1;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (reads == 1 && writes == 0) return launch<1, 0>(unroll, nontemporal, blocks, in, out, n, st);
  if (reads == 2 && writes == 0) return launch<2, 0>(unroll, nontemporal, blocks, in, out, n, st);
  if (reads == 1 && writes == 1) return launch<1, 1>(unroll, nontemporal, blocks, in, out, n, st);
  if (reads == 2 && writes == 1) return launch<2, 1>(unroll, nontemporal, blocks, in, out, n, st);
  if (reads == 3 && writes == 1) return launch<3, 1>(unroll, nontemporal, blocks, in, out, n, st);
  if (reads == 3 && writes == 2) return launch<3, 2>(unroll, nontemporal, blocks, in, out, n, st);
  if (reads == 0 && writes == 1) {
    // Write-only: the kernel's R = 0 path stores a constant pattern.
    u32x4* o0 = (u32x4*)out[0];
#define KRSI_PROBE_W(U)                                                                                           \
  if (unroll == U) {                                                                                              \
    if (nontemporal)                                                                                              \
      hipLaunchKernelGGL((stream_kernel<0, 1, U, true>), dim3(blocks), dim3(256), 0, st, nullptr, nullptr,       \
                         nullptr, o0, nullptr, n);                                                                \
    else                                                                                                          \
      hipLaunchKernelGGL((stream_kernel<0, 1, U, false>), dim3(blocks), dim3(256), 0, st, nullptr, nullptr,      \
                         nullptr, o0, nullptr, n);                                                                \
    return hipGetLastError() == hipSuccess ? 0 : 2;                                                               \
  }
    KRSI_PROBE_W(1) KRSI_PROBE_W(2) KRSI_PROBE_W(4) KRSI_PROBE_W(8)
#undef KRSI_PROBE_W
    return 1;
  }
  return 1;
}

}  // extern "C"
