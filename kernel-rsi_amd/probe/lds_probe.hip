// LDS probes for hw.py, built into libkrsi_probe.so beside the streaming probe (not part of the
// kernel library). They measure what the attention kernels' LDS traffic costs on gfx950:
//
// * krsi_probe_lds_rate: bytes per clock per CU of one LDS access form. One workgroup per CU
//   (96 KB of LDS each), `threads` threads; every wave issues 8 independent accesses, waits for
//   them (s_waitcnt lgkmcnt(0)), folds the results, and repeats `iters` times. Wave 0 of each
//   workgroup times its loop with s_memtime; the caller divides bytes by the mean cycles.
// * krsi_probe_lds_banks: one wave per pattern reads 128 bits per lane from LDS at the byte
//   addresses a pattern gives (8 reads per iteration, `iters` iterations), so that a counter
//   run (rocprofv3 --pmc SQ_LDS_BANK_CONFLICT SQ_INSTS_LDS) reads each pattern's conflict
//   cycles per instruction from its own dispatch.
//
// The accesses are inline asm, so each form is exactly the instruction named; every address
// stays inside the workgroup's LDS (checked on the host for the bank patterns).
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kLdsBytes = 96 * 1024;  // > 80 KB: one workgroup per CU

#define KRSI_LDS8(INS, OFFS)                                                                     \
  INS " %0, %8 offset:0\n " INS " %1, %8 offset:4096\n " INS " %2, %8 offset:8192\n " INS          \
      " %3, %8 offset:12288\n " INS " %4, %8 offset:16384\n " INS " %5, %8 offset:20480\n " INS    \
      " %6, %8 offset:24576\n " INS " %7, %8 offset:28672\n s_waitcnt lgkmcnt(0)"

// Forms: 0 ds_read_b128, 1 ds_read_b64, 2 ds_read_b64_tr_b16, 3 ds_read_b32, 4 ds_write_b32,
// 5 ds_write_b64, 6 ds_write_b128, 7 ds_add_f32 (no return), 8 ds_read_b128 with every lane of
// a half-wave on one address (broadcast).
template <int FORM>
__device__ __forceinline__ uint32_t lds8(uint32_t a) {
  if constexpr (FORM == 0 || FORM == 8) {
    u32x4 x0, x1, x2, x3, x4, x5, x6, x7;
    asm volatile(KRSI_LDS8("ds_read_b128", 0)
                 : "=v"(x0), "=v"(x1), "=v"(x2), "=v"(x3), "=v"(x4), "=v"(x5), "=v"(x6), "=v"(x7)
                 : "v"(a)
                 : "memory");
    return x0.x ^ x1.y ^ x2.z ^ x3.w ^ x4.x ^ x5.y ^ x6.z ^ x7.w;
  } else if constexpr (FORM == 1 || FORM == 2) {
    u32x2 x0, x1, x2, x3, x4, x5, x6, x7;
    if constexpr (FORM == 1)
      asm volatile(KRSI_LDS8("ds_read_b64", 0)
                   : "=v"(x0), "=v"(x1), "=v"(x2), "=v"(x3), "=v"(x4), "=v"(x5), "=v"(x6), "=v"(x7)
                   : "v"(a)
                   : "memory");
    else
      asm volatile(KRSI_LDS8("ds_read_b64_tr_b16", 0)
                   : "=v"(x0), "=v"(x1), "=v"(x2), "=v"(x3), "=v"(x4), "=v"(x5), "=v"(x6), "=v"(x7)
                   : "v"(a)
                   : "memory");
    return x0.x ^ x1.y ^ x2.x ^ x3.y ^ x4.x ^ x5.y ^ x6.x ^ x7.y;
  } else if constexpr (FORM == 3) {
    uint32_t x0, x1, x2, x3, x4, x5, x6, x7;
    asm volatile(KRSI_LDS8("ds_read_b32", 0)
                 : "=v"(x0), "=v"(x1), "=v"(x2), "=v"(x3), "=v"(x4), "=v"(x5), "=v"(x6), "=v"(x7)
                 : "v"(a)
                 : "memory");
    return x0 ^ x1 ^ x2 ^ x3 ^ x4 ^ x5 ^ x6 ^ x7;
  } else if constexpr (FORM == 4) {
    asm volatile(
        "ds_write_b32 %0, %1 offset:0\n ds_write_b32 %0, %1 offset:4096\n ds_write_b32 %0, %1 offset:8192\n"
        " ds_write_b32 %0, %1 offset:12288\n ds_write_b32 %0, %1 offset:16384\n ds_write_b32 %0, %1 offset:20480\n"
        " ds_write_b32 %0, %1 offset:24576\n ds_write_b32 %0, %1 offset:28672\n s_waitcnt lgkmcnt(0)" ::"v"(a),
        "v"(a)
        : "memory");
    return a;
  } else if constexpr (FORM == 5) {
    const u32x2 v = {a, a + 1};
    asm volatile(
        "ds_write_b64 %0, %1 offset:0\n ds_write_b64 %0, %1 offset:4096\n ds_write_b64 %0, %1 offset:8192\n"
        " ds_write_b64 %0, %1 offset:12288\n ds_write_b64 %0, %1 offset:16384\n ds_write_b64 %0, %1 offset:20480\n"
        " ds_write_b64 %0, %1 offset:24576\n ds_write_b64 %0, %1 offset:28672\n s_waitcnt lgkmcnt(0)" ::"v"(a),
        "v"(v)
        : "memory");
    return a;
  } else if constexpr (FORM == 6) {
    const u32x4 v = {a, a + 1, a + 2, a + 3};
    asm volatile(
        "ds_write_b128 %0, %1 offset:0\n ds_write_b128 %0, %1 offset:4096\n ds_write_b128 %0, %1 offset:8192\n"
        " ds_write_b128 %0, %1 offset:12288\n ds_write_b128 %0, %1 offset:16384\n ds_write_b128 %0, %1 offset:20480\n"
        " ds_write_b128 %0, %1 offset:24576\n ds_write_b128 %0, %1 offset:28672\n s_waitcnt lgkmcnt(0)" ::"v"(a),
        "v"(v)
        : "memory");
    return a;
  } else {  // FORM 7
    const float v = 1.0f;
    asm volatile(
        "ds_add_f32 %0, %1 offset:0\n ds_add_f32 %0, %1 offset:4096\n ds_add_f32 %0, %1 offset:8192\n"
        " ds_add_f32 %0, %1 offset:12288\n ds_add_f32 %0, %1 offset:16384\n ds_add_f32 %0, %1 offset:20480\n"
        " ds_add_f32 %0, %1 offset:24576\n ds_add_f32 %0, %1 offset:28672\n s_waitcnt lgkmcnt(0)" ::"v"(a),
        "v"(v)
        : "memory");
    return a;
  }
}

constexpr int form_bytes(int form) {
  return form == 0 || form == 6 || form == 8 ? 16 : form == 1 || form == 2 || form == 5 ? 8 : 4;
}

// Byte offset of a lane's access: distinct consecutive chunks (conflict-free), the transposed
// read's pattern over a 64-column bf16 tile with the attention kernels' chunk swizzle, or one
// address per half-wave. Waves sharing a SIMD start 1 KB apart. Largest offset: 4 KB + the
// 28 KB immediate + 16 bytes, inside the 96 KB.
template <int FORM>
__device__ __forceinline__ uint32_t lane_offset(int lane, int wave) {
  const int g = lane >> 5;
  uint32_t off;
  if constexpr (FORM == 2) {
    const int s = lane & 15, r = 4 * g + (s >> 2), j = 2 * ((lane >> 4) & 1) + ((s & 3) >> 1);
    const int sw = (((r >> 1) & 1) << 2) | ((r >> 2) & 3);
    off = (uint32_t)(r * 64 + 8 * (j ^ sw) + 4 * (s & 1)) * 2u;
  } else if constexpr (FORM == 8) {
    off = (uint32_t)g * 16u;
  } else {
    off = (uint32_t)(lane * form_bytes(FORM));
  }
  return off + (uint32_t)(wave & 3) * 1024u;
}

template <int FORM>
__global__ __launch_bounds__(1024) void lds_rate_kernel(int iters, uint32_t* __restrict__ sink,
                                                        unsigned long long* __restrict__ cycles) {
  __shared__ __attribute__((aligned(256))) unsigned char lds[kLdsBytes];
  for (int i = threadIdx.x; i < kLdsBytes / 4; i += blockDim.x)
    reinterpret_cast<uint32_t*>(lds)[i] = (uint32_t)i * 2654435761u;
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t a =
      (uint32_t)(uintptr_t)(__attribute__((address_space(3))) unsigned char*)lds + lane_offset<FORM>(lane, wave);
  uint32_t acc = 0;
  const unsigned long long t0 = __builtin_amdgcn_s_memtime();
  for (int it = 0; it < iters; ++it) acc ^= lds8<FORM>(a);
  __syncthreads();
  const unsigned long long t1 = __builtin_amdgcn_s_memtime();
  if (threadIdx.x == 0) cycles[blockIdx.x] = t1 - t0;
  sink[(size_t)blockIdx.x * blockDim.x + threadIdx.x] = acc;
}

__global__ __launch_bounds__(64) void lds_bank_kernel(const uint32_t* __restrict__ addr, int iters,
                                                      uint32_t* __restrict__ sink) {
  __shared__ __attribute__((aligned(256))) unsigned char lds[32768];
  for (int i = threadIdx.x; i < 8192; i += 64) reinterpret_cast<uint32_t*>(lds)[i] = (uint32_t)i;
  __syncthreads();
  const uint32_t a = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) unsigned char*)lds + addr[threadIdx.x];
  uint32_t acc = 0;
  for (int it = 0; it < iters; ++it) {
    u32x4 x0, x1, x2, x3, x4, x5, x6, x7;
    asm volatile(
        "ds_read_b128 %0, %8 offset:0\n ds_read_b128 %1, %8 offset:0\n ds_read_b128 %2, %8 offset:0\n"
        " ds_read_b128 %3, %8 offset:0\n ds_read_b128 %4, %8 offset:0\n ds_read_b128 %5, %8 offset:0\n"
        " ds_read_b128 %6, %8 offset:0\n ds_read_b128 %7, %8 offset:0\n s_waitcnt lgkmcnt(0)"
        : "=v"(x0), "=v"(x1), "=v"(x2), "=v"(x3), "=v"(x4), "=v"(x5), "=v"(x6), "=v"(x7)
        : "v"(a)
        : "memory");
    acc ^= x0.x ^ x1.y ^ x2.z ^ x3.w ^ x4.x ^ x5.y ^ x6.z ^ x7.w;
  }
  sink[threadIdx.x] = acc;
}

template <int FORM>
void launch_rate(int ncu, int threads, int iters, uint32_t* sink, unsigned long long* cycles, hipStream_t st) {
  hipLaunchKernelGGL(lds_rate_kernel<FORM>, dim3(ncu), dim3(threads), 0, st, iters, sink, cycles);
}

}  // namespace

extern "C" {

// Bytes one workgroup moves per wave instruction of `form` (64 lanes), for the caller's rate.
int krsi_probe_lds_form_bytes(int form) { return form < 0 || form > 8 ? 0 : 64 * form_bytes(form); }

// Runs `ncu` workgroups of `threads` threads (64..1024, a multiple of 64), `iters` iterations of
// 8 accesses of `form` per wave; cycles[ncu] receives each workgroup's s_memtime cycles; sink
// holds ncu * threads words. Returns 0, or -1 on a bad argument or a launch error.
int krsi_probe_lds_rate(int form, int ncu, int threads, int iters, void* sink, void* cycles, void* stream) {
  if (ncu <= 0 || threads < 64 || threads > 1024 || threads % 64 || iters <= 0 || !sink || !cycles) return -1;
  hipStream_t st = static_cast<hipStream_t>(stream);
  uint32_t* s = static_cast<uint32_t*>(sink);
  unsigned long long* c = static_cast<unsigned long long*>(cycles);
  switch (form) {
    case 0: launch_rate<0>(ncu, threads, iters, s, c, st); break;
    case 1: launch_rate<1>(ncu, threads, iters, s, c, st); break;
    case 2: launch_rate<2>(ncu, threads, iters, s, c, st); break;
    case 3: launch_rate<3>(ncu, threads, iters, s, c, st); break;
    case 4: launch_rate<4>(ncu, threads, iters, s, c, st); break;
    case 5: launch_rate<5>(ncu, threads, iters, s, c, st); break;
    case 6: launch_rate<6>(ncu, threads, iters, s, c, st); break;
    case 7: launch_rate<7>(ncu, threads, iters, s, c, st); break;
    case 8: launch_rate<8>(ncu, threads, iters, s, c, st); break;
    default: return -1;
  }
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

// One launch of one wave per pattern: addr_dev holds npat x 64 byte offsets (multiples of 16,
// below 32768 - 16), sink 64 words. Returns 0, or -1 on a launch error.
int krsi_probe_lds_banks(const void* addr_dev, int npat, int iters, void* sink, void* stream) {
  if (!addr_dev || npat <= 0 || iters <= 0 || !sink) return -1;
  hipStream_t st = static_cast<hipStream_t>(stream);
  for (int k = 0; k < npat; ++k)
    hipLaunchKernelGGL(lds_bank_kernel, dim3(1), dim3(64), 0, st, static_cast<const uint32_t*>(addr_dev) + 64 * k,
                       iters, static_cast<uint32_t*>(sink));
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // extern "C"
