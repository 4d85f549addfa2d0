// GEGLU forward and backward for gfx950 on a merged [a | b] GEMM output.
//
// Semantics follow library/geglu.py of the reference (kernel-rsi):
//   _gelu_parts (geglu.py:20-24), tanh form:
//     z = sqrt(2/pi) * (a + 0.044715 a^3);  t = 1 - 2 / (exp(2z) + 1);  gelu = 0.5 a (1 + t)
//   forward  (_geglu_fwd, geglu.py:27-35):  out = bf16(gelu(a)) * b       (bf16 product)
//   backward (_geglu_bwd, geglu.py:38-52):
//     db   = g * bf16(gelu(a))                                            (bf16 product)
//     dgel = float(bf16(g * b))
//     da   = dgel * (0.5 (1 + t) + 0.5 a (1 - t^2) sqrt(2/pi) (1 + 3 * 0.044715 a^2))
// The exact (erf) form, torch.nn.functional.gelu(approximate="none"), is
//   gelu = 0.5 a (1 + erf(a / sqrt 2)),  gelu' = 0.5 (1 + erf(a / sqrt 2)) + a exp(-a^2 / 2) / sqrt(2 pi)
// with the same rounding points. bf16 above stands for the activation dtype T (bf16, fp16
// or fp32: the template parameter DT), which the reference rounds to (b's and g's dtype).
//
// Design (MI355X): pure streaming. Each thread owns one 16-byte chunk of 8
// columns (4 in fp32) of one row: one 128-bit load of a, one of b (and g), one or two
// 128-bit stores; a workgroup covers 2048 contiguous columns of a row, so
// every wave touches whole 1 KiB lines. The grid is 2-D (column tiles x row
// slices) so no per-element division is needed. Non-multiple-of-8 widths or
// unaligned pointers take a scalar element-per-thread path with the same math.
#include "gelu_math.h"
#include "krsi_device.h"
#include "krsi_internal.h"

namespace krsi {
namespace {

constexpr int kThreads = 256;
template <int DT, bool TANH>
__global__ __launch_bounds__(kThreads) void geglu_fwd_vec(const typename Elem<DT>::T* __restrict__ u,
                                                          typename Elem<DT>::T* __restrict__ out,
                                                          int64_t rows, int f) {
  using El = Elem<DT>;
  constexpr int E = El::E;
  const int f8 = f / E;
  const int c = blockIdx.x * kThreads + threadIdx.x;
  if (c >= f8) return;
  for (int64_t r = blockIdx.y; r < rows; r += gridDim.y) {
    const u32x4* ur = reinterpret_cast<const u32x4*>(u + r * 2 * (int64_t)f);
    // u streams in once here: non-temporal loads (cache-cold fwd+bwd at config 3: 89.2 -> 86.1 us
    // with the backward's, 78 % of 8 TB/s).
    const u32x4 av = __builtin_nontemporal_load(&ur[c]), bv = __builtin_nontemporal_load(&ur[f8 + c]);
    float a[E], b[E], o[E];
    El::unpack(av, a);
    El::unpack(bv, b);
#pragma unroll
    for (int j = 0; j < E; ++j) o[j] = El::round(gelu_fwd<TANH>(a[j])) * b[j];
    // Streamed out once: a non-temporal store.
    __builtin_nontemporal_store(El::pack(o), &reinterpret_cast<u32x4*>(out + r * (int64_t)f)[c]);
  }
}

template <int DT, bool TANH>
__global__ __launch_bounds__(kThreads) void geglu_bwd_vec(const typename Elem<DT>::T* __restrict__ g,
                                                          const typename Elem<DT>::T* __restrict__ u,
                                                          typename Elem<DT>::T* __restrict__ du,
                                                          int64_t rows, int f) {
  using El = Elem<DT>;
  constexpr int E = El::E;
  const int f8 = f / E;
  const int c = blockIdx.x * kThreads + threadIdx.x;
  if (c >= f8) return;
  for (int64_t r = blockIdx.y; r < rows; r += gridDim.y) {
    const u32x4* ur = reinterpret_cast<const u32x4*>(u + r * 2 * (int64_t)f);
    // g, a and b stream in once: non-temporal loads. u arrives from HBM here, not from the MALL:
    // between a layer's forward and its backward the rest of the model streams several hundred
    // MB, as the cache-cold protocol of the measurements does.
    const u32x4 av = __builtin_nontemporal_load(&ur[c]), bv = __builtin_nontemporal_load(&ur[f8 + c]);
    const u32x4 gv = __builtin_nontemporal_load(&reinterpret_cast<const u32x4*>(g + r * (int64_t)f)[c]);
    float a[E], b[E], gg[E], da[E], db[E];
    El::unpack(av, a);
    El::unpack(bv, b);
    El::unpack(gv, gg);
#pragma unroll
    for (int j = 0; j < E; ++j) {
      float d;
      const float gel = gelu_fwd_bwd<TANH>(a[j], d);
      db[j] = gg[j] * El::round(gel);
      const float dgel = El::round(gg[j] * b[j]);
      da[j] = dgel * d;
    }
    u32x4* dr = reinterpret_cast<u32x4*>(du + r * 2 * (int64_t)f);
    __builtin_nontemporal_store(El::pack(da), &dr[c]);
    __builtin_nontemporal_store(El::pack(db), &dr[f8 + c]);
  }
}

template <int DT, bool TANH>
__global__ __launch_bounds__(kThreads) void geglu_fwd_scalar(const typename Elem<DT>::T* __restrict__ u,
                                                             typename Elem<DT>::T* __restrict__ out,
                                                             int64_t rows, int f) {
  using El = Elem<DT>;
  const int c = blockIdx.x * kThreads + threadIdx.x;
  if (c >= f) return;
  for (int64_t r = blockIdx.y; r < rows; r += gridDim.y) {
    const typename El::T* ur = u + r * 2 * (int64_t)f;
    const float a = El::load(ur[c]), b = El::load(ur[f + c]);
    out[r * (int64_t)f + c] = El::store(El::round(gelu_fwd<TANH>(a)) * b);
  }
}

template <int DT, bool TANH>
__global__ __launch_bounds__(kThreads) void geglu_bwd_scalar(const typename Elem<DT>::T* __restrict__ g,
                                                             const typename Elem<DT>::T* __restrict__ u,
                                                             typename Elem<DT>::T* __restrict__ du,
                                                             int64_t rows, int f) {
  using El = Elem<DT>;
  const int c = blockIdx.x * kThreads + threadIdx.x;
  if (c >= f) return;
  for (int64_t r = blockIdx.y; r < rows; r += gridDim.y) {
    const typename El::T* ur = u + r * 2 * (int64_t)f;
    const float a = El::load(ur[c]), b = El::load(ur[f + c]);
    const float gg = El::load(g[r * (int64_t)f + c]);
    float d;
    const float gel = gelu_fwd_bwd<TANH>(a, d);
    typename El::T* dr = du + r * 2 * (int64_t)f;
    dr[c] = El::store(El::round(gg * b) * d);
    dr[f + c] = El::store(gg * El::round(gel));
  }
}

// Grid: x = column tiles, y = row slices (<= 65535; rows beyond stride).
dim3 grid_for(int64_t rows, int cols_per_thread_units) {
  const int64_t gx = ceil_div(cols_per_thread_units, kThreads);
  const int64_t gy = rows < 65535 ? rows : 65535;
  return dim3((unsigned)gx, (unsigned)gy);
}

int check(int64_t rows, int32_t f, int32_t approximate, int32_t dtype) {
  if (dtype != kBf16 && dtype != kF16 && dtype != kF32) return KRSI_ERR_UNSUPPORTED;
  if (rows < 0 || f <= 0 || f > (1 << 28)) return KRSI_ERR_BAD_SHAPE;
  if (approximate != 0 && approximate != 1) return KRSI_ERR_UNSUPPORTED;
  return KRSI_OK;
}

template <int DT, bool TANH>
int geglu_fwd(const void* u, void* out, int64_t rows, int f, hipStream_t st) {
  using T = typename Elem<DT>::T;
  constexpr int E = Elem<DT>::E;
  if ((f % E == 0) && aligned16(u) && aligned16(out))
    hipLaunchKernelGGL((geglu_fwd_vec<DT, TANH>), grid_for(rows, f / E), dim3(kThreads), 0, st,
                       (const T*)u, (T*)out, rows, f);
  else
    hipLaunchKernelGGL((geglu_fwd_scalar<DT, TANH>), grid_for(rows, f), dim3(kThreads), 0, st,
                       (const T*)u, (T*)out, rows, f);
  return launch_status();
}

template <int DT, bool TANH>
int geglu_bwd(const void* g, const void* u, void* du, int64_t rows, int f, hipStream_t st) {
  using T = typename Elem<DT>::T;
  constexpr int E = Elem<DT>::E;
  if ((f % E == 0) && aligned16(g) && aligned16(u) && aligned16(du))
    hipLaunchKernelGGL((geglu_bwd_vec<DT, TANH>), grid_for(rows, f / E), dim3(kThreads), 0, st,
                       (const T*)g, (const T*)u, (T*)du, rows, f);
  else
    hipLaunchKernelGGL((geglu_bwd_scalar<DT, TANH>), grid_for(rows, f), dim3(kThreads), 0, st,
                       (const T*)g, (const T*)u, (T*)du, rows, f);
  return launch_status();
}

template <bool TANH>
int geglu_fwd_dt(const void* u, void* out, int64_t rows, int f, int dtype, hipStream_t st) {
  if (dtype == kF16) return geglu_fwd<kF16, TANH>(u, out, rows, f, st);
  if (dtype == kF32) return geglu_fwd<kF32, TANH>(u, out, rows, f, st);
  return geglu_fwd<kBf16, TANH>(u, out, rows, f, st);
}

template <bool TANH>
int geglu_bwd_dt(const void* g, const void* u, void* du, int64_t rows, int f, int dtype,
                 hipStream_t st) {
  if (dtype == kF16) return geglu_bwd<kF16, TANH>(g, u, du, rows, f, st);
  if (dtype == kF32) return geglu_bwd<kF32, TANH>(g, u, du, rows, f, st);
  return geglu_bwd<kBf16, TANH>(g, u, du, rows, f, st);
}

}  // namespace
}  // namespace krsi

extern "C" {

int krsi_geglu_fwd(const void* u, void* out, int64_t rows, int32_t f, int32_t approximate,
                   int32_t dtype, void* stream) {
  using namespace krsi;
  int rc = check(rows, f, approximate, dtype);
  if (rc != KRSI_OK) return rc;
  if (rows == 0) return KRSI_OK;
  if (!u || !out) return KRSI_ERR_NULL_POINTER;
  hipStream_t st = as_stream(stream);
  return approximate == 1 ? geglu_fwd_dt<true>(u, out, rows, f, dtype, st)
                          : geglu_fwd_dt<false>(u, out, rows, f, dtype, st);
}

int krsi_geglu_bwd(const void* g, const void* u, void* du, int64_t rows, int32_t f,
                   int32_t approximate, int32_t dtype, void* stream) {
  using namespace krsi;
  int rc = check(rows, f, approximate, dtype);
  if (rc != KRSI_OK) return rc;
  if (rows == 0) return KRSI_OK;
  if (!g || !u || !du) return KRSI_ERR_NULL_POINTER;
  hipStream_t st = as_stream(stream);
  return approximate == 1 ? geglu_bwd_dt<true>(g, u, du, rows, f, dtype, st)
                          : geglu_bwd_dt<false>(g, u, du, rows, f, dtype, st);
}

int krsi_geglu_fwd_bf16(const void* u, void* out, int64_t rows, int32_t f, int32_t approximate,
                        void* stream) {
  return krsi_geglu_fwd(u, out, rows, f, approximate, KRSI_DTYPE_BF16, stream);
}

int krsi_geglu_bwd_bf16(const void* g, const void* u, void* du, int64_t rows, int32_t f,
                        int32_t approximate, void* stream) {
  return krsi_geglu_bwd(g, u, du, rows, f, approximate, KRSI_DTYPE_BF16, stream);
}

}  // extern "C"
