// Device-side helpers shared by the gfx950 kernels: bf16 / fp16 <-> fp32
// conversion, the element-type traits, 128-bit vector types, wave64 reductions
// and the 16-bit MFMA wrapper.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace krsi {

constexpr int kWave = 64;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2;
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// bf16 is stored as raw 16-bit patterns. Widening is exact: the bf16 bits are
// the top half of the fp32 bits.
// Loads whose lanes may have no data: every lane loads (from a valid address where it has
// none) and the value is ANDed with an all-ones / zero lane mask. A select of the loaded
// value, or a conditional load, was turned by the compiler into one branch per load that
// waited for its data, so consecutive loads went to memory one after another. The mask
// passes through an empty asm, so the AND cannot be turned back into a select.
__device__ __forceinline__ uint32_t lane_mask(bool ok) {
  uint32_t m = ok ? 0xffffffffu : 0u;
  asm volatile("" : "+v"(m));
  return m;
}
__device__ __forceinline__ u32x4 masked(u32x4 v, uint32_t m) {
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] &= m;
  return v;
}

__device__ __forceinline__ float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

// fp32 -> bf16 with round-to-nearest-even (gfx950 v_cvt_pk_bf16_f32), the
// rounding torch uses for .to(torch.bfloat16).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  bf16x2 v;
  v[0] = (__bf16)lo;
  v[1] = (__bf16)hi;
  return __builtin_bit_cast(uint32_t, v);
}
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  return __builtin_bit_cast(uint16_t, (__bf16)f);
}
// Round fp32 to the nearest bf16 and widen back: the value a bf16 tensor
// would hold at this point of an eager computation.
__device__ __forceinline__ float round_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }

// Unpack 8 bf16 (one 128-bit word) to fp32.
__device__ __forceinline__ void unpack8(const u32x4& w, float* f) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = bf_lo(w[i]);
    f[2 * i + 1] = bf_hi(w[i]);
  }
}
__device__ __forceinline__ u32x4 pack8(const float* f) {
  u32x4 w;
#pragma unroll
  for (int i = 0; i < 4; ++i) w[i] = pack_bf16x2(f[2 * i], f[2 * i + 1]);
  return w;
}

// fp16 is stored as raw 16-bit patterns too; widening is exact, narrowing is
// round-to-nearest-even with overflow to inf (gfx950 v_cvt_pk_f16_f32), the
// rounding torch uses for .to(torch.float16).
__device__ __forceinline__ float h_lo(uint32_t w) { return (float)__builtin_bit_cast(f16x2, w)[0]; }
__device__ __forceinline__ float h_hi(uint32_t w) { return (float)__builtin_bit_cast(f16x2, w)[1]; }
__device__ __forceinline__ uint32_t pack_f16x2(float lo, float hi) {
  f16x2 v;
  v[0] = (_Float16)lo;
  v[1] = (_Float16)hi;
  return __builtin_bit_cast(uint32_t, v);
}

// Activation element types. The reference's kernels take any float dtype and round
// at the same points in that dtype; the values match the KRSI_DTYPE_* codes.
constexpr int kBf16 = 0, kF16 = 1, kF32 = 2;

// Elem<DT>: storage type, elements per 16-byte chunk, and the conversions:
//   load(s)   storage -> fp32 (exact);   store(f)  fp32 -> storage, RNE;
//   round(f)  the fp32 value a tensor of this dtype holds after .to(dtype);
//   unpack/pack  one 16-byte chunk <-> E fp32 values;
//   pack2(lo, hi)  two values -> one 32-bit word (16-bit types only).
template <int DT>
struct Elem;

template <>
struct Elem<kBf16> {
  using T = uint16_t;
  static constexpr int E = 8;
  static __device__ __forceinline__ float load(T h) { return bf16_to_f32(h); }
  static __device__ __forceinline__ T store(float f) { return f32_to_bf16(f); }
  static __device__ __forceinline__ float round(float f) { return round_bf16(f); }
  static __device__ __forceinline__ void unpack(const u32x4& w, float* f) { unpack8(w, f); }
  static __device__ __forceinline__ u32x4 pack(const float* f) { return pack8(f); }
  static __device__ __forceinline__ uint32_t pack2(float lo, float hi) { return pack_bf16x2(lo, hi); }
};

template <>
struct Elem<kF16> {
  using T = uint16_t;
  static constexpr int E = 8;
  static __device__ __forceinline__ float load(T h) { return (float)__builtin_bit_cast(_Float16, h); }
  static __device__ __forceinline__ T store(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }
  static __device__ __forceinline__ float round(float f) { return (float)(_Float16)f; }
  static __device__ __forceinline__ void unpack(const u32x4& w, float* f) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = h_lo(w[i]);
      f[2 * i + 1] = h_hi(w[i]);
    }
  }
  static __device__ __forceinline__ u32x4 pack(const float* f) {
    u32x4 w;
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = pack_f16x2(f[2 * i], f[2 * i + 1]);
    return w;
  }
  static __device__ __forceinline__ uint32_t pack2(float lo, float hi) { return pack_f16x2(lo, hi); }
};

template <>
struct Elem<kF32> {
  using T = float;
  static constexpr int E = 4;
  static __device__ __forceinline__ float load(T v) { return v; }
  static __device__ __forceinline__ T store(float f) { return f; }
  static __device__ __forceinline__ float round(float f) { return f; }
  static __device__ __forceinline__ void unpack(const u32x4& w, float* f) {
#pragma unroll
    for (int i = 0; i < 4; ++i) f[i] = __uint_as_float(w[i]);
  }
  static __device__ __forceinline__ u32x4 pack(const float* f) {
    return u32x4{__float_as_uint(f[0]), __float_as_uint(f[1]), __float_as_uint(f[2]),
                 __float_as_uint(f[3])};
  }
};

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, kWave);
  return v;
}

// D = A(32x16) * B(16x32) + C on bf16 or fp16 MFMA, fp32 accumulate.
// Operand convention used by every kernel in this library (wave64):
//   A: lane l holds A[m = l % 32][k = 8 * (l / 32) + j], j = 0..7
//   B: lane l holds B[k = 8 * (l / 32) + j][n = l % 32], j = 0..7
//   D: lane l, register r holds D[m = 8 * (r / 4) + 4 * (l / 32) + r % 4][n = l % 32]
// Only the pairing of A and B slots matters for K (it is summed over), so a
// kernel may assign any logical K index to (l / 32, j) as long as A and B agree.
// DT selects the bf16 or the fp16 instruction (same shapes and operand layout).
template <int DT = kBf16>
__device__ __forceinline__ f32x16 mfma32x32x16(const u32x4& a, const u32x4& b, const f32x16& c) {
  static_assert(DT == kBf16 || DT == kF16, "16-bit MFMA operands");
  if constexpr (DT == kF16)
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

}  // namespace krsi
