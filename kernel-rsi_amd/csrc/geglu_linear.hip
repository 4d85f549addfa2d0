// Merged gate|up projection with the GEGLU epilogue in one kernel, for gfx950:
//   u   = T(x w^T)                   x [rows, K], w = [Wg; Wu] [2F, K] (nn.Linear layout), T = dtype
//   out = T( T(gelu(u[:, :F])) * u[:, F:] )                                          [rows, F]
// This is library/geglu.py's operation on the output of the merged GEMM its docstring names
// (geglu.py:3-5), without writing u to HBM and reading it back. The rounding points are the
// unfused pair's: the fp32 GEMM accumulators are rounded to T (u's dtype), then the GEGLU
// forward of geglu.hip (the same gelu from gelu_math.h) runs on them.
//
// Tiling (bf16 / fp16 MFMA v_mfma_f32_32x32x16, fp32 accumulate):
//   * Workgroup = 4 waves, 128 rows x 64 output columns. The weight tile stacks the 64 gate rows
//     and the 64 up rows of those columns, so each lane holds gate and up of the same outputs
//     and the epilogue needs no exchange.
//   * Wave (wr, wc): rows 64 wr .. + 63 (two 32-row blocks) x output columns 32 wc .. + 31, four
//     accumulators (2 row blocks x {gate, up}).
//   * K is streamed in stages of 64 through double-buffered LDS. Both operands are 16-byte
//     chunks of K-contiguous rows (A: x rows, B: w rows), so both are 128-bit row reads, XOR-
//     swizzled per row to be conflict-free. Stages go HBM -> LDS directly (buffer_load ... lds),
//     with the next stage requested before the current one is computed; one barrier per stage.
//   * Rows past the end read as zero (buffer range check) and are not stored.
// Requires K % 64 == 0 and F % 64 == 0; the host checks.
#include "gelu_math.h"
#include "krsi_device.h"
#include "krsi_internal.h"
#include "relpos_common.h"

namespace krsi {
namespace {

constexpr int kGlRows = 128;   // rows (of x and out) per workgroup
constexpr int kGlCols = 64;    // output columns per workgroup: 128 rows of w (64 gate + 64 up)
constexpr int kGlK = 64;       // K per stage
constexpr int kGlGroup = 4;    // row blocks per tile group (tile order, below)
constexpr int kGlThreads = 256;
constexpr int kGlTile = 128 * kGlK;  // 16-bit elements per staged tile (x or w)
constexpr int kGlChunks = kGlTile / 8;
constexpr int kGlDmaPerThread = kGlChunks / kGlThreads;  // 4
static_assert(kGlChunks % kGlThreads == 0, "each thread fills whole chunks");

typedef __amdgpu_buffer_rsrc_t rsrc_t;
typedef __attribute__((address_space(3))) void lds_void;
constexpr int kRsrcWord3 = 0x00020000;

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, kRsrcWord3);
}
__device__ __forceinline__ uint32_t opaque(uint32_t v) {
  asm volatile("" : "+v"(v));
  return v;
}
// One 16-byte load from the buffer straight into LDS at M0 + 16 * lane.
__device__ __forceinline__ void dma16(rsrc_t r, uint32_t voff, uint32_t m0) {
  asm volatile("buffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(voff), "s"(r), "{m0}"(m0) : "memory");
}

// Chunk j (8 elements) of staged row r sits at position j ^ swz(r) of the row's 8 chunks: the 16
// rows of a 128-bit read phase (one chunk each) and a DMA wave's 64 chunks both hit distinct
// bank quads.
__device__ __forceinline__ int swz(int r) { return (((r >> 1) & 1) << 2) | ((r >> 2) & 3); }
__device__ __forceinline__ int toff(int r, int j) { return r * kGlK + 8 * (j ^ swz(r)); }

template <int DT, bool TANH>
__global__ __launch_bounds__(kGlThreads, 2) void geglu_linear_fwd_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w, uint16_t* __restrict__ out,
    int64_t rows, int K, int F, int ncb, int nrb) {
  __shared__ __attribute__((aligned(16))) uint16_t Xs[2 * kGlTile];
  __shared__ __attribute__((aligned(16))) uint16_t Ws[2 * kGlTile];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, g = lane >> 5, l32 = lane & 31;
  const int wr = wave >> 1, wc = wave & 1;
  // Tile order. xcd_tile gives each XCD a contiguous range of tiles. Inside it the tiles go in
  // groups of kGlGroup row blocks: consecutive tiles walk the group's row blocks first, then
  // its column blocks. The workgroups in flight on one XCD then share a few row blocks of x
  // and a few column blocks of w in that XCD's L2. Walking one row block across every column
  // block instead made each XCD stream all of w once per row block it owns: 4.4 GB fetched per
  // call at x [8192, 4096], F = 4096, against 0.13 GB of inputs.
  const int tile = xcd_tile(blockIdx.x, gridDim.x);
  const int per_group = kGlGroup * ncb;
  const int grp = tile / per_group, in_grp = tile - grp * per_group;
  const int rb0 = grp * kGlGroup;
  const int gsz = min(kGlGroup, nrb - rb0);
  const int64_t m0 = (int64_t)(rb0 + in_grp % gsz) * kGlRows;
  const int c0 = (in_grp / gsz) * kGlCols;

  // DMA: thread chunk p = k * 256 + tid of a tile is staged row p / 8, position p % 8, which
  // holds logical chunk (p % 8) ^ swz(row). Rows 0-63 of the w tile are gate rows c0 .., rows
  // 64-127 up rows F + c0 .. (k = 0, 1 and k = 2, 3).
  uint32_t xoff[kGlDmaPerThread], woff[kGlDmaPerThread];
#pragma unroll
  for (int k = 0; k < kGlDmaPerThread; ++k) {
    const int p = k * kGlThreads + tid;
    const int row = p >> 3;
    const int j = (p & 7) ^ swz(row);
    xoff[k] = opaque((uint32_t)(row * K + 8 * j) * 2u);
    woff[k] = opaque((uint32_t)((row & 63) * K + 8 * j) * 2u);
  }
  const uint32_t wbytes = (uint32_t)(64 * K) * 2u;
  const uint16_t* xrow0 = x + m0 * K;
  const uint64_t xleft = (uint64_t)(rows - m0) * (uint64_t)K * 2u;  // bytes of x from row m0 on
  auto stage = [&](int buf, int k0) {
    // x rows past the end fall past the resource and read as zero.
    const uint64_t left = xleft - (uint64_t)k0 * 2u;
    const rsrc_t rx = make_rsrc(xrow0 + k0, (uint32_t)(left < 0x7fffffffu ? left : 0x7fffffffu));
    const rsrc_t rg = make_rsrc(w + (int64_t)c0 * K + k0, wbytes);
    const rsrc_t ru = make_rsrc(w + ((int64_t)F + c0) * K + k0, wbytes);
    const int wv = __builtin_amdgcn_readfirstlane(wave);
#pragma unroll
    for (int k = 0; k < kGlDmaPerThread; ++k) {
      const uint32_t m0x = (uint32_t)(uintptr_t)(lds_void*)(Xs + buf * kGlTile + (k * kGlThreads + 64 * wv) * 8);
      const uint32_t m0w = (uint32_t)(uintptr_t)(lds_void*)(Ws + buf * kGlTile + (k * kGlThreads + 64 * wv) * 8);
      dma16(rx, xoff[k], m0x);
      dma16(k < 2 ? rg : ru, woff[k], m0w);
    }
  };

  f32x16 acc[2][2];  // [row block][gate, up]
#pragma unroll
  for (int rb = 0; rb < 2; ++rb)
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[rb][h][r] = 0.f;

  // Per-lane operand offsets: A rows 64 wr + 32 rb + l32; B rows 32 wc + l32 (gate), + 64 (up);
  // k-step s reads chunk 2 s + g.
  int aoff[2][4], boff[2][4];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) aoff[rb][s] = toff(64 * wr + 32 * rb + l32, 2 * s + g);
#pragma unroll
    for (int h = 0; h < 2; ++h) boff[h][s] = toff(64 * h + 32 * wc + l32, 2 * s + g);
  }

  const int nk = K / kGlK;
  stage(0, 0);
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();  // stage kt is in LDS; every wave is done with stage kt - 1
    if (kt + 1 < nk) stage(buf ^ 1, (kt + 1) * kGlK);
    const uint16_t* xs = Xs + buf * kGlTile;
    const uint16_t* ws = Ws + buf * kGlTile;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      u32x4 a[2], b[2];
#pragma unroll
      for (int rb = 0; rb < 2; ++rb) a[rb] = *reinterpret_cast<const u32x4*>(xs + aoff[rb][s]);
#pragma unroll
      for (int h = 0; h < 2; ++h) b[h] = *reinterpret_cast<const u32x4*>(ws + boff[h][s]);
#pragma unroll
      for (int rb = 0; rb < 2; ++rb)
#pragma unroll
        for (int h = 0; h < 2; ++h) acc[rb][h] = mfma32x32x16<DT>(a[rb], b[h], acc[rb][h]);
    }
  }

  // Epilogue: lane column c0 + 32 wc + l32; register r of row block rb is row
  // m0 + 64 wr + 32 rb + 8 (r / 4) + 4 g + r % 4.
  using El = Elem<DT>;
  const int col = c0 + 32 * wc + l32;
#pragma unroll
  for (int rb = 0; rb < 2; ++rb)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int64_t row = m0 + 64 * wr + 32 * rb + 8 * (r >> 2) + 4 * g + (r & 3);
      if (row < rows) {
        const float a = El::round(acc[rb][0][r]);
        const float b = El::round(acc[rb][1][r]);
        out[row * F + col] = El::store(El::round(gelu_fwd<TANH>(a)) * b);
      }
    }
}

template <int DT>
int launch_geglu_linear(const void* x, const void* w, void* out, int64_t rows, int K, int F, bool tanh_form,
                        hipStream_t st) {
  const int ncb = F / kGlCols;
  const int64_t nrb = ceil_div(rows, kGlRows);
  const int64_t tiles = nrb * ncb;
  if (tiles > 0x7fffffff) return KRSI_ERR_BAD_SHAPE;
  const dim3 grid((unsigned)tiles);
  if (tanh_form)
    hipLaunchKernelGGL((geglu_linear_fwd_kernel<DT, true>), grid, dim3(kGlThreads), 0, st, (const uint16_t*)x,
                       (const uint16_t*)w, (uint16_t*)out, rows, K, F, ncb, (int)nrb);
  else
    hipLaunchKernelGGL((geglu_linear_fwd_kernel<DT, false>), grid, dim3(kGlThreads), 0, st, (const uint16_t*)x,
                       (const uint16_t*)w, (uint16_t*)out, rows, K, F, ncb, (int)nrb);
  return launch_status();
}

}  // namespace
}  // namespace krsi

extern "C" {

int krsi_geglu_linear_fwd(const void* x, const void* w, void* out, int64_t rows, int32_t k, int32_t f,
                          int32_t approximate, int32_t dtype, void* stream) {
  using namespace krsi;
  if (dtype != kBf16 && dtype != kF16) return KRSI_ERR_UNSUPPORTED;
  if (approximate != 0 && approximate != 1) return KRSI_ERR_UNSUPPORTED;
  if (rows < 0 || k <= 0 || f <= 0) return KRSI_ERR_BAD_SHAPE;
  if (k % kGlK != 0 || f % kGlCols != 0) return KRSI_ERR_UNSUPPORTED;
  // Buffer resources: the byte offsets of one stage (128 rows of x, 64 rows of w) stay below 2^31.
  if ((int64_t)128 * k * 2 >= ((int64_t)1 << 31)) return KRSI_ERR_UNSUPPORTED;
  if (rows == 0) return KRSI_OK;
  if (!x || !w || !out) return KRSI_ERR_NULL_POINTER;
  if (!aligned16(x) || !aligned16(w)) return KRSI_ERR_MISALIGNED;
  hipStream_t st = as_stream(stream);
  return dtype == kF16 ? launch_geglu_linear<kF16>(x, w, out, rows, k, f, approximate == 1, st)
                       : launch_geglu_linear<kBf16>(x, w, out, rows, k, f, approximate == 1, st);
}

}  // extern "C"
