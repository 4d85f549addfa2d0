// Pieces shared by the 16-bit and the fp32 relative-position attention kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace krsi {

constexpr float kLog2e = 1.4426950408889634f;

// Keys per workgroup of the dK/dV kernels, which is also the length unit of the dpd partial
// rows: one row of S + kKvRows floats per (batch, head, key block).
constexpr int kKvRows = 128;

// Tile of a 1-D grid of N = (blocks per head) x (B*H) workgroups. Workgroups are handed
// to the 8 XCDs round-robin by linear id and every XCD has its own L2, so XCD x gets the
// contiguous tile range [x N/8, (x+1) N/8) in order: the blocks of one (batch, head) run
// on one XCD at about the same time and share its streamed K/V (or Q/dO) tiles in L2.
constexpr int kXcds = 8;
__device__ __forceinline__ int xcd_tile(int w, int N) {
  const int x = w % kXcds, k = w / kXcds, q = N / kXcds, r = N % kXcds;
  return x * q + min(x, r) + k;
}

// dpd (+)= sum over batches and key blocks kb0 .. kb0 + nkc - 1 of the dpd partial rows
// (fixed order), launched on `stream` after the dK/dV kernel has written `part`, which holds
// the rows of those nkc key blocks only. acc_in adds the sum to dpd instead of storing it.
// Defined in relpos_attn.hip.
void launch_dpd_reduce(const float* part, float* dpd, int B, int S, int H, int kb0, int nkc,
                       bool acc_in, hipStream_t stream);

// Key blocks whose partial rows fit a workspace of ws_bytes (delta first, then the rows),
// at most all of them; 0 when not even one block's rows fit.
int relpos_bwd_chunk_blocks(size_t ws_bytes, int B, int S, int H);

// fp32 activations (relpos_attn_f32.hip). Arguments as the 16-bit entry points; the
// caller has validated them.
int relpos_fwd_f32(const float* qkv, int64_t ld, const float* pd, float* out, float* out32,
                   float* lse, int B, int S, int H, int D, float scale, hipStream_t st);
int relpos_bwd_f32(const float* dout, const float* qkv, int64_t ld, const float* pd,
                   const float* out32, const float* lse, float* dqkv, int64_t ldd, float* dpd,
                   float* delta, float* part, int nkc, int B, int S, int H, int D, float scale,
                   hipStream_t st);

}  // namespace krsi
