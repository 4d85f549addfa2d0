// The step before and after the attention for a bucketed relative-position table
// (T5: an nn.Embedding of num_buckets x H, indexed by the bucket of j - i).
//
//   gather     pd[h, r]     = table[bucket[r], h]          r = j - i + S - 1
//   bucket sum dtable[b, h] = sum of dpd[h, r] over r with bucket[r] == b
//
// The reference's note on this step (LESSONS.md:35): the embedding backward is a
// contended scatter-add over S^2 indices; summing dBias along the diagonals into
// the per-distance table [H, 2S-1] (the attention backward does that) and then
// into the buckets needs no scatter. Here the bucket sum is a gather as well: each
// workgroup reads the whole bucket map for one head and a few buckets and adds their
// entries in a fixed order, so dtable is bitwise reproducible with no atomics. The map
// is 2S-1 int32 (32 KB at S = 4096) and stays in L2 for all the workgroups.
#include "krsi_device.h"
#include "krsi_internal.h"

namespace krsi {
namespace {

constexpr int kThreads = 256;

// One thread per distance r of one head h (grid: distance tiles x H). A bucket
// outside [0, nb) gives NaN, so a bad map shows in the output rather than as
// an out-of-bounds read.
__global__ __launch_bounds__(kThreads) void bucket_gather(const float* __restrict__ table,
                                                         const int32_t* __restrict__ bucket,
                                                         float* __restrict__ pd, int npd, int H,
                                                         int nb) {
  const int r = blockIdx.x * kThreads + threadIdx.x;
  const int h = blockIdx.y;
  if (r >= npd) return;
  const int b = bucket[r];
  pd[(int64_t)h * npd + r] = (b >= 0 && b < nb) ? table[(int64_t)b * H + h] : __builtin_nanf("");
}

// Workgroup (g, h) sums buckets b = g NBW + k, k < NBW (those below nb): thread t adds
// dpd[h, r] for r = t, t + 256, ... with bucket[r] == b, in that order, into its own sum per
// bucket, each entry and bucket id loaded once for all NBW buckets; each bucket's 256 partial
// sums are then added by a fixed tree (wave-level shuffles, then the 4 wave sums in wave
// order). Every entry is added to every sum, as +0 where the bucket differs, so the loads do
// not wait on the compares; a sum starts at +0 and no sum rounds to -0, so adding +0 leaves it
// bitwise unchanged: each bucket's result does not depend on NBW. The entry is loaded ahead of
// the compares, so no load waits behind one (the earlier `bucket[r] == b ? row[r] : 0` form took
// 6.9 us at S 4096, H 16, 32 buckets; this one 3.8 us with NBW = 1, 4.0 / 4.7 / 6.5 us with NBW =
// 2 / 4 / 8; at S <= 1024 every NBW takes 3.8-4.0 us, the launch floor).
constexpr int kBucketsPerWg = 1;
template <int NBW>
__global__ __launch_bounds__(kThreads) void bucket_sum(const float* __restrict__ dpd,
                                                      const int32_t* __restrict__ bucket,
                                                      float* __restrict__ dtable, int npd, int H, int nb) {
  __shared__ float s[NBW][kThreads / kWave];
  const int b0 = blockIdx.x * NBW, h = blockIdx.y;
  const float* row = dpd + (int64_t)h * npd;
  float acc[NBW];
#pragma unroll
  for (int k = 0; k < NBW; ++k) acc[k] = 0.f;
#pragma unroll 8
  for (int r = threadIdx.x; r < npd; r += kThreads) {
    const int br = bucket[r];
    const float v = row[r];
#pragma unroll
    for (int k = 0; k < NBW; ++k) acc[k] += br == b0 + k ? v : 0.f;
  }
#pragma unroll
  for (int k = 0; k < NBW; ++k) {
    const float w = wave_sum(acc[k]);
    if ((threadIdx.x & (kWave - 1)) == 0) s[k][threadIdx.x / kWave] = w;
  }
  __syncthreads();
  if (threadIdx.x < NBW && b0 + (int)threadIdx.x < nb) {
    const int k = threadIdx.x;
    dtable[(int64_t)(b0 + k) * H + h] = ((s[k][0] + s[k][1]) + s[k][2]) + s[k][3];
  }
}

int check_bucket(int S, int H, int nb) {
  if (S <= 0 || H <= 0 || nb <= 0) return KRSI_ERR_BAD_SHAPE;
  if (S > (1 << 24) || H > 65535 || nb > 65535) return KRSI_ERR_BAD_SHAPE;
  return KRSI_OK;
}

}  // namespace
}  // namespace krsi

extern "C" {

int krsi_relpos_bucket_gather(const float* table, const int32_t* bucket, float* pd, int32_t S,
                              int32_t H, int32_t num_buckets, void* stream) {
  using namespace krsi;
  int rc = check_bucket(S, H, num_buckets);
  if (rc != KRSI_OK) return rc;
  if (!table || !bucket || !pd) return KRSI_ERR_NULL_POINTER;
  const int npd = 2 * S - 1;
  hipLaunchKernelGGL(bucket_gather, dim3((unsigned)ceil_div(npd, kThreads), (unsigned)H),
                     dim3(kThreads), 0, as_stream(stream), table, bucket, pd, npd, (int)H,
                     (int)num_buckets);
  return launch_status();
}

int krsi_relpos_bucket_sum(const float* dpd, const int32_t* bucket, float* dtable, int32_t S,
                           int32_t H, int32_t num_buckets, void* stream) {
  using namespace krsi;
  int rc = check_bucket(S, H, num_buckets);
  if (rc != KRSI_OK) return rc;
  if (!dpd || !bucket || !dtable) return KRSI_ERR_NULL_POINTER;
  hipLaunchKernelGGL(bucket_sum<kBucketsPerWg>, dim3((unsigned)ceil_div(num_buckets, kBucketsPerWg), (unsigned)H),
                     dim3(kThreads), 0, as_stream(stream), dpd, bucket, dtable, 2 * S - 1, (int)H,
                     (int)num_buckets);
  return launch_status();
}

}  // extern "C"
