// The step before and after the attention for a bucketed relative-position table
// (T5: an nn.Embedding of num_buckets x H, indexed by the bucket of j - i).
//
//   gather     pd[h, r]     = table[bucket[r], h]          r = j - i + S - 1
//   bucket sum dtable[b, h] = sum of dpd[h, r] over r with bucket[r] == b
//
// The reference's note on this step (LESSONS.md:35): the embedding backward is a
// contended scatter-add over S^2 indices; summing dBias along the diagonals into
// the per-distance table [H, 2S-1] (the attention backward does that) and then
// into the buckets needs no scatter. Here the bucket sum is a gather as well:
// workgroup (b, h) reads the whole bucket map and adds its own entries in a fixed
// order, so dtable is bitwise reproducible with no atomics. The map is 2S-1 int32
// (32 KB at S = 4096) and stays in L2 for all num_buckets x H workgroups.
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

// Workgroup (b, h): thread t adds dpd[h, r] for r = t, t + 256, ... with
// bucket[r] == b, in that order; the 256 partial sums are then added by a fixed
// tree (wave-level shuffles, then the 4 wave sums in wave order). Every entry is
// loaded and the others add +0, so the loads do not wait on the compares; acc
// starts at +0 and no sum rounds to -0, so adding +0 leaves it bitwise unchanged.
__global__ __launch_bounds__(kThreads) void bucket_sum(const float* __restrict__ dpd,
                                                      const int32_t* __restrict__ bucket,
                                                      float* __restrict__ dtable, int npd, int H) {
  __shared__ float s[kThreads / kWave];
  const int b = blockIdx.x, h = blockIdx.y;
  const float* row = dpd + (int64_t)h * npd;
  float acc = 0.f;
#pragma unroll 8
  for (int r = threadIdx.x; r < npd; r += kThreads) acc += bucket[r] == b ? row[r] : 0.f;
  acc = wave_sum(acc);
  if ((threadIdx.x & (kWave - 1)) == 0) s[threadIdx.x / kWave] = acc;
  __syncthreads();
  if (threadIdx.x == 0) dtable[(int64_t)b * H + h] = ((s[0] + s[1]) + s[2]) + s[3];
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
  hipLaunchKernelGGL(bucket_sum, dim3((unsigned)num_buckets, (unsigned)H), dim3(kThreads), 0,
                     as_stream(stream), dpd, bucket, dtable, 2 * S - 1, (int)H);
  return launch_status();
}

}  // extern "C"
