// RMSNorm forward and backward for gfx950.
//
// Semantics follow library/rmsnorm.py of the reference (kernel-rsi):
//   forward  (_rms_fwd, rmsnorm.py:22-31):
//     rstd = 1 / sqrt(sum(x^2) / N + eps)            fp32, stored per row
//     y    = w * T(x * rstd)                         (T x T -> T)
//   backward (_rms_bwd, rmsnorm.py:34-51, and the dwp.sum(0) of :68):
//     nrm  = T(x * rstd)
//     dw  += g * nrm                                 fp32, per block, then a
//                                                    fixed-order column sum
//     dn   = float(T(g * w))
//     dx   = rstd * dn - x * rstd^3 * (sum(dn * x) / N)
//   T is the activation dtype (bf16, fp16 or fp32: the template parameter DT),
//   as the reference rounds to w's dtype; T(.) is round-to-nearest-even.
//
// Design (MI355X): each row is owned by one wavefront (WPR = 1, N <= 4096) or
// by WPR wavefronts of one workgroup (N <= 8192 / 16384). Every lane moves
// whole 16-byte chunks (8 bf16 / fp16 or 4 fp32), so a wave reads 1 KiB per instruction
// and the row lives in registers between the reduction and the write. The
// backward is persistent: a fixed grid of NB workgroups walks the rows, keeps
// its share of dw in fp32 registers and writes one partial row per workgroup;
// one small column-sum launch reduces the (at most 512) partials in a fixed
// order, so dw is bitwise reproducible. Rows whose length is not a multiple of 8, or whose
// pointers are not 16-byte aligned, take a scalar path with the same math.
#include "krsi_device.h"
#include "krsi_internal.h"

#include <initializer_list>
#include <mutex>

namespace krsi {
namespace {

constexpr int kThreads = 256;
constexpr int kWavesPerBlock = kThreads / kWave;
constexpr int kBwdMaxBlocks = 512;     // persistent grid of the backward
constexpr int kColsumWaves = 16;       // waves per column-sum workgroup (64 columns each)
constexpr int kScalarRowChunk = 64;    // rows per block of the scalar dw kernel

// ----------------------------------------------------------------- forward
template <int DT, int WPR, int VPT>
__global__ __launch_bounds__(kThreads) void rms_fwd_vec(const typename Elem<DT>::T* __restrict__ x,
                                                        const typename Elem<DT>::T* __restrict__ w,
                                                        typename Elem<DT>::T* __restrict__ y,
                                                        float* __restrict__ rstd, int64_t rows,
                                                        int n, float eps) {
  using El = Elem<DT>;
  constexpr int E = El::E;                   // elements per 16-byte chunk
  constexpr int RPB = kWavesPerBlock / WPR;  // rows per block
  constexpr int GT = WPR * kWave;            // threads per row group
  __shared__ float red[kWavesPerBlock];
  const int wave = threadIdx.x / kWave;
  const int grp = wave / WPR;
  const int gtid = threadIdx.x - grp * GT;
  const int64_t row = (int64_t)blockIdx.x * RPB + grp;
  const bool live = row < rows;
  const int nch = n / E;

  u32x4 xv[VPT];
  float ss = 0.f;
  const u32x4* xr = reinterpret_cast<const u32x4*>(x + (live ? row : 0) * (int64_t)n);
#pragma unroll
  for (int k = 0; k < VPT; ++k) {
    const int c = gtid + k * GT;
    // x streams in non-temporally (cache-cold at config 2: forward 88.0 -> 87.1 us).
    xv[k] = (live && c < nch) ? __builtin_nontemporal_load(&xr[c]) : u32x4{0u, 0u, 0u, 0u};
  }
#pragma unroll
  for (int k = 0; k < VPT; ++k) {
    float f[E];
    El::unpack(xv[k], f);
#pragma unroll
    for (int j = 0; j < E; ++j) ss += f[j] * f[j];
  }
  ss = wave_sum(ss);
  if (WPR > 1) {
    if ((threadIdx.x & (kWave - 1)) == 0) red[wave] = ss;
    __syncthreads();
    ss = 0.f;
#pragma unroll
    for (int i = 0; i < WPR; ++i) ss += red[grp * WPR + i];
  }
  if (!live) return;
  const float r = 1.0f / __fsqrt_rn(ss / (float)n + eps);
  if (gtid == 0) rstd[row] = r;
  const u32x4* wr = reinterpret_cast<const u32x4*>(w);
  u32x4* yr = reinterpret_cast<u32x4*>(y + row * (int64_t)n);
#pragma unroll
  for (int k = 0; k < VPT; ++k) {
    const int c = gtid + k * GT;
    if (c < nch) {
      float xf[E], wf[E], o[E];
      El::unpack(xv[k], xf);
      El::unpack(wr[c], wf);
#pragma unroll
      for (int j = 0; j < E; ++j) o[j] = wf[j] * El::round(xf[j] * r);
      __builtin_nontemporal_store(El::pack(o), &yr[c]);  // streamed out, not re-read
    }
  }
}

// One wave per row, any alignment, any n.
template <int DT>
__global__ __launch_bounds__(kThreads) void rms_fwd_scalar(const typename Elem<DT>::T* __restrict__ x,
                                                           const typename Elem<DT>::T* __restrict__ w,
                                                           typename Elem<DT>::T* __restrict__ y,
                                                           float* __restrict__ rstd, int64_t rows,
                                                           int n, float eps) {
  using El = Elem<DT>;
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row = (int64_t)blockIdx.x * kWavesPerBlock + threadIdx.x / kWave;
  if (row >= rows) return;
  const typename El::T* xr = x + row * (int64_t)n;
  float ss = 0.f;
  for (int c = lane; c < n; c += kWave) {
    const float f = El::load(xr[c]);
    ss += f * f;
  }
  ss = wave_sum(ss);
  const float r = 1.0f / __fsqrt_rn(ss / (float)n + eps);
  if (lane == 0) rstd[row] = r;
  typename El::T* yr = y + row * (int64_t)n;
  for (int c = lane; c < n; c += kWave)
    yr[c] = El::store(El::load(w[c]) * El::round(El::load(xr[c]) * r));
}

// ---------------------------------------------------------------- backward
// Persistent: gridDim.x blocks, each block handles row groups
// blockIdx.x, blockIdx.x + gridDim.x, ... Every group of the block runs the
// same number of iterations so that the WPR > 1 barriers stay uniform.
template <int DT, int WPR, int VPT>
__global__ __launch_bounds__(kThreads) void rms_bwd_vec(
    const typename Elem<DT>::T* __restrict__ g, const typename Elem<DT>::T* __restrict__ x,
    const typename Elem<DT>::T* __restrict__ w, const float* __restrict__ rstd,
    typename Elem<DT>::T* __restrict__ dx, float* __restrict__ part, int64_t rows, int n) {
  using El = Elem<DT>;
  constexpr int E = El::E;
  constexpr int RPB = kWavesPerBlock / WPR;
  constexpr int GT = WPR * kWave;
  __shared__ float red[2][kWavesPerBlock];
  __shared__ __attribute__((aligned(16))) float comb[4096];
  const int wave = threadIdx.x / kWave;
  const int grp = wave / WPR;
  const int gtid = threadIdx.x - grp * GT;
  const int nch = n / E;
  const float inv_n = 1.0f / (float)n;

  float wv[VPT][E];
  float dw[VPT][E];
  const u32x4* wr = reinterpret_cast<const u32x4*>(w);
#pragma unroll
  for (int k = 0; k < VPT; ++k) {
    const int c = gtid + k * GT;
    El::unpack(c < nch ? wr[c] : u32x4{0u, 0u, 0u, 0u}, wv[k]);
#pragma unroll
    for (int j = 0; j < E; ++j) dw[k][j] = 0.f;
  }

  const int64_t groups_total = (int64_t)gridDim.x * RPB;
  const int64_t iters = (rows + groups_total - 1) / groups_total;
  // The next row's g, x and rstd are requested before this row is reduced and written, so
  // every wave keeps one row of loads in flight. g, x and dx take non-temporal loads and
  // stores: at [32768, 4096] a forward + backward step takes 211 us against 215 us with g
  // loaded normally (the backward alone is slower, 137 vs 123 us, but leaves more of x in the
  // memory-side cache for the next forward; marking the forward's x loads as well: 222 us).
  u32x4 gv[VPT], xv[VPT];
  float r;
  auto fetch = [&](int64_t row, u32x4* gq, u32x4* xq, float& rq) {
    const bool live = row < rows;
    const int64_t base = (live ? row : 0) * (int64_t)n;
    const u32x4* gr = reinterpret_cast<const u32x4*>(g + base);
    const u32x4* xr = reinterpret_cast<const u32x4*>(x + base);
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
      const int c = gtid + k * GT;
      const bool ok = live && c < nch;
      gq[k] = ok ? __builtin_nontemporal_load(&gr[c]) : u32x4{0u, 0u, 0u, 0u};
      xq[k] = ok ? __builtin_nontemporal_load(&xr[c]) : u32x4{0u, 0u, 0u, 0u};
    }
    rq = live ? rstd[row] : 0.f;
  };
  int64_t row = (int64_t)blockIdx.x * RPB + grp;
  fetch(row, gv, xv, r);
  for (int64_t it = 0; it < iters; ++it, row += groups_total) {
    const bool live = row < rows;
    const int64_t base = (live ? row : 0) * (int64_t)n;
    u32x4 gn[VPT], xn[VPT];
    float rn = 0.f;
    if (it + 1 < iters) fetch(row + groups_total, gn, xn, rn);
    float sdot = 0.f;
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
      float gf[E], xf[E];
      El::unpack(gv[k], gf);
      El::unpack(xv[k], xf);
#pragma unroll
      for (int j = 0; j < E; ++j) {
        const float nrm = El::round(xf[j] * r);
        dw[k][j] += gf[j] * nrm;
        const float dn = El::round(gf[j] * wv[k][j]);
        sdot += dn * xf[j];
      }
    }
    sdot = wave_sum(sdot);
    if (WPR > 1) {
      if ((threadIdx.x & (kWave - 1)) == 0) red[it & 1][wave] = sdot;
      __syncthreads();
      sdot = 0.f;
#pragma unroll
      for (int i = 0; i < WPR; ++i) sdot += red[it & 1][grp * WPR + i];
    }
    if (live) {
      const float r3 = r * r * r;
      const float sn = sdot * inv_n;
      u32x4* dxr = reinterpret_cast<u32x4*>(dx + base);
#pragma unroll
      for (int k = 0; k < VPT; ++k) {
        const int c = gtid + k * GT;
        if (c < nch) {
          float gf[E], xf[E], o[E];
          El::unpack(gv[k], gf);
          El::unpack(xv[k], xf);
#pragma unroll
          for (int j = 0; j < E; ++j) {
            const float dn = El::round(gf[j] * wv[k][j]);
            o[j] = r * dn - (xf[j] * r3) * sn;
          }
          __builtin_nontemporal_store(El::pack(o), &dxr[c]);
        }
      }
    }
    if (it + 1 < iters) {
#pragma unroll
      for (int k = 0; k < VPT; ++k) {
        gv[k] = gn[k];
        xv[k] = xn[k];
      }
      r = rn;
    }
  }

  // Fold the RPB row groups' dw into one partial row per block, in group
  // order, through a 4096-float LDS window.
  constexpr int WCH = 4096 / E;  // chunks per LDS window
  float* prow = part + (int64_t)blockIdx.x * n;
  for (int w0 = 0; w0 < nch; w0 += WCH) {
    for (int gi = 0; gi < RPB; ++gi) {
      if (grp == gi) {
#pragma unroll
        for (int k = 0; k < VPT; ++k) {
          const int c = gtid + k * GT;
          if (c >= w0 && c < w0 + WCH && c < nch) {
            f32x4* cw = reinterpret_cast<f32x4*>(comb + (c - w0) * E);
            f32x4* pw = reinterpret_cast<f32x4*>(prow + c * E);
#pragma unroll
            for (int q = 0; q < E / 4; ++q) {
              f32x4 v{dw[k][4 * q], dw[k][4 * q + 1], dw[k][4 * q + 2], dw[k][4 * q + 3]};
              if (gi > 0) v = cw[q] + v;
              if (gi == RPB - 1)
                pw[q] = v;
              else
                cw[q] = v;
            }
          }
        }
      }
      __syncthreads();
    }
  }
}

// Scalar backward, dx only (one wave per row, two passes over the row).
template <int DT>
__global__ __launch_bounds__(kThreads) void rms_bwd_dx_scalar(
    const typename Elem<DT>::T* __restrict__ g, const typename Elem<DT>::T* __restrict__ x,
    const typename Elem<DT>::T* __restrict__ w, const float* __restrict__ rstd,
    typename Elem<DT>::T* __restrict__ dx, int64_t rows, int n) {
  using El = Elem<DT>;
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row = (int64_t)blockIdx.x * kWavesPerBlock + threadIdx.x / kWave;
  if (row >= rows) return;
  const int64_t base = row * (int64_t)n;
  const float r = rstd[row];
  float sdot = 0.f;
  for (int c = lane; c < n; c += kWave) {
    const float dn = El::round(El::load(g[base + c]) * El::load(w[c]));
    sdot += dn * El::load(x[base + c]);
  }
  sdot = wave_sum(sdot);
  const float r3 = r * r * r;
  const float sn = sdot * (1.0f / (float)n);
  for (int c = lane; c < n; c += kWave) {
    const float xf = El::load(x[base + c]);
    const float dn = El::round(El::load(g[base + c]) * El::load(w[c]));
    dx[base + c] = El::store(r * dn - (xf * r3) * sn);
  }
}

// Scalar dw partials: block (column tile, row chunk) -> part[row chunk][col].
template <int DT>
__global__ __launch_bounds__(kThreads) void rms_bwd_dw_scalar(const typename Elem<DT>::T* __restrict__ g,
                                                              const typename Elem<DT>::T* __restrict__ x,
                                                              const float* __restrict__ rstd,
                                                              float* __restrict__ part,
                                                              int64_t rows, int n, int64_t chunk) {
  const int col = blockIdx.x * kThreads + threadIdx.x;
  if (col >= n) return;
  const int64_t r0 = (int64_t)blockIdx.y * chunk;
  const int64_t r1 = r0 + chunk < rows ? r0 + chunk : rows;
  float acc = 0.f;
  for (int64_t r = r0; r < r1; ++r) {
    const int64_t i = r * n + col;
    acc += Elem<DT>::load(g[i]) * Elem<DT>::round(Elem<DT>::load(x[i]) * rstd[r]);
  }
  part[(int64_t)blockIdx.y * n + col] = acc;
}

// dw = column sums of the [R, n] fp32 partial rows (R <= 512), in fixed order, in one launch.
// Block = 64 columns (lane = column) and 16 waves: wave w adds rows w, w + 16, ... in order,
// then wave 0 adds the 16 wave sums in wave order and writes dtype DT. Each wave has at most
// 32 rows, all of whose loads it can have in flight.
template <int DT>
__global__ __launch_bounds__(kColsumWaves * kWave) void colsum(const float* __restrict__ in, int64_t R,
                                                               int n, typename Elem<DT>::T* __restrict__ out) {
  __shared__ float s[kColsumWaves][kWave];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int col = blockIdx.x * kWave + lane;
  float acc = 0.f;
  if (col < n) {
#pragma unroll 8
    for (int64_t r = wave; r < R; r += kColsumWaves) acc += in[r * n + col];
  }
  s[wave][lane] = acc;
  __syncthreads();
  if (wave == 0 && col < n) {
    float t = s[0][lane];
#pragma unroll
    for (int w = 1; w < kColsumWaves; ++w) t += s[w][lane];
    out[col] = Elem<DT>::store(t);
  }
}

bool vec_ok(int n, int e, std::initializer_list<const void*> ptrs) {
  if (n % e != 0) return false;
  for (const void* p : ptrs)
    if (!aligned16(p)) return false;
  return true;
}

template <int DT, int WPR, int VPT>
void launch_fwd(const void* x, const void* w, void* y, float* rstd, int64_t rows, int n, float eps,
                hipStream_t st) {
  using T = typename Elem<DT>::T;
  constexpr int RPB = kWavesPerBlock / WPR;
  const int64_t blocks = ceil_div(rows, RPB);
  hipLaunchKernelGGL((rms_fwd_vec<DT, WPR, VPT>), dim3((unsigned)blocks), dim3(kThreads), 0, st,
                     (const T*)x, (const T*)w, (T*)y, rstd, rows, n, eps);
}

template <int DT, int WPR, int VPT>
int64_t launch_bwd(const void* g, const void* x, const void* w, const float* rstd, void* dx,
                   float* part, int64_t rows, int n, hipStream_t st) {
  using T = typename Elem<DT>::T;
  constexpr int RPB = kWavesPerBlock / WPR;
  int64_t blocks = ceil_div(rows, RPB);
  if (blocks > kBwdMaxBlocks) blocks = kBwdMaxBlocks;
  hipLaunchKernelGGL((rms_bwd_vec<DT, WPR, VPT>), dim3((unsigned)blocks), dim3(kThreads), 0, st,
                     (const T*)g, (const T*)x, (const T*)w, rstd, (T*)dx, part, rows, n);
  return blocks;
}

// 16-byte chunks per lane for a row of nch chunks split over WPR waves, rounded
// up to a power of two (the instantiated counts).
int pick_vpt(int nch, int wpr) {
  const int need = (int)ceil_div(nch, (int64_t)wpr * kWave);
  int v = 1;
  while (v < need) v <<= 1;
  return v;
}

// Rows wider than 256 chunks (4 KiB) take a whole workgroup (4 waves): fewer
// registers per lane, more waves in flight.
int pick_wpr(int nch) { return nch <= 256 ? 1 : 4; }
// The backward holds w, its dw share and two rows of g and x per lane, so it
// spreads a row over more waves: 2 waves per row up to 512 chunks (4 chunks per
// lane, occupancy 2: at [32768, 4096] bf16 123 us against 136 us with 4 waves
// per row and 2 chunks per lane, whose per-row barrier then costs more than the
// registers save), 4 beyond.
int pick_wpr_bwd(int nch) { return nch <= 128 ? 1 : (nch <= 512 ? 2 : 4); }

// Rows per block of the scalar dw kernel: at least kScalarRowChunk, and few
// enough blocks that the partials stay within kBwdMaxBlocks rows.
int64_t scalar_chunk(int64_t rows) {
  const int64_t c = ceil_div(rows, kBwdMaxBlocks);
  return c > kScalarRowChunk ? c : kScalarRowChunk;
}

// Rows of partials the backward writes before the column sums (<= 512), for
// elements of e per chunk.
int64_t bwd_partial_rows(int64_t rows, int n, bool vec, int e) {
  if (vec) {
    const int64_t rpb = kWavesPerBlock / pick_wpr_bwd(n / e);
    const int64_t b = ceil_div(rows, rpb);
    return b < kBwdMaxBlocks ? b : kBwdMaxBlocks;
  }
  return ceil_div(rows, scalar_chunk(rows));
}

// The most any dtype and path needs, so the workspace size depends on neither.
int64_t bwd_partial_rows_max(int64_t rows, int n) {
  int64_t m = bwd_partial_rows(rows, n, false, 8);
  for (int e : {8, 4}) {
    const int64_t a = bwd_partial_rows(rows, n, true, e);
    if (a > m) m = a;
  }
  return m;
}

template <int DT>
int rmsnorm_fwd(const void* x, const void* w, void* y, float* rstd, int64_t rows, int n, float eps,
                hipStream_t st) {
  using T = typename Elem<DT>::T;
  constexpr int E = Elem<DT>::E;
  if (vec_ok(n, E, {x, w, y})) {
    const int nch = n / E;
    const int wpr = pick_wpr(nch);
    const int vpt = pick_vpt(nch, wpr);
#define KRSI_FWD_CASE(W, V)                                  \
  if (wpr == W && vpt == V) {                                \
    launch_fwd<DT, W, V>(x, w, y, rstd, rows, n, eps, st);   \
    return launch_status();                                  \
  }
    KRSI_FWD_CASE(1, 1) KRSI_FWD_CASE(1, 2) KRSI_FWD_CASE(1, 4)
    KRSI_FWD_CASE(4, 2) KRSI_FWD_CASE(4, 4) KRSI_FWD_CASE(4, 8)
#undef KRSI_FWD_CASE
    // Wider than 8 chunks per lane (fp32 rows above 8192): the scalar path.
  }
  hipLaunchKernelGGL((rms_fwd_scalar<DT>), dim3((unsigned)ceil_div(rows, kWavesPerBlock)),
                     dim3(kThreads), 0, st, (const T*)x, (const T*)w, (T*)y, rstd, rows, n, eps);
  return launch_status();
}

template <int DT>
int rmsnorm_bwd(const void* g, const void* x, const void* w, const float* rstd, void* dx, void* dw,
                void* workspace, int64_t rows, int n, hipStream_t st) {
  using T = typename Elem<DT>::T;
  constexpr int E = Elem<DT>::E;
  float* part = static_cast<float*>(workspace);
  int64_t p1 = 0;
  bool done = false;
  if (vec_ok(n, E, {g, x, w, dx})) {
    const int nch = n / E;
    const int wpr = pick_wpr_bwd(nch);
    const int vpt = pick_vpt(nch, wpr);
#define KRSI_BWD_CASE(W, V)                                                \
  if (!done && wpr == W && vpt == V) {                                     \
    p1 = launch_bwd<DT, W, V>(g, x, w, rstd, dx, part, rows, n, st);       \
    done = true;                                                           \
  }
    KRSI_BWD_CASE(1, 1) KRSI_BWD_CASE(1, 2) KRSI_BWD_CASE(2, 1) KRSI_BWD_CASE(2, 2)
    KRSI_BWD_CASE(2, 4) KRSI_BWD_CASE(4, 2) KRSI_BWD_CASE(4, 4) KRSI_BWD_CASE(4, 8)
#undef KRSI_BWD_CASE
  }
  if (!done) {
    hipLaunchKernelGGL((rms_bwd_dx_scalar<DT>), dim3((unsigned)ceil_div(rows, kWavesPerBlock)),
                       dim3(kThreads), 0, st, (const T*)g, (const T*)x, (const T*)w, rstd, (T*)dx,
                       rows, n);
    const int64_t chunk = scalar_chunk(rows);
    p1 = ceil_div(rows, chunk);
    hipLaunchKernelGGL((rms_bwd_dw_scalar<DT>), dim3((unsigned)ceil_div(n, kThreads), (unsigned)p1),
                       dim3(kThreads), 0, st, (const T*)g, (const T*)x, rstd, part, rows, n, chunk);
  }
  int rc = launch_status();
  if (rc != KRSI_OK) return rc;
  hipLaunchKernelGGL((colsum<DT>), dim3((unsigned)ceil_div(n, kWave)), dim3(kColsumWaves * kWave), 0, st,
                     (const float*)part, p1, (int)n, (T*)dw);
  return launch_status();
}

// dw of an empty batch is zero; one column-sum launch over zero rows writes it.
template <int DT>
int rmsnorm_bwd_empty(void* dw, int n, hipStream_t st) {
  using T = typename Elem<DT>::T;
  hipLaunchKernelGGL((colsum<DT>), dim3((unsigned)ceil_div(n, kWave)), dim3(kColsumWaves * kWave), 0, st,
                     (const float*)nullptr, (int64_t)0, (int)n, (T*)dw);
  return launch_status();
}

bool known_dtype(int32_t dt) { return dt == kBf16 || dt == kF16 || dt == kF32; }

// ------------------------------------------------- backward without allocation
// The partial-row workspace of the backward, as a device array the library owns, for callers
// that cannot allocate (code under HIP graph capture, serving loops that forbid hipMalloc). Every
// GPU the library runs on holds its own copy from load until the process ends. In host code the
// name `scratch` is only a stand-in for the symbol: its device address is looked up once per
// device with hipGetSymbolAddress, and only that address is ever passed to kernels.
constexpr size_t kScratchBytes = size_t(16) << 20;
__device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch[kMaxDevices] = {};

// This device's copy of `scratch` (current device), looked up on its first use.
int scratch_on_current_device(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return KRSI_ERR_LAUNCH;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return KRSI_ERR_LAUNCH;
    g_scratch[dev] = p;
  }
  *out = g_scratch[dev];
  return KRSI_OK;
}

}  // namespace

}  // namespace krsi

extern "C" {

size_t krsi_rmsnorm_bwd_workspace_bytes(int64_t rows, int32_t n) {
  using namespace krsi;
  if (rows <= 0 || n <= 0) return 0;
  return align256((size_t)bwd_partial_rows_max(rows, n) * n * sizeof(float));
}

int krsi_rmsnorm_fwd(const void* x, const void* w, void* y, float* rstd, int64_t rows, int32_t n,
                     float eps, int32_t dtype, void* stream) {
  using namespace krsi;
  if (!known_dtype(dtype)) return KRSI_ERR_UNSUPPORTED;
  if (rows < 0 || n <= 0 || n > 16384) return KRSI_ERR_BAD_SHAPE;
  if (!(eps == eps) || eps > 3.0e38f || eps < -3.0e38f) return KRSI_ERR_BAD_SCALE;
  if (rows == 0) return KRSI_OK;
  if (!x || !w || !y || !rstd) return KRSI_ERR_NULL_POINTER;
  hipStream_t st = as_stream(stream);
  switch (dtype) {
    case kF16:
      return rmsnorm_fwd<kF16>(x, w, y, rstd, rows, n, eps, st);
    case kF32:
      return rmsnorm_fwd<kF32>(x, w, y, rstd, rows, n, eps, st);
    default:
      return rmsnorm_fwd<kBf16>(x, w, y, rstd, rows, n, eps, st);
  }
}

int krsi_rmsnorm_bwd(const void* g, const void* x, const void* w, const float* rstd, void* dx,
                     void* dw, void* workspace, size_t workspace_bytes, int64_t rows, int32_t n,
                     int32_t dtype, void* stream) {
  using namespace krsi;
  if (!known_dtype(dtype)) return KRSI_ERR_UNSUPPORTED;
  if (rows < 0 || n <= 0 || n > 16384) return KRSI_ERR_BAD_SHAPE;
  if (!dw) return KRSI_ERR_NULL_POINTER;
  hipStream_t st = as_stream(stream);
  if (rows == 0) {
    switch (dtype) {
      case kF16:
        return rmsnorm_bwd_empty<kF16>(dw, n, st);
      case kF32:
        return rmsnorm_bwd_empty<kF32>(dw, n, st);
      default:
        return rmsnorm_bwd_empty<kBf16>(dw, n, st);
    }
  }
  if (!g || !x || !w || !rstd || !dx) return KRSI_ERR_NULL_POINTER;
  const size_t need = krsi_rmsnorm_bwd_workspace_bytes(rows, n);
  if (!workspace || workspace_bytes < need) return KRSI_ERR_WORKSPACE;
  if (!aligned16(workspace)) return KRSI_ERR_MISALIGNED;
  switch (dtype) {
    case kF16:
      return rmsnorm_bwd<kF16>(g, x, w, rstd, dx, dw, workspace, rows, n, st);
    case kF32:
      return rmsnorm_bwd<kF32>(g, x, w, rstd, dx, dw, workspace, rows, n, st);
    default:
      return rmsnorm_bwd<kBf16>(g, x, w, rstd, dx, dw, workspace, rows, n, st);
  }
}

int krsi_rmsnorm_bwd_noalloc(const void* g, const void* x, const void* w, const float* rstd, void* dx,
                             void* dw, int64_t rows, int32_t n, int32_t dtype, void* stream) {
  using namespace krsi;
  if (!known_dtype(dtype)) return KRSI_ERR_UNSUPPORTED;
  if (rows < 0 || n <= 0 || n > 16384) return KRSI_ERR_BAD_SHAPE;
  if (!dw) return KRSI_ERR_NULL_POINTER;
  if (rows > 0 && (!g || !x || !w || !rstd || !dx)) return KRSI_ERR_NULL_POINTER;
  const size_t need = krsi_rmsnorm_bwd_workspace_bytes(rows, n);
  if (need > kScratchBytes) return KRSI_ERR_TOO_LARGE;
  void* ws = nullptr;
  const int rc = scratch_on_current_device(&ws);
  if (rc != KRSI_OK) return rc;
  return krsi_rmsnorm_bwd(g, x, w, rstd, dx, dw, ws, kScratchBytes, rows, n, dtype, stream);
}

int krsi_rmsnorm_fwd_bf16(const void* x, const void* w, void* y, float* rstd, int64_t rows,
                          int32_t n, float eps, void* stream) {
  return krsi_rmsnorm_fwd(x, w, y, rstd, rows, n, eps, KRSI_DTYPE_BF16, stream);
}

int krsi_rmsnorm_bwd_bf16(const void* g, const void* x, const void* w, const float* rstd, void* dx,
                          void* dw, void* workspace, size_t workspace_bytes, int64_t rows,
                          int32_t n, void* stream) {
  return krsi_rmsnorm_bwd(g, x, w, rstd, dx, dw, workspace, workspace_bytes, rows, n,
                          KRSI_DTYPE_BF16, stream);
}

}  // extern "C"
