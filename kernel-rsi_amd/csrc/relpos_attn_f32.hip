// Relative-position-bias flash attention with fp32 activations, on fp32 MFMA
// (v_mfma_f32_32x32x2_f32).
//
// The semantics are those of the 16-bit kernels in relpos_attn.hip, and so of
// library/relpos_attention.py of the reference (kernel-rsi):
//   * :46 for the scores;
//   * :26-59 for the forward;
//   * :62-126 and :144-156 for the backward.
// With fp32 activations the reference rounds P and dS to fp32, which is no rounding at
// all (`p.to(v.dtype)`, :53; `ds.to(q.dtype)`, :92, :125). These kernels keep every
// product in fp32: gfx950 has no reduced-precision fp32 matrix path.
// Every product is one v_mfma_f32_32x32x2_f32 chain with fp32 accumulation.
//
// Layout (wave64, 32x32 output blocks; see mfma32x32x16 in krsi_device.h for D):
//   A operand: lane l holds A[m = l % 32][k = l / 32];
//   B operand: lane l holds B[k = l / 32][n = l % 32].
//   * Head-dim contractions (scores, dP) split D into two halves. Lane half g = l / 32 takes
//     d = g * D/2 + s at step s, for s < D/2, so each lane reads 4 consecutive d with one
//     128-bit load.
//   * Position contractions (P V, dS K, P^T dO, dS^T Q) take one register of the score
//     block per step. The score block's lane l holds positions 8 (r / 4) + 4 g + r % 4 in
//     register r. Step j pairs register j of the B operand with position 8 (j / 4) + 4 g + j % 4
//     of the A operand, so no register is moved between lanes.
//   * Streamed tiles (64 positions x D floats) are staged in LDS with a row stride of
//     32 DB + 4 floats. That stride puts the 16 rows of one 128-bit read phase on distinct bank
//     quads, and pads columns [D, 32 DB) with zeros for the 32-wide output blocks.
//   * Workgroup = 4 waves x 32 queries (forward, dQ) or keys (dK/dV), XCD-aware grid.
//   * The dpd partial rows use the 16-bit kernels' layout (one row of S + 128 diagonals per
//     128-key block), so relpos_dpd_reduce sums them the same way. In the dK/dV kernel the
//     workgroup writes its fp32 dS block [64 queries x 128 keys] to LDS each step. One thread
//     per diagonal then sums that diagonal in query order into a 256-slot ring. Diagonals that
//     can get no further contribution are stored to the partial row. The order is fixed, so
//     dpd is bitwise reproducible.
#include <math.h>

#include "krsi_device.h"
#include "krsi_internal.h"
#include "relpos_common.h"

namespace krsi {
namespace {

constexpr int kRowsF = 128;                 // queries (forward, dQ) or keys (dK/dV) per workgroup
constexpr int kStepF = 64;                  // streamed positions per step
constexpr int kThreadsF = 256;
constexpr int kWinF = kRowsF + kStepF - 1;  // bias-window entries of one step
static_assert(kRowsF == kKvRows, "the dpd partial rows are shared with the 16-bit kernels");

template <int DB>
struct GeoF {
  static constexpr int LD = 32 * DB + 4;  // LDS row stride of a staged tile, floats
  static constexpr int HM = 16 * DB;      // contraction steps per half, at most (D / 2 <= 16 DB)
  static constexpr int TILE = kStepF * LD;
};

__device__ __forceinline__ f32x16 mma(float a, float b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// (q.k scale + bias) in log2 units, rounded on its own: never fused with the subtraction of the
// running max (forward) or of lse (backward), so both passes form bitwise the same exponent
// argument (at S = 1, p is then exactly 1 in the backward, as in the forward).
__device__ __forceinline__ float log2_units(float t) {
#pragma clang fp contract(off)
  return t * kLog2e;
}

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int r = 0; r < 16; ++r) z[r] = 0.f;
  return z;
}

// One step's tile rows held in registers between their global loads and their LDS stores, so
// the loads of step t + 1 are in flight while step t computes. Thread t holds 16-byte chunks
// t, t + 256, ... of the tile (at most 2 DB of them: D <= 32 DB). The stored tile holds rows
// p0 .. p0 + 63 of the [S, D] slice at `base` (row stride ld floats), zero past S; columns
// [D, 32 DB) keep what zero_tile_pad wrote. Every load reads a valid address (the last row,
// masked, stands in for rows past S) so none waits behind a branch.
template <int DB>
struct TileRegs {
  static constexpr int CPT = 2 * DB;
  f32x4 v[CPT];
  __device__ __forceinline__ void load(const float* base, int64_t ld, int p0, int S, int D) {
    const int cpr = D >> 2, n = kStepF * cpr;
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int c = min((int)threadIdx.x + k * kThreadsF, n - 1);
      const int r = c / cpr, j = c - r * cpr;
      const bool ok = (int)threadIdx.x + k * kThreadsF < n && p0 + r < S;
      const int row = p0 + r < S ? p0 + r : S - 1;
      f32x4 x = *reinterpret_cast<const f32x4*>(base + (int64_t)row * ld + 4 * j);
      if (!ok) x = f32x4{0.f, 0.f, 0.f, 0.f};
      v[k] = x;
    }
  }
  __device__ __forceinline__ void store(float* tile, int D) const {
    const int cpr = D >> 2, n = kStepF * cpr;
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int c = threadIdx.x + k * kThreadsF;
      if (c < n) {
        const int r = c / cpr, j = c - r * cpr;
        *reinterpret_cast<f32x4*>(tile + r * GeoF<DB>::LD + 4 * j) = v[k];
      }
    }
  }
};

// Bias window entry x = threadIdx.x (x < kWinF): pd[h, wb + x], zero outside [0, 2S - 1), loaded
// into a register one step ahead.
__device__ __forceinline__ float window_entry(const float* pdh, int npd, int wb) {
  const int k = wb + (int)threadIdx.x;
  return (threadIdx.x < (unsigned)kWinF && k >= 0 && k < npd) ? pdh[k] : 0.f;
}
__device__ __forceinline__ void store_window(float* bw, float v) {
  if (threadIdx.x < (unsigned)kWinF) bw[threadIdx.x] = v;
}

template <int DB>
__device__ __forceinline__ void zero_tile_pad(float* tile, int D) {
  constexpr int LD = GeoF<DB>::LD;
  const int w = LD - D;
  for (int c = threadIdx.x; c < kStepF * w; c += kThreadsF) {
    const int r = c / w;
    tile[r * LD + D + (c - r * w)] = 0.f;
  }
}

// The lane's half of a row of D floats into registers: dst[s] = row[s] for s < ns = D / 2
// (row points at column g D/2), zero past ns or when !ok.
template <int DB>
__device__ __forceinline__ void load_half_row(float* dst, const float* row, int ns, bool ok) {
#pragma unroll
  for (int s = 0; s < GeoF<DB>::HM; s += 4) {
    f32x4 v = {0.f, 0.f, 0.f, 0.f};
    if (ok && s < ns) v = *reinterpret_cast<const f32x4*>(row + s);
#pragma unroll
    for (int e = 0; e < 4; ++e) dst[s + e] = v[e];
  }
}

// Head-dim contraction: acc += A B with A's row m = row `row0 + l32` of a staged tile and
// B's column n = the lane's register half `breg`.
template <int DB>
__device__ __forceinline__ f32x16 dot_rows(const float* tile, int row, int g, int ns, const float* breg,
                                           f32x16 acc) {
  const float* a = tile + row * GeoF<DB>::LD + g * ns;
#pragma unroll
  for (int s = 0; s < GeoF<DB>::HM; s += 4) {
    if (s < ns) {
      const f32x4 v = *reinterpret_cast<const f32x4*>(a + s);
#pragma unroll
      for (int e = 0; e < 4; ++e) acc = mma(v[e], breg[s + e], acc);
    }
  }
  return acc;
}

// Position contraction: acc[db] += sum over the 32 positions base + 8 (j / 4) + 4 g + j % 4 of
// tile[position][32 db + l32] * b[j]: output rows are head dims, columns the lane's own.
template <int DB>
__device__ __forceinline__ void dot_positions(const float* tile, int base, int g, int l32,
                                              const f32x16& b, f32x16* acc) {
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const float* rowp = tile + (base + 8 * (j >> 2) + 4 * g + (j & 3)) * GeoF<DB>::LD + l32;
#pragma unroll
    for (int db = 0; db < DB; ++db) acc[db] = mma(rowp[32 * db], b[j], acc[db]);
  }
}

// Store a 32x32-block accumulator column (head dims 32 db + 8 a + 4 g .. + 3 of this lane's
// position) times `mul` to row `dst` (16-byte aligned, D % 8 == 0).
template <int DB>
__device__ __forceinline__ void store_dims(float* dst, const f32x16* acc, float mul, int g, int D) {
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      const int d0 = 32 * db + 8 * a + 4 * g;
      if (d0 < D) {
        f32x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = acc[db][4 * a + e] * mul;
        *reinterpret_cast<f32x4*>(dst + d0) = v;
      }
    }
}

// -------------------------------------------------------------------- forward
template <int DB>
__global__ __launch_bounds__(kThreadsF) void relpos_fwd_f32_kernel(
    const float* __restrict__ qkv, int64_t ld, const float* __restrict__ pd, float* __restrict__ out,
    float* __restrict__ out32, float* __restrict__ lse, int S, int H, int D, float scale) {
  using G = GeoF<DB>;
  __shared__ __attribute__((aligned(16))) float Ks[G::TILE];
  __shared__ __attribute__((aligned(16))) float Vs[G::TILE];
  __shared__ float bw[kWinF];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, g = lane >> 5, l32 = lane & 31;
  const int nqb = (S + kRowsF - 1) / kRowsF;
  const int tile = xcd_tile(blockIdx.x, gridDim.x);
  const int bh = tile / nqb, b = bh / H, h = bh - b * H;
  const int i_wg = (tile - bh * nqb) * kRowsF;
  const int ii = wave * 32 + l32, qi = i_wg + ii;
  const bool qvalid = qi < S;
  const int ns = D >> 1;
  const int64_t HD = (int64_t)H * D;
  const float* q0 = qkv + (int64_t)b * S * ld + (int64_t)h * D;
  const int npd = 2 * S - 1;
  const float* pdh = pd + (int64_t)h * npd;

  float qr[G::HM];
  load_half_row<DB>(qr, q0 + (int64_t)(qvalid ? qi : 0) * ld + g * ns, ns, qvalid);
  zero_tile_pad<DB>(Ks, D);
  zero_tile_pad<DB>(Vs, D);
  f32x16 oacc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) oacc[db] = zero16();
  // The most negative finite float, not -inf: a step whose scores are all -inf (keys masked by
  // -inf bias entries) gives p = 0, not exp2(-inf - -inf) = NaN.
  float m_run = -3.40282347e+38f, l_run = 0.f;

  const int T = (S + kStepF - 1) / kStepF;
  const int wb0 = -i_wg - (kRowsF - 1) + S - 1;
  TileRegs<DB> kn, vn;
  kn.load(q0 + HD, ld, 0, S, D);
  vn.load(q0 + 2 * HD, ld, 0, S, D);
  float wn = window_entry(pdh, npd, wb0);
  for (int t = 0; t < T; ++t) {
    const int j0 = t * kStepF;
    __syncthreads();  // every wave is done with the previous step's tiles
    kn.store(Ks, D);
    vn.store(Vs, D);
    store_window(bw, wn);
    __syncthreads();
    if (t + 1 < T) {  // step t + 1's loads, in flight while step t computes
      kn.load(q0 + HD, ld, j0 + kStepF, S, D);
      vn.load(q0 + 2 * HD, ld, j0 + kStepF, S, D);
      wn = window_entry(pdh, npd, wb0 + j0 + kStepF);
    }
    // Scores in log2 units, (q.k scale + bias) log2(e), keys past S at -inf; exact running max.
    f32x16 sc[2];
    float mx = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      sc[kb] = dot_rows<DB>(Ks, kb * 32 + l32, g, ns, qr, zero16());
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int jj = kb * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
        // The window entry (index in [0, kWinF)) is read for every key, so the read does not
        // wait behind the key test; keys past S then take -inf.
        const float xv = log2_units(fmaf(sc[kb][r], scale, bw[jj - ii + kRowsF - 1]));
        const float x = j0 + jj < S ? xv : -INFINITY;
        sc[kb][r] = x;
        mx = fmaxf(mx, x);
      }
    }
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float m_new = fmaxf(m_run, mx);
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
    l_run *= alpha;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) oacc[db][r] *= alpha;
    m_run = m_new;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = __builtin_amdgcn_exp2f(sc[kb][r] - m_new);
        sc[kb][r] = p;
        l_run += p;
      }
      dot_positions<DB>(Vs, kb * 32, g, l32, sc[kb], oacc);
    }
  }
  const float l = l_run + __shfl_xor(l_run, 32);
  if (qvalid) {
    const int64_t ob = ((int64_t)b * S + qi) * HD + (int64_t)h * D;
    store_dims<DB>(out + ob, oacc, 1.f / l, g, D);
    if (out32 && out32 != out) store_dims<DB>(out32 + ob, oacc, 1.f / l, g, D);
    if (g == 0 && lse) lse[(int64_t)bh * S + qi] = m_run + log2f(l);
  }
}

// --------------------------------------------------------- backward: delta and dQ
// At head dims up to 64 the dQ kernel fits two waves per SIMD (256 registers each), which the
// bound keeps (grids of more than one workgroup per CU then overlap two).
template <int DB>
__global__ __launch_bounds__(kThreadsF, DB <= 2 ? 2 : 1) void relpos_bwd_dq_f32_kernel(
    const float* __restrict__ qkv, int64_t ld, const float* __restrict__ pd,
    const float* __restrict__ dout, const float* __restrict__ out32, const float* __restrict__ lse,
    float* __restrict__ delta_ws, float* __restrict__ dqkv, int64_t ldd, int S, int H, int D,
    float scale) {
  using G = GeoF<DB>;
  __shared__ __attribute__((aligned(16))) float Ks[G::TILE];
  __shared__ __attribute__((aligned(16))) float Vs[G::TILE];
  __shared__ float bw[kWinF];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, g = lane >> 5, l32 = lane & 31;
  const int nqb = (S + kRowsF - 1) / kRowsF;
  const int tile = xcd_tile(blockIdx.x, gridDim.x);
  const int bh = tile / nqb, b = bh / H, h = bh - b * H;
  const int i_wg = (tile - bh * nqb) * kRowsF;
  const int ii = wave * 32 + l32, qi = i_wg + ii;
  const bool qvalid = qi < S;
  const int ns = D >> 1;
  const int64_t HD = (int64_t)H * D;
  const float* q0 = qkv + (int64_t)b * S * ld + (int64_t)h * D;
  const int npd = 2 * S - 1;
  const float* pdh = pd + (int64_t)h * npd;

  float qr[G::HM], dr[G::HM];
  const int qs = qvalid ? qi : 0;
  load_half_row<DB>(qr, q0 + (int64_t)qs * ld + g * ns, ns, qvalid);
  const int64_t ob = ((int64_t)b * S + qs) * HD + (int64_t)h * D + g * ns;
  load_half_row<DB>(dr, dout + ob, ns, qvalid);
  float delta;
  {
    float o[G::HM];
    load_half_row<DB>(o, out32 + ob, ns, qvalid);
    float part = 0.f;
#pragma unroll
    for (int s = 0; s < G::HM; ++s) part = fmaf(dr[s], o[s], part);
    delta = part + __shfl_xor(part, 32);
  }
  if (qvalid && g == 0) delta_ws[(int64_t)bh * S + qi] = delta;
  // +inf makes p = exp2(x - lse) exactly 0 on query lanes past S.
  const float nlse = qvalid ? lse[(int64_t)bh * S + qi] : INFINITY;
  zero_tile_pad<DB>(Ks, D);
  zero_tile_pad<DB>(Vs, D);
  f32x16 dq[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) dq[db] = zero16();

  const int T = (S + kStepF - 1) / kStepF;
  const int wb0 = -i_wg - (kRowsF - 1) + S - 1;
  TileRegs<DB> kn, vn;
  kn.load(q0 + HD, ld, 0, S, D);
  vn.load(q0 + 2 * HD, ld, 0, S, D);
  float wn = window_entry(pdh, npd, wb0);
  for (int t = 0; t < T; ++t) {
    const int j0 = t * kStepF;
    __syncthreads();
    kn.store(Ks, D);
    vn.store(Vs, D);
    store_window(bw, wn);
    __syncthreads();
    if (t + 1 < T) {
      kn.load(q0 + HD, ld, j0 + kStepF, S, D);
      vn.load(q0 + 2 * HD, ld, j0 + kStepF, S, D);
      wn = window_entry(pdh, npd, wb0 + j0 + kStepF);
    }
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      f32x16 s = dot_rows<DB>(Ks, kb * 32 + l32, g, ns, qr, zero16());
      const f32x16 dp = dot_rows<DB>(Vs, kb * 32 + l32, g, ns, dr, zero16());
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int jj = kb * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
        // Computed for every key (the window read and exp2 do not wait behind the key test;
        // keys past S have zero K rows and window entries, so the value is finite) and then
        // dropped past S.
        const float pv = __builtin_amdgcn_exp2f(log2_units(fmaf(s[r], scale, bw[jj - ii + kRowsF - 1])) - nlse);
        const float p = j0 + jj < S ? pv : 0.f;
        s[r] = p * (dp[r] - delta);  // ds
      }
      dot_positions<DB>(Ks, kb * 32, g, l32, s, dq);
    }
  }
  if (qvalid) store_dims<DB>(dqkv + ((int64_t)b * S + qi) * ldd + (int64_t)h * D, dq, scale, g, D);
}

// ------------------------------------------------------ backward: dK, dV and dpd
template <int DB>
__global__ __launch_bounds__(kThreadsF) void relpos_bwd_dkdv_f32_kernel(
    const float* __restrict__ qkv, int64_t ld, const float* __restrict__ pd,
    const float* __restrict__ dout, const float* __restrict__ lse, const float* __restrict__ delta_ws,
    float* __restrict__ dqkv, int64_t ldd, float* __restrict__ part, int S, int H, int D, float scale,
    int kb0, int nkc) {
  using G = GeoF<DB>;
  // The dS block [query][key] sits at columns kStepF .. kStepF + kRowsF - 1 of rows of DSL
  // floats whose other columns stay zero, so every term of a diagonal sum below is a plain
  // load (a key outside the block reads +0, which leaves the sum bitwise unchanged).
  constexpr int DSL = kRowsF + 2 * kStepF;
  constexpr int RING = 256;        // > the 191 diagonals live across two steps
  __shared__ __attribute__((aligned(16))) float Qs[G::TILE];
  __shared__ __attribute__((aligned(16))) float Os[G::TILE];
  __shared__ float dsb[kStepF * DSL];
  __shared__ float ring[RING];
  __shared__ float bw[kWinF];
  __shared__ float Lq[kStepF], Dq[kStepF];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, g = lane >> 5, l32 = lane & 31;
  // Key blocks [kb0, kb0 + nkc) of every (batch, head).
  const int tile = xcd_tile(blockIdx.x, gridDim.x);
  const int bh = tile / nkc, b = bh / H, h = bh - b * H;
  const int kbl = tile - bh * nkc;
  const int j_wg = (kb0 + kbl) * kRowsF;
  const int kk = wave * 32 + l32, kj = j_wg + kk;
  const bool kvalid = kj < S;
  const int ns = D >> 1;
  const int64_t HD = (int64_t)H * D;
  const float* q0 = qkv + (int64_t)b * S * ld + (int64_t)h * D;
  const float* o0 = dout + (int64_t)b * S * HD + (int64_t)h * D;
  const int npd = 2 * S - 1;
  const float* pdh = pd + (int64_t)h * npd;
  const float* lse_bh = lse + (int64_t)bh * S;
  const float* dl_bh = delta_ws + (int64_t)bh * S;
  float* prow = part + ((int64_t)bh * nkc + kbl) * (S + kRowsF);
  const int rlen = S + kRowsF - 1;  // diagonals of the partial row

  float kr[G::HM], vr[G::HM];
  const int64_t krow = (int64_t)(kvalid ? kj : 0) * ld + g * ns;
  load_half_row<DB>(kr, q0 + HD + krow, ns, kvalid);
  load_half_row<DB>(vr, q0 + 2 * HD + krow, ns, kvalid);
  zero_tile_pad<DB>(Qs, D);
  zero_tile_pad<DB>(Os, D);
  for (int e = tid; e < RING; e += kThreadsF) ring[e] = 0.f;
  for (int e = tid; e < kStepF * 2 * kStepF; e += kThreadsF) {  // the zero margins of dsb
    const int row = e / (2 * kStepF), c = e - row * (2 * kStepF);
    dsb[row * DSL + (c < kStepF ? c : kRowsF + c)] = 0.f;
  }
  f32x16 dk[DB], dv[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) dk[db] = dv[db] = zero16();

  const int T = (S + kStepF - 1) / kStepF;
  // Window entry x = kk - iq + 63 holds pd[h, (j_wg + kk) - (i0 + iq) + S - 1].
  const int wb0 = j_wg - (kStepF - 1) + S - 1;
  TileRegs<DB> qn, on;
  qn.load(q0, ld, 0, S, D);
  on.load(o0, HD, 0, S, D);
  float wn = window_entry(pdh, npd, wb0);
  float ln = 0.f, dn = 0.f;  // lse and delta of query tid (threads tid < 64)
  auto stats = [&](int i0) {
    const int q = min(i0 + tid, S - 1);
    ln = lse_bh[q];
    dn = dl_bh[q];
  };
  stats(0);
  for (int t = 0; t < T; ++t) {
    const int i0 = t * kStepF;
    __syncthreads();
    qn.store(Qs, D);
    on.store(Os, D);
    store_window(bw, wn);
    if (tid < kStepF) {
      const bool ok = i0 + tid < S;
      Lq[tid] = ok ? ln : INFINITY;  // queries past S: p = 0
      Dq[tid] = ok ? dn : 0.f;
    }
    __syncthreads();
    if (t + 1 < T) {
      qn.load(q0, ld, i0 + kStepF, S, D);
      on.load(o0, HD, i0 + kStepF, S, D);
      wn = window_entry(pdh, npd, wb0 - i0 - kStepF);
      stats(i0 + kStepF);
    }
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      // S and dP [query][key]: rows are this step's queries, columns the lane's key.
      f32x16 p = dot_rows<DB>(Qs, qb * 32 + l32, g, ns, kr, zero16());
      f32x16 ds = dot_rows<DB>(Os, qb * 32 + l32, g, ns, vr, zero16());
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int iq = qb * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
        const float pv = __builtin_amdgcn_exp2f(log2_units(fmaf(p[r], scale, bw[kk - iq + kStepF - 1])) - Lq[iq]);
        // Keys past S have p != 0 (their bias is real) but no gradient: their dK and dV are
        // never stored and their dS is kept out of dpd.
        const float dd = Dq[iq];  // read for every lane, so it does not wait behind kvalid
        const float dsv = kvalid ? pv * (ds[r] - dd) : 0.f;
        p[r] = pv;
        ds[r] = dsv;
        dsb[iq * DSL + kStepF + kk] = dsv;
      }
      dot_positions<DB>(Os, qb * 32, g, l32, p, dv);   // dV^T += dO^T P
      dot_positions<DB>(Qs, qb * 32, g, l32, ds, dk);  // dK^T += Q^T dS
    }
    __syncthreads();
    // Local diagonal x = kk - iq + 63 of this step is partial-row entry R = x - 64 - i0 + S.
    if (tid < kWinF) {
      float acc = 0.f;
      // Column c = tid - 63 + iq of the block is entry kStepF + c of its row, in [1, 254].
#pragma unroll 16
      for (int iq = 0; iq < kStepF; ++iq) acc += dsb[iq * DSL + tid + 1 + iq];
      const int R = tid - kStepF - i0 + S;
      if (R >= 0) ring[R & (RING - 1)] += acc;
    }
    __syncthreads();
    // Later steps reach R <= S + 62 - i0 only: entries [S + 63 - i0, S + 126 - i0] are final.
    if (tid < kStepF) {
      const int R = S + (kStepF - 1) - i0 + tid;
      if (R >= 0 && R < rlen) {
        prow[R] = ring[R & (RING - 1)];
        ring[R & (RING - 1)] = 0.f;
      }
    }
  }
  __syncthreads();
  const int rmax = S + kStepF - 2 - kStepF * (T - 1);  // the rest: [0, rmax]
  for (int R = tid; R <= rmax; R += kThreadsF)
    if (R < rlen) prow[R] = ring[R & (RING - 1)];

  if (kvalid) {
    float* row = dqkv + ((int64_t)b * S + kj) * ldd + (int64_t)h * D;
    store_dims<DB>(row + HD, dk, scale, g, D);
    store_dims<DB>(row + 2 * HD, dv, 1.f, g, D);
  }
}

template <int DB>
void launch_fwd_f32(const float* qkv, int64_t ld, const float* pd, float* out, float* out32, float* lse,
                    int B, int S, int H, int D, float scale, hipStream_t st) {
  const dim3 grid((unsigned)(ceil_div(S, kRowsF) * B * H));
  hipLaunchKernelGGL((relpos_fwd_f32_kernel<DB>), grid, dim3(kThreadsF), 0, st, qkv, ld, pd, out, out32,
                     lse, S, H, D, scale);
}

template <int DB>
void launch_bwd_f32(const float* dout, const float* qkv, int64_t ld, const float* pd, const float* out32,
                    const float* lse, float* dqkv, int64_t ldd, float* dpd, float* delta, float* part,
                    int nkc, int B, int S, int H, int D, float scale, hipStream_t st) {
  const int nkb = (int)ceil_div(S, kRowsF);
  hipLaunchKernelGGL((relpos_bwd_dq_f32_kernel<DB>), dim3((unsigned)(nkb * B * H)), dim3(kThreadsF), 0, st, qkv,
                     ld, pd, dout, out32, lse, delta, dqkv, ldd, S, H, D, scale);
  // Key blocks in chunks of nkc (all of them with the full workspace); each chunk's partial
  // rows are summed into dpd before the next chunk overwrites them.
  for (int kb0 = 0; kb0 < nkb; kb0 += nkc) {
    const int n = min(nkc, nkb - kb0);
    hipLaunchKernelGGL((relpos_bwd_dkdv_f32_kernel<DB>), dim3((unsigned)(n * B * H)), dim3(kThreadsF), 0, st,
                       qkv, ld, pd, dout, lse, (const float*)delta, dqkv, ldd, part, S, H, D, scale, kb0, n);
    launch_dpd_reduce(part, dpd, B, S, H, kb0, n, kb0 > 0, st);
  }
}

}  // namespace

int relpos_fwd_f32(const float* qkv, int64_t ld, const float* pd, float* out, float* out32, float* lse,
                   int B, int S, int H, int D, float scale, hipStream_t st) {
  switch ((D + 31) / 32) {
    case 1: launch_fwd_f32<1>(qkv, ld, pd, out, out32, lse, B, S, H, D, scale, st); break;
    case 2: launch_fwd_f32<2>(qkv, ld, pd, out, out32, lse, B, S, H, D, scale, st); break;
    case 3: launch_fwd_f32<3>(qkv, ld, pd, out, out32, lse, B, S, H, D, scale, st); break;
    case 4: launch_fwd_f32<4>(qkv, ld, pd, out, out32, lse, B, S, H, D, scale, st); break;
    default: return KRSI_ERR_UNSUPPORTED;
  }
  return launch_status();
}

int relpos_bwd_f32(const float* dout, const float* qkv, int64_t ld, const float* pd, const float* out32,
                   const float* lse, float* dqkv, int64_t ldd, float* dpd, float* delta, float* part,
                   int nkc, int B, int S, int H, int D, float scale, hipStream_t st) {
#define KRSI_BWD_F32(DB_) \
  launch_bwd_f32<DB_>(dout, qkv, ld, pd, out32, lse, dqkv, ldd, dpd, delta, part, nkc, B, S, H, D, scale, st)
  switch ((D + 31) / 32) {
    case 1: KRSI_BWD_F32(1); break;
    case 2: KRSI_BWD_F32(2); break;
    case 3: KRSI_BWD_F32(3); break;
    case 4: KRSI_BWD_F32(4); break;
    default: return KRSI_ERR_UNSUPPORTED;
  }
#undef KRSI_BWD_F32
  return launch_status();
}

}  // namespace krsi
