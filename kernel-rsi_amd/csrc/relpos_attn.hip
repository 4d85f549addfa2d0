// Relative-position-bias flash attention (non-causal), forward and backward,
// for gfx950 on 16-bit MFMA (v_mfma_f32_32x32x16_bf16 or _f16, by the activation
// dtype DT), fp32 softmax. P and dS are rounded to DT before their products, as the
// reference rounds them to the dtype of v and q.
//
// Semantics follow library/relpos_attention.py of the reference (kernel-rsi):
//   s[i,j]   = (q_i . k_j * scale + pd[h, j - i + S - 1]) * log2(e)     (:46)
//   forward  : online softmax over key blocks with exp2, o = sum_j bf16(p_ij) v_j / l_i,
//              stored as bf16 and fp32, lse_i = m_i + log2(l_i)             (:26-59)
//   backward : delta_i = sum_d dO_id * O32_id                                (:144)
//              p = exp2(s - lse), dp = dO v^T, ds = p (dp - delta)          (:86-90, :121-124)
//              dV = bf16(p)^T dO, dK = scale * bf16(ds)^T q,
//              dQ = scale * bf16(ds) k                                       (:88-94, :125-126)
//              dpd[h, k] = sum over b, i, j with j - i + S - 1 = k of ds     (:154-156)
//
// Layout and tiling (MI355X-native, not the reference's):
//   * A wavefront owns 32 queries (forward, dQ) or 32 keys (dK/dV); a
//     workgroup of NW wavefronts owns 32*NW. The register-resident side (Q and
//     dO, or K and V) is loaded once from HBM with 128-bit loads straight into
//     MFMA operand registers.
//   * The streamed side (64 positions per step) is fetched with raw buffer
//     loads whose resource ends at the last valid row of the (batch, head), so
//     rows past S and head-dim padding read as zero in hardware with no
//     per-element mask; loads of step t+1 are issued before the MFMAs of step t.
//     It is staged in LDS row-major with 128-bit writes only. Products that
//     contract over the head dim read it with 128-bit row reads; products that
//     contract over positions read it with ds_read_b64_tr_b16, which returns,
//     per lane, 4 consecutive rows of one column of a 4x16 block, so no
//     transposed copy is ever written.
//   * Scores are computed transposed (S^T = K Q^T) in the forward and dQ
//     kernels, so each lane owns one query: the row max and row sum are in-lane
//     reductions plus one cross-half exchange, and lse/delta are registers.
//     The fp32 score tile is converted in place to the bf16 operand of the next
//     MFMA: registers 8u..8u+7 of half-wave g hold positions 16u + 4g + {0..3}
//     and 16u + 8 + 4g + {0..3}, exactly the two 4-row groups two transposed
//     reads return, so the K order of both operands agrees without shuffles.
//   * The bias is folded into the score MFMA: with c = |scale| log2(e) the
//     accumulator starts at pd * log2(e) / c and the exponent is one fma,
//     exp2(acc * c - m). A negative scale flips the sign bits of the
//     register-resident bf16 operand (exact); scale 0 zeroes it (c = 1).
//   * The Toeplitz bias of a (32*NW) x 64 tile is a window of consecutive table
//     entries, staged once per step in 4 copies shifted by one entry, so every
//     lane reads its 4 consecutive entries with one aligned 128-bit LDS read;
//     the copy placement puts the 16 lanes of one read phase on distinct banks.
//   * Online softmax keeps a running reference point m per query that trails
//     the running max by at most kRescaleSlack (2^8 in p): it moves, and the
//     fp32 accumulators are rescaled, only when a step's max exceeds it by more,
//     so p <= 2^8 and most steps rescale nothing. l and O are sums relative to m
//     and lse = m + log2 l is exact for any m. The row sum adds the fp32 p, as
//     the reference; the PV product takes p rounded to the activation dtype.
//   * dpd is reduced along the diagonals j - i inside the dK/dV kernel: each
//     (wave, half-wave) adds its fp32 ds into private LDS rings indexed by
//     diagonal, two diagonals per 64-bit read-modify-write. Within one
//     instruction the lanes of a ring hit distinct slots and a wave's LDS
//     operations complete in order, so the plain read-modify-write is exact and
//     deterministic. Diagonals that can get no further contribution are folded
//     in a fixed order into one partial row per key block; a last kernel sums
//     the partial rows over batch and key blocks in a fixed order. No
//     [B, H, S, S] buffer exists.
#include <math.h>

#include <type_traits>

#include "krsi_device.h"
#include "krsi_internal.h"
#include "relpos_common.h"

namespace krsi {
namespace {

constexpr int kStep = 64;  // streamed positions per iteration

constexpr int align_up(int x, int a) { return (x + a - 1) / a * a; }

// Start of the running max: the most negative finite float rather than -inf. A step whose
// scores are all -inf (keys masked by -inf entries of the bias table) then gives p = exp2(-inf)
// = 0 instead of exp2(-inf - -inf) = NaN; with any finite score the max, and every p, is the
// same as from -inf (alpha = exp2(-FLT_MAX - m) = 0 = exp2(-inf)).
constexpr float kMaxStart = -3.40282347e+38f;

// How far (log2 units) a step's max may exceed the forward's running reference point m before
// m moves and the accumulators are rescaled: p = exp2(s - m) <= 2^8, l <= 2^8 S.
constexpr float kRescaleSlack = 8.f;

// Compile-time buffer index and tail flag for the unrolled step loops.
constexpr std::integral_constant<int, 0> kBuf0{};
constexpr std::integral_constant<int, 1> kBuf1{};
constexpr std::integral_constant<bool, false> kFull{};
constexpr std::integral_constant<bool, true> kTail{};

template <int DP>
struct Geo {
  static constexpr int KS = DP / 16;         // K steps of 16 over the head dim
  static constexpr int DB = (DP + 31) / 32;  // 32-wide head-dim blocks of head-dim outputs
  static constexpr int DPV = DB * 32;        // staged row length (bf16), zero padded past DP
  static constexpr int CPR = DP / 8;         // 16-byte chunks per staged row
  static constexpr int NCH = kStep * CPR;    // chunks per streamed tile
};

template <int NW>
struct Blk {
  static constexpr int ROWS = 32 * NW;             // queries or keys per workgroup
  static constexpr int NT = 64 * NW;               // threads per workgroup
  static constexpr int WIN = ROWS + kStep;         // distinct window entries loaded
  static constexpr int WLD = ROWS + kStep + 16;    // bias copy stride, = 16 (mod 64) floats
  static constexpr int BPT = (WIN + NT - 1) / NT;  // window entries per thread
};

// Scale folding: scores are acc * c with acc = q'.k + pd * bmul, q' = (q & qand) ^ qxor
// on the register-resident bf16 operand.
struct Fold {
  float c;        // |scale| * log2(e), or 1 when scale == 0
  float bmul;     // log2(e) / c
  uint32_t qand;  // 0 when scale == 0
  uint32_t qxor;  // bf16 sign bits when scale < 0
};

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
typedef __attribute__((address_space(3))) void lds_void;

__device__ __forceinline__ u32x4 ld16(const uint16_t* p) { return *reinterpret_cast<const u32x4*>(p); }

__device__ __forceinline__ u32x4 fold_operand(u32x4 v, const Fold& f) {
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = (v[i] & f.qand) ^ f.qxor;
  return v;
}

// Raw buffer resources (gfx9 descriptor word 3): a load whose byte offset is at or
// past num_records returns zero. kOob is past every resource built here (the
// launchers keep them below 2^31 bytes).
typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr int kRsrcWord3 = 0x00020000;
constexpr uint32_t kOob = 0x80000000u;

// The whole byte offset must reach the instruction in the VGPR: the range check is
// made on the VGPR offset, so a constant the compiler split off into the immediate
// field would turn a valid offset whose variable part is negative into a zero read.
// An empty asm makes the offset opaque, so no constant can be split off.
__device__ __forceinline__ uint32_t opaque(uint32_t v) {
  asm volatile("" : "+v"(v));
  return v;
}

// Prologue loads of the register-resident operands: every lane loads (from `safe`, a valid
// address of the same buffer, where it has no data) and masks the value (lane_mask).
__device__ __forceinline__ u32x4 ld16_masked(const uint16_t* p, const uint16_t* safe, bool ok, uint32_t m) {
  return masked(ld16(ok ? p : safe), m);
}
__device__ __forceinline__ f32x4 ld16f_masked(const float* p, const float* safe, bool ok, uint32_t m) {
  return __builtin_bit_cast(f32x4, masked(*reinterpret_cast<const u32x4*>(ok ? p : safe), m));
}

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, kRsrcWord3);
}
__device__ __forceinline__ float bload4(rsrc_t r, uint32_t voff) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (int)voff, 0, 0));
}

// Staged tiles are row-major, DPV bf16 per row, with the 16-byte chunks of row r
// permuted by chunk j -> j ^ swz(r). With 64 LDS banks of 4 bytes (16 quads of 16 bytes)
// the permutation makes every access pattern of these kernels conflict-free:
//   * 128-bit row reads (16 lanes per cycle = 16 consecutive rows, one chunk),
//   * transposed 64-bit reads (32 lanes per cycle = 4 consecutive rows x 4 chunks),
//   * 128-bit staging writes of whole rows (DP a multiple of 32).
// swz only depends on bits 0-3 of r, so rows 16 apart share it.
template <int DPV>
__device__ __forceinline__ int swz(int r) {
  constexpr int C = DPV / 8;
  if constexpr (C == 8) return (((r >> 1) & 1) << 2) | ((r >> 2) & 3);
  else if constexpr (C == 16) return ((r & 3) << 2) | ((r >> 2) & 3);
  else return (r >> 2) & 3;  // C = 4 or 12: permute within aligned groups of 4 chunks
}
template <int DPV>
__device__ __forceinline__ int tile_off(int r, int j) { return r * DPV + 8 * (j ^ swz<DPV>(r)); }

// Per-lane element offsets into a staged tile, fixed for the kernel's life.
//   row[s]:    A/B operand of a product over the head dim: row l%32, columns 16s + 8(l/32) ..+7
//              (add base * DPV for rows base + l%32, base a multiple of 16).
//   tr[db][h]: transposed read for rows k + 8h + s/4, k = 16m + 4(l/32), s = l%16,
//              columns 32db + 16((l/16)%2) + 4(s%4) ..+3 (add 16m * DPV).
template <int DP>
struct TileLane {
  int row[Geo<DP>::KS];
  int tr[Geo<DP>::DB][2];
  __device__ __forceinline__ void init(int lane) {
    constexpr int DPV = Geo<DP>::DPV;
    const int l32 = lane & 31, g = lane >> 5, s = lane & 15;
#pragma unroll
    for (int k = 0; k < Geo<DP>::KS; ++k) row[k] = tile_off<DPV>(l32, 2 * k + g);
#pragma unroll
    for (int db = 0; db < Geo<DP>::DB; ++db)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int r = 4 * g + 8 * h + (s >> 2);
        const int j = 4 * db + 2 * ((lane >> 4) & 1) + ((s & 3) >> 1);
        tr[db][h] = tile_off<DPV>(r, j) + 4 * (s & 1);
      }
  }
};

// MFMA operand whose 8 K values are rows [k, k+4) and [k+8, k+12) (k = 16m + 4(l/32))
// of column 32db + l%32 of a staged tile: two ds_read_b64_tr_b16, in each of which lane
// s of a 16-lane group supplies the address of row (k + s/4), columns 4(s%4)..+3 of its
// 16-column block, and receives 4 consecutive rows of its own column.
template <int DP>
__device__ __forceinline__ u32x4 tr_operand(const uint16_t* tile, const TileLane<DP>& L, int m, int db) {
  const uint16_t* t = tile + 16 * m * Geo<DP>::DPV;
  const s16x4 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(t + L.tr[db][0]));
  const s16x4 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(t + L.tr[db][1]));
  const uint2 ua = __builtin_bit_cast(uint2, a), ub = __builtin_bit_cast(uint2, b);
  return u32x4{ua.x, ua.y, ub.x, ub.y};
}

// 128-bit row read of the operand for head-dim step s: rows base + l%32.
template <int DP>
__device__ __forceinline__ u32x4 row_operand(const uint16_t* tile, const TileLane<DP>& L, int base, int s) {
  return ld16(tile + base * Geo<DP>::DPV + L.row[s]);
}

// Lane l gets max / sum of x over lanes l % 32 and l % 32 + 32 (v_permlane32_swap_b32
// exchanges the upper half of its first operand with the lower half of its second). The
// builtin, unlike inline asm, leaves the scheduler free to move LDS accesses across it, and
// the compiler inserts the VALU-write -> permlane-read wait itself.
__device__ __forceinline__ void xhalf_pair(float x, float& a, float& b) {
  const unsigned u = __builtin_bit_cast(unsigned, x);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  a = __builtin_bit_cast(float, (unsigned)r[0]);
  b = __builtin_bit_cast(float, (unsigned)r[1]);
}
__device__ __forceinline__ float xhalf_max(float x) {
  float a, b;
  xhalf_pair(x, a, b);
  return fmaxf(a, b);
}
__device__ __forceinline__ float xhalf_sum(float x) {
  float a, b;
  xhalf_pair(x, a, b);
  return a + b;
}

// Streamed tiles go straight from HBM into LDS (buffer_load_dwordx4 ... lds): lane l of
// a wave writes the 16 bytes it loads to M0 + 16 l, so a wave fills 64 consecutive
// 16-byte chunks of the staged tile. Group k of thread t fills LDS chunk p = k NT + t,
// which is position p % C of staged row p / C (C = DPV / 8 chunks per row), so it loads
// logical chunk (p % C) ^ swz(row) of that row. Chunks past D (the zero padding up to DPV)
// get kOob and land as zeros, as do rows past S (the resource ends at row S - 1).
template <int DP, int NT>
struct Dma {
  static constexpr int C = Geo<DP>::DPV / 8;
  static constexpr int NCHV = kStep * C;                // 16-byte chunks per staged tile
  static constexpr int GPT = (NCHV + NT - 1) / NT;      // chunks per thread per tile
  static_assert(NCHV % 64 == 0, "a wave fills whole 64-chunk runs");
};

// tid: the thread's index within the NT threads that share the tile (threadIdx.x unless a
// workgroup stages several tiles with separate thread groups).
template <int DP, int NT>
__device__ __forceinline__ void dma_offsets(uint32_t* voff, int64_t ld, int D, int tid) {
  constexpr int C = Dma<DP, NT>::C;
#pragma unroll
  for (int k = 0; k < Dma<DP, NT>::GPT; ++k) {
    const int p = min(k * NT + tid, Dma<DP, NT>::NCHV - 1);  // past the tile: unused
    const int row = p / C;
    const int j = (p - row * C) ^ swz<Geo<DP>::DPV>(row);
    voff[k] = opaque(8 * j < D ? (uint32_t)(row * ld + 8 * j) * 2u : kOob);
  }
}

// One buffer_load_dwordx4 ... lds. It is issued from asm on purpose: the compiler treats
// the builtin form as an LDS write of unknown extent and waits for it before every later
// LDS read, which would complete each step's prefetch before that step's own compute.
// Invisible to the compiler, the request stays in flight until the kernel's explicit
// wait (drain_and_sync) at the top of the step that reads it; the compiler's own vmcnt
// waits only ever over-wait because of it.
__device__ __forceinline__ void dma16(rsrc_t r, uint32_t voff, uint32_t m0) {
  asm volatile("buffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(voff), "s"(r), "{m0}"(m0) : "memory");
}

// Rows p0..p0+63 of the [S, D] slice whose row 0 is `origin` (row stride ld) into the
// staged tile at `tile`, asynchronously (vmcnt): wait and barrier before reading it.
template <int DP, int NT>
__device__ __forceinline__ void dma_offsets(uint32_t* voff, int64_t ld, int D) {
  dma_offsets<DP, NT>(voff, ld, D, (int)threadIdx.x);
}

// w: the wave's index within the thread group (wave-uniform).
template <int DP, int NT>
__device__ __forceinline__ void dma_tile(uint16_t* tile, const uint32_t* voff, const uint16_t* origin,
                                         int64_t ld, int p0, int S, int D, int w) {
  const rsrc_t r = make_rsrc(origin + (int64_t)p0 * ld, (uint32_t)(((int64_t)(S - 1 - p0) * ld + D) * 2));
#pragma unroll
  for (int k = 0; k < Dma<DP, NT>::GPT; ++k)
    if (Dma<DP, NT>::NCHV % NT == 0 || k * NT + 64 * w < Dma<DP, NT>::NCHV)
      dma16(r, voff[k], (uint32_t)(uintptr_t)(lds_void*)(tile + (k * NT + 64 * w) * 8));
}
template <int DP, int NT>
__device__ __forceinline__ void dma_tile(uint16_t* tile, const uint32_t* voff, const uint16_t* origin,
                                         int64_t ld, int p0, int S, int D) {
  dma_tile<DP, NT>(tile, voff, origin, ld, p0, S, D, __builtin_amdgcn_readfirstlane(threadIdx.x >> 6));
}

// Wait for this thread's outstanding loads (the tile DMA among them) and LDS operations,
// then synchronise the workgroup.
__device__ __forceinline__ void drain_and_sync() {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
}

// Bias window entry x (0 <= x < WIN) holds T[wb + sgn * x] * bmul, zero outside
// [0, 2S - 1) (out-of-range offsets, negative ones included, fall past the
// resource); it is stored at position x + cc of copy cc. The raw entries are loaded
// one step ahead and scaled only when stashed, so nothing waits on the load (or on
// the tile DMA issued next to it) before the step that consumes it.
template <int NW>
__device__ __forceinline__ void load_bias(float* regs, const float* pdh, int npd, int wb, int sgn,
                                          int tid = -1) {
  using K = Blk<NW>;
  const rsrc_t r = make_rsrc(pdh, (uint32_t)npd * 4u);
  if (tid < 0) tid = threadIdx.x;
#pragma unroll
  for (int k = 0; k < K::BPT; ++k) {
    const int x = tid + k * K::NT;
    regs[k] = bload4(r, opaque(x < K::WIN ? (uint32_t)(wb + sgn * x) * 4u : kOob));
  }
}

// Copy cc starts at cc * WLD, copy 0 at 4: with WLD = 16 (mod 64) the 16 lanes of one
// 128-bit read phase (16 consecutive rows or columns, i.e. 16 consecutive x0) hit 16
// distinct bank quads.
template <int NW>
__device__ __forceinline__ constexpr int copy_base(int cc) { return cc == 0 ? 4 : cc * Blk<NW>::WLD; }

template <int NW>
__device__ __forceinline__ void stash_bias(const float* regs, float* bw, float bmul, int tid = -1) {
  using K = Blk<NW>;
  if (tid < 0) tid = threadIdx.x;
#pragma unroll
  for (int k = 0; k < K::BPT; ++k) {
    const int x = tid + k * K::NT;
    if (x < K::WIN) {
      const float v = regs[k] * bmul;
#pragma unroll
      for (int cc = 0; cc < 4; ++cc) bw[copy_base<NW>(cc) + x + cc] = v;
    }
  }
}

// The 16 bias values of one 32x32 D tile, as the tile's initial accumulator:
// window entries x0 + 8a + b (a, b = 0..3), read from the copy that makes x0
// 16-byte aligned.
template <int NW>
__device__ __forceinline__ f32x16 read_bias16(const float* bw, int x0) {
  const int cc = (-x0) & 3;
  const float* p = bw + copy_base<NW>(cc) + x0 + cc;
  f32x16 out;
#pragma unroll
  for (int a = 0; a < 4; ++a) {
    const f32x4 v = *reinterpret_cast<const f32x4*>(p + 8 * a);
#pragma unroll
    for (int b = 0; b < 4; ++b) out[4 * a + b] = v[b];
  }
  return out;
}

// ------------------------------------------------------------------- forward
// One 64-key step of the forward for this lane's query: scores (bias folded into
// the accumulator), running reference point m, p = exp2(acc c - m), l += p (fp32, as the
// reference's row sum, relpos_attention.py:51), O^T += V^T P^T with P rounded to the
// activation dtype. TAIL masks keys >= S (last step only).
template <int DT, int DP, int NW, bool TAIL>
__device__ __forceinline__ void fwd_step(const uint16_t* Ks, const uint16_t* Vs, const float* Bw,
                                         const TileLane<DP>& L, const u32x4* qreg, f32x16* oacc,
                                         float& m_run, float* l_run, int j0, int S, int ii, int g,
                                         float c) {
  using G = Geo<DP>;
  using K = Blk<NW>;
  f32x16 sc[2];
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
    sc[kb] = read_bias16<NW>(Bw, kb * 32 + 4 * g + (K::ROWS - 1) - ii);
#pragma unroll
    for (int s = 0; s < G::KS; ++s) sc[kb] = mfma32x32x16<DT>(row_operand<DP>(Ks, L, kb * 32, s), qreg[s], sc[kb]);
  }
  if (TAIL) {
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        if (j0 + kb * 32 + 8 * (r >> 2) + 4 * g + (r & 3) >= S) sc[kb][r] = -INFINITY;
  }
  float mx = fmaxf(sc[0][0], sc[1][0]);
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int r = 1; r < 16; ++r) mx = fmaxf(mx, sc[kb][r]);
  mx = xhalf_max(mx) * c;
  // The reference moves m to the exact running max every step (relpos_attention.py:48-50).
  // Here m moves only when the step's max exceeds it by more than kRescaleSlack, so p stays
  // below 2^kRescaleSlack (bf16 and fp16 hold it, rounded relative to its own magnitude as
  // any p) and the accumulators are rescaled on few steps: at config 5 the exact max moves
  // in about three steps of four, each rescale ~36 VALU instructions.
  const bool need = mx > m_run + kRescaleSlack;
  if (__any(need)) {
    const float mnew = need ? mx : m_run;
    const float alpha = __builtin_amdgcn_exp2f(m_run - mnew);
    l_run[0] *= alpha;
    l_run[1] *= alpha;
#pragma unroll
    for (int db = 0; db < G::DB; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) oacc[db][r] *= alpha;
    m_run = mnew;
  }
  const float negm = -m_run;
  // The softmax below (exp, row sum, packing) is the VALU-bound part of the step: raised wave
  // priority lets this wave's VALU work issue ahead of other waves' while their MFMAs run
  // (-1.9 % forward at config 5; priority 2 or 3, or raising it before the row max, the same
  // or slower).
  __builtin_amdgcn_s_setprio(1);
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
    float p[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) p[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[kb][r], c, negm));
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const u32x4 pb = Elem<DT>::pack(&p[8 * u]);
#pragma unroll
      for (int w = 0; w < 8; ++w) l_run[w & 1] += p[8 * u + w];
#pragma unroll
      for (int db = 0; db < G::DB; ++db)
        oacc[db] = mfma32x32x16<DT>(tr_operand<DP>(Vs, L, 2 * kb + u, db), pb, oacc[db]);
    }
  }
  __builtin_amdgcn_s_setprio(0);
}

// O = acc / l stored as fp32 and in the activation dtype (head-dim columns 32db + 8a + 4g
// ..+3 of this lane's query), lse = m + log2 l. out32 and lse_q are null together when the
// caller wants O only (no backward to follow): then only O in the activation dtype is stored.
template <int DT, int DP>
__device__ __forceinline__ void fwd_store(const f32x16* oacc, float m_run, const float* l_run,
                                          bool qvalid, int g, int64_t obase, int D,
                                          uint16_t* __restrict__ out, float* __restrict__ out32,
                                          float* __restrict__ lse_q) {
  const float l = xhalf_sum(l_run[0] + l_run[1]);
  if (!qvalid) return;
#pragma unroll
  for (int db = 0; db < Geo<DP>::DB; ++db)
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      const int d0 = db * 32 + 8 * a + 4 * g;
      if (d0 < D) {
        f32x4 o;
#pragma unroll
        for (int b4 = 0; b4 < 4; ++b4) o[b4] = oacc[db][4 * a + b4] / l;
        if (out32) *reinterpret_cast<f32x4*>(out32 + obase + d0) = o;
        uint2 ob;
        ob.x = Elem<DT>::pack2(o[0], o[1]);
        ob.y = Elem<DT>::pack2(o[2], o[3]);
        *reinterpret_cast<uint2*>(out + obase + d0) = ob;
      }
    }
  if (g == 0 && lse_q) *lse_q = m_run + log2f(l);
}

// Staged stores. A wave's transposed accumulators (lane l32 holds row l32; register 4a + b4 of
// block db holds column 32db + 8a + 4g + b4) go through a wave-private LDS tile `wt` (32 rows x
// kStoreLd floats), one 32-column block at a time, so each global store instruction writes whole
// row segments (8 lanes per 128-byte fp32 row block, 4 lanes per 64-byte 16-bit one) instead of
// 16 or 8 bytes in each of 32 rows. Every lane of the wave must call them; rows >= nrows are not
// stored. row0: element offset of the wave's first row; rstride: row stride in elements.
constexpr int kStoreLd = 36;  // tile row stride in floats: 16 rows of one column hit 16 bank quads
constexpr int kWaveTile = 32 * kStoreLd;  // floats per wave
template <int DT, int DP, bool W32, typename Op>
__device__ __forceinline__ void store_rows_staged(const f32x16* acc, Op op, int lane, int nrows, int64_t row0,
                                                  int64_t rstride, int D, uint16_t* __restrict__ out,
                                                  float* __restrict__ out32, float* wt, int db_lo = 0,
                                                  int db_hi = Geo<DP>::DB) {
  const int g = lane >> 5, l32 = lane & 31;
#pragma unroll
  for (int db = 0; db < Geo<DP>::DB; ++db) {
    const int ncol = min(32, D - 32 * db);  // a multiple of 8
    if (ncol <= 0) break;
    if (db < db_lo || db >= db_hi) continue;  // wave-uniform
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      f32x4 o;
#pragma unroll
      for (int b4 = 0; b4 < 4; ++b4) o[b4] = op(acc[db][4 * a + b4]);
      *reinterpret_cast<f32x4*>(wt + l32 * kStoreLd + 8 * a + 4 * g) = o;
    }
    // Other lanes' values are read back: keep every tile write of this block before the reads
    // (the LDS executes one wave's operations in order).
    asm volatile("" ::: "memory");
    if (W32 && out32) {
#pragma unroll
      for (int k = 0; k < 4; ++k) {  // fp32: 32 rows x 8 chunks of 4
        const int c = lane + 64 * k, r = c >> 3, j = c & 7;
        if (r < nrows && 4 * j < ncol)
          *reinterpret_cast<f32x4*>(out32 + row0 + r * rstride + 32 * db + 4 * j) =
              *reinterpret_cast<const f32x4*>(wt + r * kStoreLd + 4 * j);
      }
    }
#pragma unroll
    for (int k = 0; k < 2; ++k) {  // activation dtype: 32 rows x 4 chunks of 8
      const int c = lane + 64 * k, r = c >> 2, j = c & 3;
      if (r < nrows && 8 * j < ncol) {
        const f32x4 x = *reinterpret_cast<const f32x4*>(wt + r * kStoreLd + 8 * j);
        const f32x4 y = *reinterpret_cast<const f32x4*>(wt + r * kStoreLd + 8 * j + 4);
        const u32x4 v = {Elem<DT>::pack2(x[0], x[1]), Elem<DT>::pack2(x[2], x[3]), Elem<DT>::pack2(y[0], y[1]),
                         Elem<DT>::pack2(y[2], y[3])};
        *reinterpret_cast<u32x4*>(out + row0 + r * rstride + 32 * db + 8 * j) = v;
      }
    }
    asm volatile("" ::: "memory");  // the next block's writes after these reads
  }
}

// Forward outputs: O = acc / l (fp32 and the activation dtype), lse = m + log2 l.
template <int DT, int DP>
__device__ __forceinline__ void fwd_store_staged(const f32x16* oacc, float m_run, const float* l_run,
                                                 int lane, int nrows, int64_t row0, int64_t HD, int D,
                                                 uint16_t* __restrict__ out, float* __restrict__ out32,
                                                 float* __restrict__ lse_q, float* wt, int db_lo = 0,
                                                 int db_hi = Geo<DP>::DB) {
  const float l = xhalf_sum(l_run[0] + l_run[1]);
  if (lse_q && (lane >> 5) == 0 && (lane & 31) < nrows) *lse_q = m_run + log2f(l);
  store_rows_staged<DT, DP, true>(oacc, [l](float x) { return x / l; }, lane, nrows, row0, HD, D, out, out32,
                                  wt, db_lo, db_hi);
}

// At head dims 49-64 (DP = 64) the forward runs 4 waves per SIMD (128 VGPRs; spills only in the
// prologue and the last step): more waves give one wave's VALU softmax more MFMA work of the
// others to overlap with (-2% at config 5 against 3 waves).
template <int DT, int DP, int NW>
__global__ __launch_bounds__(64 * NW, (DP == 64 ? 4 : 2)) void relpos_fwd_kernel(
    const uint16_t* __restrict__ qkv, int64_t ld, const float* __restrict__ pd,
    uint16_t* __restrict__ out, float* __restrict__ out32, float* __restrict__ lse, int S, int H,
    int D, Fold f) {
  using G = Geo<DP>;
  using K = Blk<NW>;
  constexpr int TILE = kStep * G::DPV;
  constexpr int BWIN = 4 * K::WLD;
  // K tiles, then V tiles (one array, so the output staging can reuse all of it).
  __shared__ __attribute__((aligned(16))) uint16_t KVs[4 * TILE];
  __shared__ __attribute__((aligned(16))) float Bw[2 * BWIN];
  uint16_t* const Ks = KVs;
  uint16_t* const Vs = KVs + 2 * TILE;

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, g = lane >> 5, l32 = lane & 31;
  TileLane<DP> L;
  L.init(lane);
  const int nqb = (S + K::ROWS - 1) / K::ROWS;
  const int tile = xcd_tile(blockIdx.x, gridDim.x);
  const int bh = tile / nqb, b = bh / H, h = bh - b * H;
  const int qb = tile - bh * nqb;
  const int i_wg = qb * K::ROWS;
  const int ii = wave * 32 + l32;
  const int qi = i_wg + ii;
  const bool qvalid = qi < S;
  const int64_t tok0 = (int64_t)b * S;
  const int64_t HD = (int64_t)H * D;
  const uint16_t* q0 = qkv + tok0 * ld + (int64_t)h * D;  // row 0 of this (batch, head)'s Q
  const uint16_t* k0p = q0 + HD;
  const uint16_t* v0p = q0 + 2 * HD;
  const int npd = 2 * S - 1;
  const float* pdh = pd + (int64_t)h * npd;
  const float c = f.c;

  u32x4 qreg[G::KS];
#pragma unroll
  for (int s = 0; s < G::KS; ++s) {
    const int d0 = 16 * s + 8 * g;
    const bool ok = qvalid && d0 < D;
    qreg[s] = masked(fold_operand(ld16(ok ? q0 + (int64_t)qi * ld + d0 : q0), f), lane_mask(ok));
  }

  f32x16 oacc[G::DB];
#pragma unroll
  for (int db = 0; db < G::DB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) oacc[db][r] = 0.f;
  float m_run = kMaxStart, l_run[2] = {0.f, 0.f};

  uint32_t voff[Dma<DP, K::NT>::GPT];
  dma_offsets<DP, K::NT>(voff, ld, D);
  float bst[K::BPT];
  const int T = (S + kStep - 1) / kStep;
  // Window base of step t: entry x is table index wb + x, wb = j0 - i_wg - (ROWS-1) + S-1.
  const int wb0 = S - 1 - i_wg - (K::ROWS - 1);
  dma_tile<DP, K::NT>(Ks, voff, k0p, ld, 0, S, D);
  dma_tile<DP, K::NT>(Vs, voff, v0p, ld, 0, S, D);
  load_bias<NW>(bst, pdh, npd, wb0, 1);

  // Step t computes from buffer t & 1, requested one step earlier. The one barrier per
  // step publishes that buffer and retires every wave's reads of the other one (step t-1),
  // which the requests for step t+1 then overwrite.
  auto step = [&](int t, auto buf, auto tail) {
    constexpr int B = decltype(buf)::value;
    stash_bias<NW>(bst, Bw + B * BWIN, f.bmul);
    drain_and_sync();
    if (t + 1 < T) {
      const int j1 = (t + 1) * kStep;
      dma_tile<DP, K::NT>(Ks + (1 - B) * TILE, voff, k0p, ld, j1, S, D);
      dma_tile<DP, K::NT>(Vs + (1 - B) * TILE, voff, v0p, ld, j1, S, D);
      load_bias<NW>(bst, pdh, npd, wb0 + j1, 1);
    }
    fwd_step<DT, DP, NW, decltype(tail)::value>(Ks + B * TILE, Vs + B * TILE, Bw + B * BWIN, L, qreg, oacc,
                                            m_run, l_run, t * kStep, S, ii, g, c);
  };
  // Full 64-key steps carry no key mask; a partial last step (S % 64 != 0) runs once after
  // the loop. The loop is unrolled by two so every buffer offset is a constant.
  const int Tfull = S / kStep;
  int t = 0;
  for (; t + 1 < Tfull; t += 2) {
    step(t, kBuf0, kFull);
    step(t + 1, kBuf1, kFull);
  }
  if (t < Tfull) step(t++, kBuf0, kFull);
  if (t < T) {
    if (t & 1)
      step(t, kBuf1, kTail);
    else
      step(t, kBuf0, kTail);
  }

  if constexpr (NW * kWaveTile * 4 <= (int)sizeof(KVs)) {
    __syncthreads();  // every wave is done with the last tiles
    fwd_store_staged<DT, DP>(oacc, m_run, l_run, lane, min(32, S - (i_wg + wave * 32)),
                             (tok0 + i_wg + wave * 32) * HD + (int64_t)h * D, HD, D, out, out32,
                             (lse ? lse + (int64_t)bh * S + qi : nullptr), reinterpret_cast<float*>(KVs) + wave * kWaveTile);
  } else {
    fwd_store<DT, DP>(oacc, m_run, l_run, qvalid, g, (tok0 + qi) * HD + (int64_t)h * D, D, out, out32,
                      (lse ? lse + (int64_t)bh * S + qi : nullptr));
  }
}

// ------------------------------------------- forward, keys split inside the workgroup
// For grids too small to give every SIMD more than one wave (fewer than two workgroups of
// relpos_fwd_kernel per CU): a workgroup of 8 waves owns the same 128 queries; waves 0-3
// stream key steps [0, T - T1) and waves 4-7 steps [T - T1, T), T1 = ceil(T / 2), each group
// with its own staged tiles and bias windows and the same step code as relpos_fwd_kernel.
// Both groups pass the same T1 barriers (group 0 idles in its last iteration when T is odd);
// only group 1's last step can be partial, and it runs in the last iteration. At
// the end group 1 hands its running max, row sum and accumulators to group 0 through LDS,
// which merges them: m = max(m0, m1), x = x0 2^(m0 - m) + x1 2^(m1 - m) for l and O. Each
// half keeps its own running reference point, so p of the second half is rounded relative to
// that half's reference point rather than to one carried over all earlier keys.
// WIDE: the grid has at most one workgroup per CU, so nothing is gained by leaving registers for
// a second one (at D 49-64: 172 VGPRs and no spills, against 128 and 72 bytes spilled).
template <int DT, int DP, bool WIDE>
__global__ __launch_bounds__(512, (!WIDE && (DP == 64 || DP <= 32) ? 4 : 2)) void relpos_fwd_ks_kernel(
    const uint16_t* __restrict__ qkv, int64_t ld, const float* __restrict__ pd,
    uint16_t* __restrict__ out, float* __restrict__ out32, float* __restrict__ lse, int S, int H,
    int D, Fold f) {
  constexpr int NW = 4;  // waves per key group
  using G = Geo<DP>;
  using K = Blk<NW>;
  constexpr int TILE = kStep * G::DPV;
  constexpr int BWIN = 4 * K::WLD;
  constexpr int GRP_HALVES = 2 * TILE;  // one group's double-buffered tile, in uint16
  // K tiles of both groups, then V tiles of both groups; reused for the hand-over at the end.
  __shared__ __attribute__((aligned(16))) uint16_t stage[4 * GRP_HALVES];
  __shared__ __attribute__((aligned(16))) float Bw[2 * 2 * BWIN];
  uint16_t* const Ks = stage;
  uint16_t* const Vs = stage + 2 * GRP_HALVES;

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, g = lane >> 5, l32 = lane & 31;
  const int grp = __builtin_amdgcn_readfirstlane(wave >> 2);
  const int gw = __builtin_amdgcn_readfirstlane(wave & 3);  // wave within the group
  const int gtid = threadIdx.x & (K::NT - 1);
  TileLane<DP> L;
  L.init(lane);
  const int nqb = (S + K::ROWS - 1) / K::ROWS;
  const int tile = xcd_tile(blockIdx.x, gridDim.x);
  const int bh = tile / nqb, b = bh / H, h = bh - b * H;
  const int qb = tile - bh * nqb;
  const int i_wg = qb * K::ROWS;
  const int ii = gw * 32 + l32;
  const int qi = i_wg + ii;
  const bool qvalid = qi < S;
  const int64_t tok0 = (int64_t)b * S;
  const int64_t HD = (int64_t)H * D;
  const uint16_t* q0 = qkv + tok0 * ld + (int64_t)h * D;
  const uint16_t* k0p = q0 + HD;
  const uint16_t* v0p = q0 + 2 * HD;
  const int npd = 2 * S - 1;
  const float* pdh = pd + (int64_t)h * npd;
  const float c = f.c;
  uint16_t* Kg = Ks + grp * GRP_HALVES;
  uint16_t* Vg = Vs + grp * GRP_HALVES;
  float* Bg = Bw + grp * 2 * BWIN;

  u32x4 qreg[G::KS];
#pragma unroll
  for (int s = 0; s < G::KS; ++s) {
    const int d0 = 16 * s + 8 * g;
    const bool ok = qvalid && d0 < D;
    qreg[s] = masked(fold_operand(ld16(ok ? q0 + (int64_t)qi * ld + d0 : q0), f), lane_mask(ok));
  }
  f32x16 oacc[G::DB];
#pragma unroll
  for (int db = 0; db < G::DB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) oacc[db][r] = 0.f;
  float m_run = kMaxStart, l_run[2] = {0.f, 0.f};

  uint32_t voff[Dma<DP, K::NT>::GPT];
  dma_offsets<DP, K::NT>(voff, ld, D, gtid);
  float bst[K::BPT];
  const int T = (S + kStep - 1) / kStep;
  const int T1 = (T + 1) / 2;
  const int tbeg = grp == 0 ? 0 : T - T1;      // this group's first step
  const int tend = grp == 0 ? T - T1 : T;      // one past its last
  const int wb0 = S - 1 - i_wg - (K::ROWS - 1);
  if (tbeg < tend) {
    dma_tile<DP, K::NT>(Kg, voff, k0p, ld, tbeg * kStep, S, D, gw);
    dma_tile<DP, K::NT>(Vg, voff, v0p, ld, tbeg * kStep, S, D, gw);
    load_bias<NW>(bst, pdh, npd, wb0 + tbeg * kStep, 1, gtid);
  }

  // Iteration it handles step tbeg + it of this group from buffer it & 1 (requested one
  // iteration earlier); the barrier (shared by both groups) publishes it and retires every
  // wave's reads of the other buffer.
  auto step = [&](int it, auto buf, auto tail) {
    constexpr int B = decltype(buf)::value;
    const int t = tbeg + it;
    const bool live = t < tend;
    if (live) stash_bias<NW>(bst, Bg + B * BWIN, f.bmul, gtid);
    drain_and_sync();
    if (t + 1 < tend) {
      const int j1 = (t + 1) * kStep;
      dma_tile<DP, K::NT>(Kg + (1 - B) * TILE, voff, k0p, ld, j1, S, D, gw);
      dma_tile<DP, K::NT>(Vg + (1 - B) * TILE, voff, v0p, ld, j1, S, D, gw);
      load_bias<NW>(bst, pdh, npd, wb0 + j1, 1, gtid);
    }
    if (live)
      fwd_step<DT, DP, NW, decltype(tail)::value>(Kg + B * TILE, Vg + B * TILE, Bg + B * BWIN, L, qreg,
                                                  oacc, m_run, l_run, t * kStep, S, ii, g, c);
  };
  // Every step before the last iteration is full; the last may hold group 1's partial step.
  int it = 0;
  for (; it + 2 < T1; it += 2) {
    step(it, kBuf0, kFull);
    step(it + 1, kBuf1, kFull);
  }
  if (it + 1 < T1) {
    step(it, kBuf0, kFull);
    step(it + 1, kBuf1, kTail);
  } else {
    step(it, kBuf0, kTail);
  }

  // Hand-over through the (now idle) tile buffers, at [wave-in-group][slot][lane] so every
  // access is one coalesced row. With more than one 32-column block the two groups split the
  // merge and the store: group 0 takes blocks [0, DB0) and lse, group 1 blocks [DB0, DB), each
  // handing the other its m, its l and the accumulator blocks the other stores. Both compute
  // m = max(m0, m1), x = x0 2^(m0 - m) + x1 2^(m1 - m) with the same operations in the same
  // order, so the outputs are those of a single merge.
  constexpr int DB = G::DB;
  constexpr int DB0 = DB > 1 ? (DB + 1) / 2 : DB;
  constexpr int SENT = DB0 > DB - DB0 ? DB0 : DB - DB0;  // blocks one wave hands over, at most
  constexpr int SLOTS = 2 + 16 * SENT;
  static_assert((DB > 1 ? 8 : 4) * SLOTS * 64 * 4 <= (int)sizeof(stage), "the hand-over fits the tile buffers");
  static_assert(32 * kStoreLd <= SLOTS * 64, "the staging tile fits a wave's hand-over rows");
  // Group 1 writes region [gw] (read by group 0), group 0 region [4 + gw].
  float* const sent = reinterpret_cast<float*>(stage) + ((grp == 1 ? 0 : 4) + gw) * SLOTS * 64 + lane;
  float* const got = reinterpret_cast<float*>(stage) + ((grp == 1 ? 4 : 0) + gw) * SLOTS * 64 + lane;
  __syncthreads();
  if (grp == 1 || DB > 1) {
    const int lo = grp == 1 ? 0 : DB0, hi = grp == 1 ? DB0 : DB;  // blocks the other group stores
    sent[0] = m_run;
    sent[64] = l_run[0] + l_run[1];
#pragma unroll
    for (int db = 0; db < DB; ++db)
      if (db >= lo && db < hi)
#pragma unroll
        for (int r = 0; r < 16; ++r) sent[(2 + 16 * (db - lo) + r) * 64] = oacc[db][r];
  }
  __syncthreads();
  if (grp == 0 || DB > 1) {
    const int lo = grp == 0 ? 0 : DB0, hi = grp == 0 ? DB0 : DB;  // blocks this group stores
    const float mo = got[0], lo_l = got[64];
    const float m0 = grp == 0 ? m_run : mo, m1 = grp == 0 ? mo : m_run;
    const float l0 = grp == 0 ? l_run[0] + l_run[1] : lo_l, l1 = grp == 0 ? lo_l : l_run[0] + l_run[1];
    const float m = fmaxf(m0, m1);
    const float a0 = __builtin_amdgcn_exp2f(m0 - m);
    const float a1 = __builtin_amdgcn_exp2f(m1 - m);  // 0 when group 1 saw no finite score
    const float lm[2] = {l0 * a0 + l1 * a1, 0.f};
#pragma unroll
    for (int db = 0; db < DB; ++db)
      if (db >= lo && db < hi)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float xo = got[(2 + 16 * (db - lo) + r) * 64];
          const float x0 = grp == 0 ? oacc[db][r] : xo, x1 = grp == 0 ? xo : oacc[db][r];
          oacc[db][r] = x0 * a0 + x1 * a1;
        }
    // The wave's received rows, all read above, become its output staging tile.
    asm volatile("" ::: "memory");
    fwd_store_staged<DT, DP>(oacc, m, lm, lane, min(32, S - (i_wg + gw * 32)),
                             (tok0 + i_wg + gw * 32) * HD + (int64_t)h * D, HD, D, out, out32,
                             (lse && grp == 0 ? lse + (int64_t)bh * S + qi : nullptr), got - lane, lo, hi);
  }
}

// ------------------------------------------------ backward: delta, dQ and dpd
// One 64-key step of the dQ kernel for this lane's query: p = exp2(acc c - lse),
// ds = p (dp - delta), dQ^T += K^T dS^T. The dP accumulator starts from negd, a register
// block holding -delta, so ds = p dP needs no subtract (16 VGPRs for the kernel's life:
// 2 waves per SIMD instead of 3, and -1.2% backward at config 5, -4 to -6% at S <= 2048).
// Invalid query lanes carry lse = +inf, so their p is 0 without a mask; TAIL masks keys
// >= S (last step only).
template <int DT, int DP, int NW, bool TAIL>
__device__ __forceinline__ void dq_step(const uint16_t* Ks, const uint16_t* Vs, const float* Bw,
                                        const TileLane<DP>& L, const u32x4* qreg, const u32x4* doreg,
                                        f32x16* dq, float neg_lse, const f32x16& negd, int j0, int S, int ii,
                                        int g, float c) {
  using G = Geo<DP>;
  using K = Blk<NW>;
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
    const int x0 = kb * 32 + 4 * g + (K::ROWS - 1) - ii;
    f32x16 acc = read_bias16<NW>(Bw, x0), accp;
#pragma unroll
    for (int s = 0; s < G::KS; ++s) {
      acc = mfma32x32x16<DT>(row_operand<DP>(Ks, L, kb * 32, s), qreg[s], acc);
      accp = mfma32x32x16<DT>(row_operand<DP>(Vs, L, kb * 32, s), doreg[s], s == 0 ? negd : accp);
    }
    float ds[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      float p = __builtin_amdgcn_exp2f(__builtin_fmaf(acc[r], c, neg_lse));
      if (TAIL && j0 + kb * 32 + 8 * (r >> 2) + 4 * g + (r & 3) >= S) p = 0.f;
      ds[r] = p * accp[r];
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const u32x4 dsb = Elem<DT>::pack(&ds[8 * u]);
#pragma unroll
      for (int db = 0; db < G::DB; ++db)
        dq[db] = mfma32x32x16<DT>(tr_operand<DP>(Ks, L, 2 * kb + u, db), dsb, dq[db]);
    }
  }
}

// LDS of the dQ kernel: the K tiles, then the V tiles (one array, so the dQ staging can reuse
// all of it), then the bias windows; each region 256-byte aligned.
template <int DP, int NW>
struct DqLds {
  static constexpr int TILE = kStep * Geo<DP>::DPV;
  static constexpr int KV_BYTES = 4 * TILE * 2;
  static constexpr int BW_OFF = align_up(KV_BYTES, 256);
  static constexpr int BYTES = BW_OFF + 2 * 4 * Blk<NW>::WLD * 4;
};

// The dQ kernel's work for query block `tile` (of the grid's B H ceil(S / 128)), with its LDS
// at `lds` (DqLds). DELTA_GIVEN: delta is read from delta_ws (written by relpos_delta_kernel)
// rather than formed from dO and O32 and written there.
template <int DT, int DP, int NW, bool DELTA_GIVEN>
__device__ __forceinline__ void bwd_dq_body(
    int tile, unsigned char* lds, const uint16_t* __restrict__ qkv, int64_t ld, const float* __restrict__ pd,
    const uint16_t* __restrict__ dout, const float* __restrict__ out32,
    const float* __restrict__ lse, float* __restrict__ delta_ws, uint16_t* __restrict__ dqkv,
    int64_t ldd, int S, int H, int D, Fold f, float scale) {
  using G = Geo<DP>;
  using K = Blk<NW>;
  constexpr int TILE = kStep * G::DPV;
  constexpr int BWIN = 4 * K::WLD;
  uint16_t* const KVs = reinterpret_cast<uint16_t*>(lds);
  float* const Bw = reinterpret_cast<float*>(lds + DqLds<DP, NW>::BW_OFF);
  uint16_t* const Ks = KVs;
  uint16_t* const Vs = KVs + 2 * TILE;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, g = lane >> 5, l32 = lane & 31;
  TileLane<DP> L;
  L.init(lane);
  const int nqb = (S + K::ROWS - 1) / K::ROWS;
  const int bh = tile / nqb, b = bh / H, h = bh - b * H;
  const int qb = tile - bh * nqb;
  const int i_wg = qb * K::ROWS;
  const int ii = wave * 32 + l32;
  const int qi = i_wg + ii;
  const bool qvalid = qi < S;
  const int64_t tok0 = (int64_t)b * S;
  const int64_t HD = (int64_t)H * D;
  const uint16_t* q0 = qkv + tok0 * ld + (int64_t)h * D;
  const uint16_t* k0p = q0 + HD;
  const uint16_t* v0p = q0 + 2 * HD;
  const int npd = 2 * S - 1;
  const float* pdh = pd + (int64_t)h * npd;
  const float c = f.c;


  // Register-resident operands and per-query statistics.
  u32x4 qreg[G::KS], doreg[G::KS];
  float dsum = 0.f;
  const int64_t obase = (tok0 + qi) * HD + (int64_t)h * D;
#pragma unroll
  for (int s = 0; s < G::KS; ++s) {
    const int d0 = 16 * s + 8 * g;
    const bool ok = qvalid && d0 < D;
    const uint32_t m = lane_mask(ok);
    qreg[s] = masked(fold_operand(ld16(ok ? q0 + (int64_t)qi * ld + d0 : q0), f), m);
    doreg[s] = ld16_masked(dout + obase + d0, dout, ok, m);
    if constexpr (!DELTA_GIVEN) {
      const f32x4 o0 = ld16f_masked(out32 + obase + d0, out32, ok, m);
      const f32x4 o1 = ld16f_masked(out32 + obase + d0 + 4, out32, ok, m);
      float df[8];
      Elem<DT>::unpack(doreg[s], df);
#pragma unroll
      for (int e = 0; e < 4; ++e) dsum += df[e] * o0[e];
#pragma unroll
      for (int e = 0; e < 4; ++e) dsum += df[4 + e] * o1[e];
    }
  }
  const float delta = DELTA_GIVEN ? (qvalid ? delta_ws[(int64_t)bh * S + qi] : 0.f) : xhalf_sum(dsum);
  f32x16 negd;
#pragma unroll
  for (int r = 0; r < 16; ++r) negd[r] = -delta;
  // -inf makes p = exp2(acc c - lse) exactly 0 on lanes past S (their acc is finite).
  const float neg_lse = qvalid ? -lse[(int64_t)bh * S + qi] : -INFINITY;
  if (!DELTA_GIVEN && qvalid && g == 0) delta_ws[(int64_t)bh * S + qi] = delta;

  f32x16 dq[G::DB];
#pragma unroll
  for (int db = 0; db < G::DB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) dq[db][r] = 0.f;

  uint32_t voff[Dma<DP, K::NT>::GPT];
  dma_offsets<DP, K::NT>(voff, ld, D);
  float bst[K::BPT];
  const int T = (S + kStep - 1) / kStep;
  const int wb0 = S - 1 - i_wg - (K::ROWS - 1);
  dma_tile<DP, K::NT>(Ks, voff, k0p, ld, 0, S, D);
  dma_tile<DP, K::NT>(Vs, voff, v0p, ld, 0, S, D);
  load_bias<NW>(bst, pdh, npd, wb0, 1);

  // Step t computes from buffer t & 1 (requested one step earlier); the barrier publishes
  // it and retires every wave's reads of the other buffer.
  auto step = [&](int t, auto buf, auto tail) {
    constexpr int B = decltype(buf)::value;
    stash_bias<NW>(bst, Bw + B * BWIN, f.bmul);
    drain_and_sync();
    if (t + 1 < T) {
      const int j1 = (t + 1) * kStep;
      dma_tile<DP, K::NT>(Ks + (1 - B) * TILE, voff, k0p, ld, j1, S, D);
      dma_tile<DP, K::NT>(Vs + (1 - B) * TILE, voff, v0p, ld, j1, S, D);
      load_bias<NW>(bst, pdh, npd, wb0 + j1, 1);
    }
    dq_step<DT, DP, NW, decltype(tail)::value>(Ks + B * TILE, Vs + B * TILE, Bw + B * BWIN, L, qreg, doreg,
                                           dq, neg_lse, negd, t * kStep, S, ii, g, c);
  };
  // Full 64-key steps carry no key mask; a partial last step runs once after the loop.
  const int Tfull = S / kStep;
  int t = 0;
  for (; t + 1 < Tfull; t += 2) {
    step(t, kBuf0, kFull);
    step(t + 1, kBuf1, kFull);
  }
  if (t < Tfull) step(t++, kBuf0, kFull);
  if (t < T) {
    if (t & 1)
      step(t, kBuf1, kTail);
    else
      step(t, kBuf0, kTail);
  }

  if constexpr (NW * kWaveTile * 4 <= DqLds<DP, NW>::KV_BYTES) {
    __syncthreads();  // every wave is done with the last tiles
    store_rows_staged<DT, DP, false>(dq, [scale](float x) { return x * scale; }, lane,
                                     min(32, S - (i_wg + wave * 32)), (tok0 + i_wg + wave * 32) * ldd + (int64_t)h * D,
                                     ldd, D, dqkv, nullptr, reinterpret_cast<float*>(KVs) + wave * kWaveTile);
  } else if (qvalid) {
    const int64_t qbase = (tok0 + qi) * ldd + (int64_t)h * D;
#pragma unroll
    for (int db = 0; db < G::DB; ++db)
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const int d0 = db * 32 + 8 * a + 4 * g;
        if (d0 < D) {
          uint2 ob;
          ob.x = Elem<DT>::pack2(dq[db][4 * a] * scale, dq[db][4 * a + 1] * scale);
          ob.y = Elem<DT>::pack2(dq[db][4 * a + 2] * scale, dq[db][4 * a + 3] * scale);
          *reinterpret_cast<uint2*>(dqkv + qbase + d0) = ob;
        }
      }
  }
}

template <int DT, int DP, int NW>
__global__ __launch_bounds__(64 * NW, (DP <= 96 ? 2 : 1)) void relpos_bwd_dq_kernel(
    const uint16_t* __restrict__ qkv, int64_t ld, const float* __restrict__ pd,
    const uint16_t* __restrict__ dout, const float* __restrict__ out32,
    const float* __restrict__ lse, float* __restrict__ delta_ws, uint16_t* __restrict__ dqkv,
    int64_t ldd, int S, int H, int D, Fold f, float scale) {
  __shared__ __attribute__((aligned(256))) unsigned char lds[DqLds<DP, NW>::BYTES];
  bwd_dq_body<DT, DP, NW, false>(xcd_tile(blockIdx.x, gridDim.x), lds, qkv, ld, pd, dout, out32, lse, delta_ws,
                                 dqkv, ldd, S, H, D, f, scale);
}

// ---------------------------------------------------------- backward: dK, dV, dpd
// dpd is reduced along the diagonals inside the dK/dV kernel, in LDS, with no [B,H,S,S]
// buffer. The workgroup diagonal of key kk (key j_wg + kk) and query i is
// r = kk - i + S - 1 (dpd index r + j_wg, 0 <= r < S + ROWS - 1). In a step, register pair
// p of row group a of query block qb holds ds at the consecutive diagonals r_s, r_s + 1
// with r_s = r0 - d, r0 = kk + S - 2 - 4g - 64t, d = 8a + 32qb + 2p, so one 64-bit
// read-modify-write adds both. Each (wave, half-wave) owns 2 ring copies and key kk uses
// copy k = (kk + S) & 1: within one instruction the lanes of a copy are 2 apart in kk and
// hit disjoint slot pairs, and a wave's LDS operations complete in order, so the plain
// read-modify-write is exact and deterministic (LDS float atomics are ~30x slower here).
// Copy k keeps diagonal r at slot (r - k) & 255, or 256 above it: the pair of r_s starts
// at slot ((r0 - k - 58) & 255) + 58 - d, which is even (r_s - k is) and never wraps. A
// step touches 191 diagonals and the 64 that can get no further contribution are folded
// at the next step into one partial row per key block, so at most 255 are live: distinct
// mod 256. The fold reads and clears both slots of a copy with one read2st64/write2st64.
// Bank rules measured on gfx950: b64 reads are served 32 lanes at a time over 64 banks,
// b64 writes 16 lanes at a time over 32 banks, b32 accesses 32 lanes at a time over 32
// banks. Column l of the wave's score tile holds key kperm(l) = 2 (l % 16) + l / 16, so a
// 16-lane write phase touches one copy only (32 contiguous floats); copy 1 sits 32 (S even)
// or 34 (S odd) floats past a 64-float boundary, which puts the two copies of a 32-lane
// read phase on distinct banks; the copies of (wave, half) index wg are skewed by 4 wg
// floats, which puts the 32 lanes of one fold phase (8 diagonals x 4 rings) on distinct
// banks.
constexpr int kRingSlots = 576;  // floats per ring copy (>= 512 + 34 + 28, a multiple of 64)
__device__ __forceinline__ int ring_base(int wg, int k, int off1) {
  return (2 * wg + k) * kRingSlots + 4 * wg + (k ? off1 : 0);
}
__device__ __forceinline__ int kperm(int l) { return 2 * (l & 15) + (l >> 4); }

// Staged store of a dK or dV accumulator (lane l32 holds head dim 32db + l32; register r holds
// tile row 8(r/4) + 4g + r%4, i.e. key kperm(row) of the wave): each 32-column block goes into
// the wave-private tile `wt` as [key][dim] (32 consecutive floats per half-wave write: no bank
// conflict), then whole row segments are stored, 4 lanes per 64-byte row block, instead of one
// 16-bit value per lane. Rows (keys) >= nrows are not stored. Every lane of the wave must call it.
constexpr int kColLd = 40;                // tile row stride in floats
constexpr int kColTile = 32 * kColLd;     // floats per wave
template <int DT, int DP, typename Op>
__device__ __forceinline__ void store_cols_staged(const f32x16* acc, Op op, int lane, int nrows, int64_t row0,
                                                  int64_t rstride, int D, uint16_t* __restrict__ out, float* wt) {
  const int g = lane >> 5, l32 = lane & 31;
#pragma unroll
  for (int db = 0; db < Geo<DP>::DB; ++db) {
    const int ncol = min(32, D - 32 * db);  // a multiple of 8
    if (ncol <= 0) break;
#pragma unroll
    for (int r = 0; r < 16; ++r) wt[kperm(8 * (r >> 2) + 4 * g + (r & 3)) * kColLd + l32] = op(acc[db][r]);
    asm volatile("" ::: "memory");  // the writes before the other lanes' reads
#pragma unroll
    for (int k = 0; k < 2; ++k) {  // 32 rows x 4 chunks of 8
      const int c = lane + 64 * k, r = c >> 2, j = c & 3;
      if (r < nrows && 8 * j < ncol) {
        const f32x4 x = *reinterpret_cast<const f32x4*>(wt + r * kColLd + 8 * j);
        const f32x4 y = *reinterpret_cast<const f32x4*>(wt + r * kColLd + 8 * j + 4);
        const u32x4 v = {Elem<DT>::pack2(x[0], x[1]), Elem<DT>::pack2(x[2], x[3]), Elem<DT>::pack2(y[0], y[1]),
                         Elem<DT>::pack2(y[2], y[3])};
        *reinterpret_cast<u32x4*>(out + row0 + r * rstride + 32 * db + 8 * j) = v;
      }
    }
    asm volatile("" ::: "memory");  // the next block's writes after these reads
  }
}

__device__ __forceinline__ float quad_sum(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, true));
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, true));
  return v;
}

// Fold diagonal r >= 0 out of the rings (4 lanes per diagonal, lane part = tid % 4 takes
// the rings of (wave, half) 2 part and 2 part + 1) and clear its slots; every lane of the
// quad returns the same fixed-order sum. All reads are issued before the clears.
__device__ __forceinline__ float ring_fold(float* ring, int r, int off1) {
  const int part = threadIdx.x & 3;
  float* pa[4];
#pragma unroll
  for (int e = 0; e < 4; ++e)
    pa[e] = ring + ring_base(2 * part + (e >> 1), e & 1, off1) + ((r - (e & 1)) & 255);
  float x[8];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    x[2 * e] = pa[e][0];
    x[2 * e + 1] = pa[e][256];
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) pa[e][0] = pa[e][256] = 0.f;
  float v = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) v += x[e];
  return quad_sum(v);
}
// LDS of the dK/dV kernel, each region 256-byte aligned: the dpd rings, a sink for the ds of
// keys past S, the Q and dO tiles, the step's -lse and -delta windows, the bias windows.
template <int DP, int NW>
struct DkdvLds {
  static constexpr int TILE = kStep * Geo<DP>::DPV;
  static constexpr int RINGF = 2 * 2 * NW * kRingSlots;
  static constexpr int RING_OFF = 0;
  static constexpr int SINK_OFF = align_up(RING_OFF + RINGF * 4, 256);
  static constexpr int QS_OFF = align_up(SINK_OFF + 320 * 4, 256);
  static constexpr int TILES_BYTES = 2 * TILE * 2;  // one double-buffered tile array
  static constexpr int OS_OFF = align_up(QS_OFF + TILES_BYTES, 256);
  static constexpr int LQ_OFF = align_up(OS_OFF + TILES_BYTES, 256);
  static constexpr int DQ_OFF = align_up(LQ_OFF + 2 * kStep * 4, 256);
  static constexpr int BW_OFF = align_up(DQ_OFF + 2 * kStep * 4, 256);
  static constexpr int BYTES = BW_OFF + 2 * 4 * Blk<NW>::WLD * 4;
};

// The dK/dV kernel's work for key block `tile`, with its LDS at `lds` (DkdvLds).
template <int DT, int DP, int NW>
__device__ __forceinline__ void bwd_dkdv_body(
    int tile, unsigned char* lds, const uint16_t* __restrict__ qkv, int64_t ld, const float* __restrict__ pd,
    const uint16_t* __restrict__ dout, const float* __restrict__ lse,
    const float* __restrict__ delta_ws, uint16_t* __restrict__ dqkv, int64_t ldd,
    float* __restrict__ part, int S, int H, int D, Fold f, float scale, int kb0, int nkc) {
  using G = Geo<DP>;
  using K = Blk<NW>;
  using LY = DkdvLds<DP, NW>;
  static_assert(K::ROWS <= 128, "the dpd rings hold 256 live diagonals");
  static_assert(K::NT == 256, "the ring fold maps 4 lanes to each of 64 diagonals");
  constexpr int TILE = kStep * G::DPV;
  constexpr int BWIN = 4 * K::WLD;
  constexpr int RINGF = LY::RINGF;
  float* const ring = reinterpret_cast<float*>(lds + LY::RING_OFF);
  float* const sink = reinterpret_cast<float*>(lds + LY::SINK_OFF);
  uint16_t* const Qs = reinterpret_cast<uint16_t*>(lds + LY::QS_OFF);
  uint16_t* const Os = reinterpret_cast<uint16_t*>(lds + LY::OS_OFF);
  float* const Lq = reinterpret_cast<float*>(lds + LY::LQ_OFF);
  float* const Dq = reinterpret_cast<float*>(lds + LY::DQ_OFF);
  float* const Bw = reinterpret_cast<float*>(lds + LY::BW_OFF);

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, g = lane >> 5, l32 = lane & 31;
  TileLane<DP> L;
  L.init(lane);
  // Key blocks [kb0, kb0 + nkc) of every (batch, head), nkc per (batch, head) in the grid.
  const int bh = tile / nkc, b = bh / H, h = bh - b * H;
  const int kbl = tile - bh * nkc;
  const int kblk = kb0 + kbl;
  const int j_wg = kblk * K::ROWS;
  const int kk = wave * 32 + kperm(l32);  // this lane's key (score tile column l32)
  const int kj = j_wg + kk;
  const bool kvalid = kj < S;
  const int64_t tok0 = (int64_t)b * S;
  const int64_t HD = (int64_t)H * D;
  const uint16_t* q0 = qkv + tok0 * ld + (int64_t)h * D;
  const uint16_t* o0 = dout + tok0 * HD + (int64_t)h * D;  // row 0 of this (batch, head)'s dO
  const int npd = 2 * S - 1;
  const float* pdh = pd + (int64_t)h * npd;
  const float* lse_bh = lse + (int64_t)bh * S;
  const float* dl_bh = delta_ws + (int64_t)bh * S;
  const float c = f.c;

  u32x4 kreg[G::KS], vreg[G::KS];
#pragma unroll
  for (int s = 0; s < G::KS; ++s) {
    const int d0 = 16 * s + 8 * g;
    const bool ok = kvalid && d0 < D;
    const uint32_t m = lane_mask(ok);
    kreg[s] = masked(fold_operand(ld16(ok ? q0 + HD + (int64_t)kj * ld + d0 : q0), f), m);
    vreg[s] = ld16_masked(q0 + 2 * HD + (int64_t)kj * ld + d0, q0, ok, m);
  }

  f32x16 dk[G::DB], dv[G::DB];
#pragma unroll
  for (int db = 0; db < G::DB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) dk[db][r] = dv[db][r] = 0.f;

  // dpd rings (published by the first step's barrier) and this key block's partial row.
  for (int e = tid; e < RINGF; e += K::NT) ring[e] = 0.f;
  const int off1 = (S & 1) ? 34 : 32;
  const int rcopy = (kk + S) & 1;
  // Keys past S have p != 0 (their bias is real) but no dpd term: their ds go to a sink.
  float* myring = kvalid ? ring + ring_base(2 * wave + g, rcopy, off1) : sink;
  float* prow = part + ((int64_t)bh * nkc + kbl) * (S + K::ROWS);

  uint32_t qoff[Dma<DP, K::NT>::GPT], ooff[Dma<DP, K::NT>::GPT];
  dma_offsets<DP, K::NT>(qoff, ld, D);
  dma_offsets<DP, K::NT>(ooff, HD, D);
  float bst[K::BPT];
  float sst = 0.f;
  const int T = (S + kStep - 1) / kStep;
  // Per-query statistics of the step, loaded one step ahead: wave 0 lse, wave 1 delta
  // (zero past S through the buffer range check). Stashed as -lse, with -inf past S, which
  // makes those rows' p = exp2(acc c - lse) exactly 0 (acc is finite there), and -delta.
  const rsrc_t rstat =
      make_rsrc(__builtin_amdgcn_readfirstlane(wave) == 0 ? lse_bh : dl_bh, (uint32_t)S * 4u);
  auto stats = [&](int i0) {
    if (wave < 2) sst = bload4(rstat, opaque((uint32_t)(i0 + lane) * 4u));
  };
  // Reversed window: entry x holds T[rb - x], rb = (j_wg + ROWS - 1) - i0 + S - 1 the largest
  // diagonal of the step.
  const int rb0 = (j_wg + K::ROWS - 1) + S - 1;
  dma_tile<DP, K::NT>(Qs, qoff, q0, ld, 0, S, D);
  dma_tile<DP, K::NT>(Os, ooff, o0, HD, 0, S, D);
  load_bias<NW>(bst, pdh, npd, rb0, -1);
  stats(0);

  // Step t computes from buffer t & 1 (requested one step earlier); the barrier publishes
  // it and retires every wave's reads of the other buffer (step t-1).
  auto step = [&](int t, auto buf) {
    constexpr int B = decltype(buf)::value;
    const uint16_t* Qb = Qs + B * TILE;
    const uint16_t* Ob = Os + B * TILE;
    const float* Bb = Bw + B * BWIN;
    const float* Lb = Lq + B * kStep;
    const float* Db = Dq + B * kStep;
    stash_bias<NW>(bst, Bw + B * BWIN, f.bmul);
    if (wave == 0)
      Lq[B * kStep + lane] = t * kStep + lane < S ? -sst : -INFINITY;
    else if (wave == 1)
      Dq[B * kStep + lane] = -sst;
    drain_and_sync();
    if (t + 1 < T) {
      const int i1 = (t + 1) * kStep;
      dma_tile<DP, K::NT>(Qs + (1 - B) * TILE, qoff, q0, ld, i1, S, D);
      dma_tile<DP, K::NT>(Os + (1 - B) * TILE, ooff, o0, HD, i1, S, D);
      load_bias<NW>(bst, pdh, npd, rb0 - i1, -1);
      stats(i1);
    }
    const int rp0 = ((kk + S - 2 - 4 * g - kStep * t - rcopy - 58) & 255) + 58;  // slot of r0
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      // dP starts at -D of its row, so the product below is ds / p directly.
      f32x16 acc = read_bias16<NW>(Bb, (K::ROWS - 1) - kk + qb * 32 + 4 * g), accp;
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const f32x4 d4 = *reinterpret_cast<const f32x4*>(Db + qb * 32 + 8 * a + 4 * g);
#pragma unroll
        for (int b4 = 0; b4 < 4; ++b4) accp[4 * a + b4] = d4[b4];
      }
#pragma unroll
      for (int s = 0; s < G::KS; ++s) {
        acc = mfma32x32x16<DT>(row_operand<DP>(Qb, L, qb * 32, s), kreg[s], acc);
        accp = mfma32x32x16<DT>(row_operand<DP>(Ob, L, qb * 32, s), vreg[s], accp);
      }
      // In two halves u (row groups 2u, 2u + 1): p and ds, the dV/dK products of that half,
      // then its dpd ring updates. Each ring read waits for the write before it (lanes of
      // consecutive pairs share slots); placed after the products, the chain overlaps their
      // execution and the next half's softmax (-1.5% backward against one chain per block).
      // Ring pair p of row group a holds diagonals r_s (register 4a + 2p + 1) and r_s + 1
      // (register 4a + 2p); the accesses are volatile so they stay in program order.
      float p[16], ds[16];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
#pragma unroll
        for (int a = 2 * u; a < 2 * u + 2; ++a) {
          const f32x4 nl4 = *reinterpret_cast<const f32x4*>(Lb + qb * 32 + 8 * a + 4 * g);
#pragma unroll
          for (int b4 = 0; b4 < 4; ++b4) {
            const int r = 4 * a + b4;
            const float pv = __builtin_amdgcn_exp2f(__builtin_fmaf(acc[r], c, nl4[b4]));
            p[r] = pv;
            ds[r] = pv * accp[r];
          }
        }
        const u32x4 pa = Elem<DT>::pack(&p[8 * u]);
        const u32x4 dsa = Elem<DT>::pack(&ds[8 * u]);
#pragma unroll
        for (int db = 0; db < G::DB; ++db) {
          dv[db] = mfma32x32x16<DT>(pa, tr_operand<DP>(Ob, L, 2 * qb + u, db), dv[db]);
          dk[db] = mfma32x32x16<DT>(dsa, tr_operand<DP>(Qb, L, 2 * qb + u, db), dk[db]);
        }
#pragma unroll
        for (int a = 2 * u; a < 2 * u + 2; ++a)
#pragma unroll
          for (int pp = 0; pp < 2; ++pp) {
            typedef float f32x2 __attribute__((ext_vector_type(2)));
            typedef __attribute__((address_space(3))) f32x2 lds_f32x2;
            volatile lds_f32x2* rs = (volatile lds_f32x2*)(myring + rp0 - (8 * a + 32 * qb + 2 * pp));
            f32x2 v = *rs;
            v.x += ds[4 * a + 2 * pp + 1];
            v.y += ds[4 * a + 2 * pp];
            *rs = v;
          }
      }
      // Diagonals [S + 63 - 64(t-1), S + 126 - 64(t-1)] got their last ds in step t-1 (step
      // t touches [S - 64 - 64t, S + 62 - 64(t-1)], distinct mod 256): fold them into the
      // partial row (r > 0 here), mid-step so the wait overlaps the MFMAs in flight.
      if (qb == 0 && t > 0) {
        const int r = S + 63 - kStep * (t - 1) + (tid >> 2);
        const float v = ring_fold(ring, r, off1);
        if ((tid & 3) == 0) prow[r] = v;
      }
    }
  };
  // Queries past S carry -lse = -inf (p = 0), so every step is unmasked; the loop is
  // unrolled by two so every buffer offset is a constant.
  int t = 0;
  for (; t + 1 < T; t += 2) {
    step(t, kBuf0);
    step(t + 1, kBuf1);
  }
  if (t < T) step(t, kBuf0);

  // Fold every diagonal still in the rings: [0, S + 126 - 64(T-1)].
  __syncthreads();
  const int nrem = S + K::ROWS - 1 - kStep * (T - 1);
  for (int r0 = 0; r0 < nrem; r0 += kStep) {
    const int r = r0 + (tid >> 2);
    if (r < nrem) {  // uniform per quad
      const float v = ring_fold(ring, r, off1);
      if ((tid & 3) == 0) prow[r] = v;
    }
  }

  // D layout: lane = head dim d (n), register r = tile row 8(r/4) + 4g + r%4, which holds
  // key kperm(row) of this wave.
  if constexpr (2 * kColTile * 4 <= LY::TILES_BYTES) {
    // Staged: waves 0-1 in the Q tiles, 2-3 in the dO tiles (free since the fold's barrier).
    float* wt = reinterpret_cast<float*>(wave < 2 ? Qs : Os) + (wave & 1) * kColTile;
    const int nrows = min(32, S - (j_wg + wave * 32));
    const int64_t row0 = (tok0 + j_wg + wave * 32) * ldd + HD + (int64_t)h * D;
    store_cols_staged<DT, DP>(dk, [scale](float x) { return x * scale; }, lane, nrows, row0, ldd, D, dqkv, wt);
    store_cols_staged<DT, DP>(dv, [](float x) { return x; }, lane, nrows, row0 + HD, ldd, D, dqkv, wt);
  } else {
#pragma unroll
    for (int db = 0; db < G::DB; ++db) {
      const int d = db * 32 + l32;
      if (d < D) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = j_wg + wave * 32 + kperm(8 * (r >> 2) + 4 * g + (r & 3));
          if (key < S) {
            uint16_t* rowp = dqkv + (tok0 + key) * ldd + HD + (int64_t)h * D + d;
            rowp[0] = Elem<DT>::store(dk[db][r] * scale);
            rowp[HD] = Elem<DT>::store(dv[db][r]);
          }
        }
      }
    }
  }
}

template <int DT, int DP, int NW>
__global__ __launch_bounds__(64 * NW, (DP <= 64 ? 2 : 1)) void relpos_bwd_dkdv_kernel(
    const uint16_t* __restrict__ qkv, int64_t ld, const float* __restrict__ pd,
    const uint16_t* __restrict__ dout, const float* __restrict__ lse,
    const float* __restrict__ delta_ws, uint16_t* __restrict__ dqkv, int64_t ldd,
    float* __restrict__ part, int S, int H, int D, Fold f, float scale, int kb0, int nkc) {
  __shared__ __attribute__((aligned(256))) unsigned char lds[DkdvLds<DP, NW>::BYTES];
  bwd_dkdv_body<DT, DP, NW>(xcd_tile(blockIdx.x, gridDim.x), lds, qkv, ld, pd, dout, lse, delta_ws, dqkv, ldd,
                            part, S, H, D, f, scale, kb0, nkc);
}

// --------------------------------------------- backward on small grids: one launch for both
// delta[bh, i] = sum_d dO[i, d] O32[i, d], summed exactly as the dQ kernel's prologue sums it
// (the lower half-wave's 8-element chunks 16s..16s+7, the upper half's 16s+8..16s+15, each in
// order, then lower + upper), so delta is bitwise the same. Two threads per (query, head), one
// per half; the even one adds the odd one's sum to its own. D <= 64 (the paired backward's).
template <int DT>
__global__ __launch_bounds__(256) void relpos_delta_kernel(const uint16_t* __restrict__ dout,
                                                           const float* __restrict__ out32,
                                                           float* __restrict__ delta_ws, int B, int S, int H,
                                                           int D) {
  const int64_t n = (int64_t)B * H * S;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int g = (int)(t & 1);
  const int64_t e = t >> 1;
  const bool live = e < n;
  const int64_t ec = live ? e : 0;
  const int64_t bh = ec / S, i = ec - bh * S;
  const int64_t b = bh / H, h = bh - b * H;
  const int64_t base = (b * S + i) * H * D + h * D;
  float half = 0.f;
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const int d0 = 16 * s + 8 * g;
    if (live && d0 < D) {
      float df[8];
      Elem<DT>::unpack(ld16(dout + base + d0), df);
      const f32x4 o0 = *reinterpret_cast<const f32x4*>(out32 + base + d0);
      const f32x4 o1 = *reinterpret_cast<const f32x4*>(out32 + base + d0 + 4);
#pragma unroll
      for (int q = 0; q < 4; ++q) half += df[q] * o0[q];
#pragma unroll
      for (int q = 0; q < 4; ++q) half += df[4 + q] * o1[q];
    }
  }
  const float upper = __shfl_xor(half, 1);
  if (live && g == 0) delta_ws[e] = half + upper;
}

// The dQ and dK/dV kernels in one grid, for grids too small to give every CU two workgroups
// of either alone (at most 256 workgroups each): half the workgroups take dQ blocks and half
// dK/dV blocks, so the two kinds run side by side on each CU, and the two kinds of the same
// (batch, head) share an XCD's L2. delta comes from relpos_delta_kernel.
template <int DT, int DP>
__global__ __launch_bounds__(256, (DP <= 64 ? 2 : 1)) void relpos_bwd_pair_kernel(
    const uint16_t* __restrict__ qkv, int64_t ld, const float* __restrict__ pd,
    const uint16_t* __restrict__ dout, const float* __restrict__ out32, const float* __restrict__ lse,
    float* __restrict__ delta_ws, uint16_t* __restrict__ dqkv, int64_t ldd, float* __restrict__ part, int S, int H,
    int D, Fold f, float scale) {
  constexpr int BYTES = DqLds<DP, 4>::BYTES > DkdvLds<DP, 4>::BYTES ? DqLds<DP, 4>::BYTES : DkdvLds<DP, 4>::BYTES;
  __shared__ __attribute__((aligned(256))) unsigned char lds[BYTES];
  // XCD x holds tiles [x q, (x + 1) q) of the XCD-ordered grid and its 32 CUs take them in
  // order, one per CU before any takes a second: with q even the first half of an XCD's range
  // runs dQ blocks and the second half the dK/dV blocks of the same (batch, head)s, so a CU
  // holding two workgroups holds one of each. Otherwise the kinds alternate.
  const int c = xcd_tile(blockIdx.x, gridDim.x);
  const int N = gridDim.x;
  int kind = c & 1, idx = c >> 1;
  if (N % (2 * kXcds) == 0) {
    const int q = N / kXcds, half = q / 2, x = c / q, k = c - x * q;
    kind = k >= half;
    idx = x * half + k - kind * half;
  }
  // The dK/dV blocks carry about 1.7x the dQ blocks' work, so they set the launch's length: their
  // waves issue ahead of the dQ waves sharing their SIMDs (outputs bitwise the same; backward,
  // interleaved A/B: B4 S512 H16 D64 39.4 -> 36.5 us, B2 S1024 H16 57.1 -> 52.2, B1 S2048 H16
  // 92.8 -> 87.1; priority 3, or the dQ waves lowered instead, measured the same).
  if (kind) {
    __builtin_amdgcn_s_setprio(1);
    bwd_dkdv_body<DT, DP, 4>(idx, lds, qkv, ld, pd, dout, lse, delta_ws, dqkv, ldd, part, S, H, D, f, scale, 0,
                             (S + 127) / 128);
  } else
    bwd_dq_body<DT, DP, 4, true>(idx, lds, qkv, ld, pd, dout, out32, lse, delta_ws, dqkv, ldd, S, H, D, f,
                                 scale);
}

// dpd[h, k] (+)= sum over b and key blocks kb0 .. kb0 + nqb - 1 of the partial rows (row of
// key block kb holds k - rows kb; part holds the rows of those nqb blocks only), fixed order.
// Block: 64 diagonals (lane) of head h; the 4 waves take every 4th (b, key block) term, then
// the 4 wave sums are added in wave order; acc_in adds the total to dpd's value.
__global__ __launch_bounds__(256) void relpos_dpd_reduce(const float* __restrict__ part,
                                                         float* __restrict__ dpd, int B, int S,
                                                         int H, int kb0, int nqb, int rows, int acc_in) {
  __shared__ float s[4][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int k = blockIdx.x * 64 + lane;
  const int h = blockIdx.y;
  const int npd = 2 * S - 1;
  const int RS = S + rows;
  const int rlen = S + rows - 1;
  // Terms e = wave, wave + 4, ... are loaded 16 at a time (all requests in flight together:
  // the kernel is latency-bound otherwise) and added in e order; absent terms add 0.
  constexpr int kBatch = 16;
  float acc = 0.f;
  if (k < npd) {
    const int terms = B * nqb;
    for (int e0 = wave; e0 < terms; e0 += 4 * kBatch) {
      float v[kBatch];
#pragma unroll
      for (int i = 0; i < kBatch; ++i) {
        const int e = e0 + 4 * i;
        const int b = e / nqb, kbl = e - b * nqb;
        const int r = k - rows * (kb0 + kbl);
        v[i] = (e < terms && r >= 0 && r < rlen) ? part[((int64_t)(b * H + h) * nqb + kbl) * RS + r] : 0.f;
      }
#pragma unroll
      for (int i = 0; i < kBatch; ++i) acc += v[i];
    }
  }
  s[wave][lane] = acc;
  __syncthreads();
  if (wave == 0 && k < npd) {
    const float t = ((s[0][lane] + s[1][lane]) + s[2][lane]) + s[3][lane];
    float* o = dpd + (int64_t)h * npd + k;
    *o = acc_in ? *o + t : t;
  }
}

// The same sum, 4 consecutive diagonals per lane with 128-bit loads, for S % 4 == 0 (then
// every partial row starts 16-byte aligned and k - rows kb is a multiple of 4). Each
// diagonal gets the same terms in the same order as in relpos_dpd_reduce, so the result is
// bitwise the same; entries at or past the row's end (index rlen) are masked to 0.
__global__ __launch_bounds__(256) void relpos_dpd_reduce4(const float* __restrict__ part,
                                                          float* __restrict__ dpd, int B, int S,
                                                          int H, int kb0, int nqb, int rows, int acc_in) {
  __shared__ f32x4 s[4][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int k0 = 4 * (blockIdx.x * 64 + lane);
  const int h = blockIdx.y;
  const int npd = 2 * S - 1;
  const int RS = S + rows;
  const int rlen = S + rows - 1;
  constexpr int kBatch = 16;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  if (k0 < npd) {
    const int terms = B * nqb;
    for (int e0 = wave; e0 < terms; e0 += 4 * kBatch) {
      f32x4 v[kBatch];
#pragma unroll
      for (int i = 0; i < kBatch; ++i) {
        const int e = e0 + 4 * i;
        const int b = e / nqb, kbl = e - b * nqb;
        const int r = k0 - rows * (kb0 + kbl);
        v[i] = (e < terms && r >= 0 && r < rlen)
                   ? *reinterpret_cast<const f32x4*>(part + ((int64_t)(b * H + h) * nqb + kbl) * RS + r)
                   : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (r + j >= rlen) v[i][j] = 0.f;
      }
#pragma unroll
      for (int i = 0; i < kBatch; ++i) acc += v[i];
    }
  }
  s[wave][lane] = acc;
  __syncthreads();
  if (wave == 0) {
    const f32x4 t = ((s[0][lane] + s[1][lane]) + s[2][lane]) + s[3][lane];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (k0 + j < npd) {
        float* o = dpd + (int64_t)h * npd + k0 + j;
        *o = acc_in ? *o + t[j] : t[j];
      }
  }
}

// Waves per workgroup of the three attention kernels.
constexpr int kFwdNW = 4;
// Forward grids of fewer workgroups than this (two per CU of the MI355X's 256) split each
// workgroup's keys over two wave groups (relpos_fwd_ks_kernel).
constexpr unsigned kFwdSplitBelow = 512;
// Split-key grids of at most this many workgroups (one per CU) take the kernel's register
// budget for 2 waves per SIMD at D 49-64 instead of 4. Interleaved A/B of the forward: B4 S512
// H16 D64 14.80 -> 14.42 us, B2 S1024 H16 21.0 -> 20.0 us, B1 S2048 H16 34.6 -> 32.2 us, B1 S300
// H16 10.2 -> 9.45 us; at 384 workgroups it holds one per CU and lost (29.3 -> 35.6 us).
constexpr unsigned kFwdWideMax = 256;
constexpr int kDqNW = 4;
constexpr int kDkdvNW = 4;
// Backward grids of at most this many workgroups per kernel (the MI355X's 256 CUs) run the dQ
// and dK/dV work in one launch (relpos_bwd_pair_kernel), at head dims up to 64, where the
// dK/dV kernel's LDS and registers leave room for two workgroups per CU. Above 128 per kernel
// the grid must split evenly over the 8 XCDs in halves (2n % 16 == 0), so that the two
// workgroups a CU holds are one of each kind. A/B, backward, builds interleaved in one
// process: B1 S300 H16 D64 (48 workgroups each) 27.1 -> 23.6 us, B1 S130 H8 D64 (16) 21.3 ->
// 19.0 us, B2 S1024 H16 D64 (256) 59.5 -> 56.3 us, B1 S2048 H16 D64 (256) 98.0 -> 92.3 us,
// B4 S512 H16 D64 (256) 39.9 -> 40.0 us; pairing by parity of the tile instead put two of the
// same kind on each CU and lost at 256 (B2 S1024 H16 D64 59.5 -> 61.2 us).
constexpr int kPairBwdMax = 256;

// Smallest nonzero |scale| * log2(e) the folded bias accepts: pd * log2(e) / c must
// stay finite for any realistic table.
constexpr float kMinScaleLog2 = 8.67361737988403547e-19f;  // 2^-60

// esize: bytes per activation element (2 for bf16 / fp16, 4 for fp32).
int check_attn(const void* qkv, int64_t ld, int B, int S, int H, int D, float scale, int esize) {
  if (B <= 0 || S <= 0 || H <= 0 || D <= 0) return KRSI_ERR_BAD_SHAPE;
  if (D % 8 != 0 || D > 128) return KRSI_ERR_UNSUPPORTED;
  if ((int64_t)B * H > 65535 || S > (1 << 24)) return KRSI_ERR_BAD_SHAPE;
  if (ld < 3 * (int64_t)H * D) return KRSI_ERR_BAD_SHAPE;
  // The 16-bit kernels' buffer resources of one (batch, head) slice hold S rows of ld values
  // in < 2^31 bytes (the fp32 kernels address with 64-bit offsets).
  if (esize == 2 && (int64_t)S * ld * 2 >= ((int64_t)1 << 31)) return KRSI_ERR_UNSUPPORTED;
  if ((ld * esize) % 16 != 0 || !aligned16(qkv)) return KRSI_ERR_MISALIGNED;
  if (!(scale == scale) || scale > 3.0e38f || scale < -3.0e38f) return KRSI_ERR_BAD_SCALE;
  // Only the 16-bit kernels fold the bias into the score accumulator as pd / c; the fp32
  // kernels compute q.k * scale + bias directly and take any finite scale.
  const float c = fabsf(scale * kLog2e);
  if (esize == 2 && c != 0.f && c < kMinScaleLog2) return KRSI_ERR_BAD_SCALE;
  return KRSI_OK;
}

Fold fold_scale(float scale) {
  const float c = scale * kLog2e;
  if (c == 0.f) return Fold{1.f, kLog2e, 0u, 0u};
  const float a = fabsf(c);
  return Fold{a, kLog2e / a, 0xffffffffu, c < 0.f ? 0x80008000u : 0u};
}

int padded_dim(int D) { return (D + 15) / 16 * 16; }

static_assert(Blk<kDkdvNW>::ROWS == kKvRows, "dpd partial rows: one per kKvRows keys");

size_t ws_delta_bytes(int B, int S, int H) { return align256((size_t)B * H * S * sizeof(float)); }
// One dpd partial row of S + rows floats per (b, h, key block).
size_t ws_part_bytes(int B, int S, int H) {
  const size_t nkb = (size_t)ceil_div(S, kKvRows);
  return align256((size_t)B * H * nkb * (size_t)(S + kKvRows) * sizeof(float));
}

template <int DT, int DP>
void launch_fwd(const void* qkv, int64_t ld, const float* pd, void* out, float* out32, float* lse,
                int B, int S, int H, int D, Fold f, hipStream_t st) {
  using K = Blk<kFwdNW>;
  const dim3 grid((unsigned)(ceil_div(S, K::ROWS) * B * H));
  if (grid.x < kFwdSplitBelow && S > kStep) {
    if constexpr (DP == 64) {
      if (grid.x <= kFwdWideMax) {
        hipLaunchKernelGGL((relpos_fwd_ks_kernel<DT, DP, true>), grid, dim3(2 * K::NT), 0, st,
                           (const uint16_t*)qkv, ld, pd, (uint16_t*)out, out32, lse, S, H, D, f);
        return;
      }
    }
    hipLaunchKernelGGL((relpos_fwd_ks_kernel<DT, DP, false>), grid, dim3(2 * K::NT), 0, st,
                       (const uint16_t*)qkv, ld, pd, (uint16_t*)out, out32, lse, S, H, D, f);
    return;
  }
  hipLaunchKernelGGL((relpos_fwd_kernel<DT, DP, kFwdNW>), grid, dim3(K::NT), 0, st,
                     (const uint16_t*)qkv, ld, pd, (uint16_t*)out, out32, lse, S, H, D, f);
}

template <int DT, int DP>
void launch_bwd(const void* dout, const void* qkv, int64_t ld, const float* pd, const float* out32,
                const float* lse, void* dqkv, int64_t ldd, float* dpd, void* ws, int nkc, int B, int S,
                int H, int D, Fold f, float scale, hipStream_t st) {
  using KQ = Blk<kDqNW>;
  using KK = Blk<kDkdvNW>;
  float* delta = static_cast<float*>(ws);
  float* part = reinterpret_cast<float*>(static_cast<char*>(ws) + ws_delta_bytes(B, S, H));
  const int nqb = (int)ceil_div(S, KQ::ROWS);
  const int nkb = (int)ceil_div(S, KK::ROWS);
  static_assert(KQ::ROWS == KK::ROWS && kDqNW == 4 && kDkdvNW == 4, "the pair kernel pairs equal grids");
  const int nblk = nqb * B * H;
  // Larger head dims: 1 workgroup of either kind per CU.
  if (DP <= 64 && nkc == nkb &&
      (nblk <= kPairBwdMax / 2 || (nblk <= kPairBwdMax && (2 * nblk) % (2 * kXcds) == 0))) {
    const int64_t n = (int64_t)B * H * S;
    hipLaunchKernelGGL((relpos_delta_kernel<DT>), dim3((unsigned)ceil_div(2 * n, 256)), dim3(256), 0, st,
                       (const uint16_t*)dout, out32, delta, B, S, H, D);
    hipLaunchKernelGGL((relpos_bwd_pair_kernel<DT, DP>), dim3((unsigned)(2 * nqb * B * H)), dim3(256), 0, st,
                       (const uint16_t*)qkv, ld, pd, (const uint16_t*)dout, out32, lse, delta, (uint16_t*)dqkv,
                       ldd, part, S, H, D, f, scale);
    launch_dpd_reduce(part, dpd, B, S, H, 0, nkb, false, st);
    return;
  }
  hipLaunchKernelGGL((relpos_bwd_dq_kernel<DT, DP, kDqNW>), dim3((unsigned)(nqb * B * H)),
                     dim3(KQ::NT), 0, st, (const uint16_t*)qkv, ld, pd, (const uint16_t*)dout, out32,
                     lse, delta, (uint16_t*)dqkv, ldd, S, H, D, f, scale);
  // A workspace that holds the partial rows of nkc < nkb key blocks: the key blocks go in
  // chunks of nkc, each one's rows summed into dpd before the next chunk overwrites them.
  for (int kb0 = 0; kb0 < nkb; kb0 += nkc) {
    const int n = min(nkc, nkb - kb0);
    hipLaunchKernelGGL((relpos_bwd_dkdv_kernel<DT, DP, kDkdvNW>), dim3((unsigned)(n * B * H)),
                       dim3(KK::NT), 0, st, (const uint16_t*)qkv, ld, pd, (const uint16_t*)dout, lse,
                       (const float*)delta, (uint16_t*)dqkv, ldd, part, S, H, D, f, scale, kb0, n);
    launch_dpd_reduce(part, dpd, B, S, H, kb0, n, kb0 > 0, st);
  }
}

template <int DT>
int dispatch_fwd(const void* qkv, int64_t ld, const float* pd, void* out, float* out32, float* lse,
                 int B, int S, int H, int D, Fold f, hipStream_t st) {
  switch (padded_dim(D)) {
#define KRSI_CASE(DPV_)                                                                \
  case DPV_:                                                                           \
    launch_fwd<DT, DPV_>(qkv, ld, pd, out, out32, lse, B, S, H, D, f, st);             \
    break;
    KRSI_CASE(16) KRSI_CASE(32) KRSI_CASE(48) KRSI_CASE(64) KRSI_CASE(80) KRSI_CASE(96)
    KRSI_CASE(112) KRSI_CASE(128)
#undef KRSI_CASE
    default:
      return KRSI_ERR_UNSUPPORTED;
  }
  return launch_status();
}

template <int DT>
int dispatch_bwd(const void* dout, const void* qkv, int64_t ld, const float* pd, const float* out32,
                 const float* lse, void* dqkv, int64_t ldd, float* dpd, void* ws, int nkc, int B, int S,
                 int H, int D, Fold f, float scale, hipStream_t st) {
  switch (padded_dim(D)) {
#define KRSI_CASE(DPV_)                                                                          \
  case DPV_:                                                                                     \
    launch_bwd<DT, DPV_>(dout, qkv, ld, pd, out32, lse, dqkv, ldd, dpd, ws, nkc, B, S, H, D, f,  \
                         scale, st);                                                             \
    break;
    KRSI_CASE(16) KRSI_CASE(32) KRSI_CASE(48) KRSI_CASE(64) KRSI_CASE(80) KRSI_CASE(96)
    KRSI_CASE(112) KRSI_CASE(128)
#undef KRSI_CASE
    default:
      return KRSI_ERR_UNSUPPORTED;
  }
  return launch_status();
}

}  // namespace

void launch_dpd_reduce(const float* part, float* dpd, int B, int S, int H, int kb0, int nkc,
                       bool acc_in, hipStream_t st) {
  if (S % 4 == 0) {
    const dim3 rgrid((unsigned)ceil_div(2 * S - 1, 256), (unsigned)H);
    hipLaunchKernelGGL(relpos_dpd_reduce4, rgrid, dim3(256), 0, st, part, dpd, B, S, H, kb0, nkc, kKvRows,
                       (int)acc_in);
  } else {
    const dim3 rgrid((unsigned)ceil_div(2 * S - 1, 64), (unsigned)H);
    hipLaunchKernelGGL(relpos_dpd_reduce, rgrid, dim3(256), 0, st, part, dpd, B, S, H, kb0, nkc, kKvRows,
                       (int)acc_in);
  }
}

int relpos_bwd_chunk_blocks(size_t ws_bytes, int B, int S, int H) {
  const size_t delta = ws_delta_bytes(B, S, H);
  if (ws_bytes < delta) return 0;
  const size_t row_set = (size_t)B * H * (size_t)(S + kKvRows) * sizeof(float);
  const size_t fit = (ws_bytes - delta) / row_set;
  const int nkb = (int)ceil_div(S, kKvRows);
  return fit >= (size_t)nkb ? nkb : (int)fit;
}

}  // namespace krsi

extern "C" {

int krsi_relpos_fwd(const void* qkv, int64_t ld_qkv, const float* pd, void* out, float* out32,
                    float* lse, int32_t B, int32_t S, int32_t H, int32_t D, float scale,
                    int32_t dtype, void* stream) {
  using namespace krsi;
  if (dtype != kBf16 && dtype != kF16 && dtype != kF32) return KRSI_ERR_UNSUPPORTED;
  // out32 and lse may both be null (O only, for a forward no backward follows), not one alone.
  if (!qkv || !pd || !out || (!out32 != !lse)) return KRSI_ERR_NULL_POINTER;
  int rc = check_attn(qkv, ld_qkv, B, S, H, D, scale, dtype == kF32 ? 4 : 2);
  if (rc != KRSI_OK) return rc;
  if (!aligned16(out) || (out32 && !aligned16(out32))) return KRSI_ERR_MISALIGNED;
  hipStream_t st = as_stream(stream);
  if (dtype == kF32)
    return relpos_fwd_f32(static_cast<const float*>(qkv), ld_qkv, pd, static_cast<float*>(out), out32, lse,
                          B, S, H, D, scale, st);
  const Fold f = fold_scale(scale);
  return dtype == kF16 ? dispatch_fwd<kF16>(qkv, ld_qkv, pd, out, out32, lse, B, S, H, D, f, st)
                       : dispatch_fwd<kBf16>(qkv, ld_qkv, pd, out, out32, lse, B, S, H, D, f, st);
}

int krsi_relpos_fwd_bf16(const void* qkv, int64_t ld_qkv, const float* pd, void* out, float* out32,
                         float* lse, int32_t B, int32_t S, int32_t H, int32_t D, float scale,
                         void* stream) {
  return krsi_relpos_fwd(qkv, ld_qkv, pd, out, out32, lse, B, S, H, D, scale, KRSI_DTYPE_BF16,
                         stream);
}

size_t krsi_relpos_bwd_workspace_bytes(int32_t B, int32_t S, int32_t H, int32_t D) {
  using namespace krsi;
  (void)D;
  if (B <= 0 || S <= 0 || H <= 0) return 0;
  return ws_delta_bytes(B, S, H) + ws_part_bytes(B, S, H);
}

size_t krsi_relpos_bwd_workspace_min_bytes(int32_t B, int32_t S, int32_t H, int32_t D) {
  using namespace krsi;
  (void)D;
  if (B <= 0 || S <= 0 || H <= 0) return 0;
  return ws_delta_bytes(B, S, H) + (size_t)B * H * (size_t)(S + kKvRows) * sizeof(float);
}

int krsi_relpos_bwd(const void* dout, const void* qkv, int64_t ld_qkv, const float* pd,
                    const float* out32, const float* lse, void* dqkv, int64_t ld_dqkv, float* dpd,
                    void* workspace, size_t workspace_bytes, int32_t B, int32_t S, int32_t H,
                    int32_t D, float scale, int32_t dtype, void* stream) {
  using namespace krsi;
  if (dtype != kBf16 && dtype != kF16 && dtype != kF32) return KRSI_ERR_UNSUPPORTED;
  if (!dout || !qkv || !pd || !out32 || !lse || !dqkv || !dpd) return KRSI_ERR_NULL_POINTER;
  const int esize = dtype == kF32 ? 4 : 2;
  int rc = check_attn(qkv, ld_qkv, B, S, H, D, scale, esize);
  if (rc != KRSI_OK) return rc;
  if (ld_dqkv < 3 * (int64_t)H * D) return KRSI_ERR_BAD_SHAPE;
  if ((ld_dqkv * esize) % 16 != 0 || !aligned16(dqkv) || !aligned16(dout) || !aligned16(out32))
    return KRSI_ERR_MISALIGNED;
  if (!workspace || workspace_bytes < krsi_relpos_bwd_workspace_min_bytes(B, S, H, D))
    return KRSI_ERR_WORKSPACE;
  if (!aligned16(workspace)) return KRSI_ERR_MISALIGNED;
  // Key blocks per dK/dV launch: all of them with the full workspace, fewer (then several
  // launches, each followed by its dpd sum) with a smaller one.
  const int nkc = relpos_bwd_chunk_blocks(workspace_bytes, B, S, H);
  hipStream_t st = as_stream(stream);
  if (dtype == kF32) {
    float* delta = static_cast<float*>(workspace);
    float* part = reinterpret_cast<float*>(static_cast<char*>(workspace) + ws_delta_bytes(B, S, H));
    return relpos_bwd_f32(static_cast<const float*>(dout), static_cast<const float*>(qkv), ld_qkv, pd, out32,
                          lse, static_cast<float*>(dqkv), ld_dqkv, dpd, delta, part, nkc, B, S, H, D, scale,
                          st);
  }
  const Fold f = fold_scale(scale);
  return dtype == kF16
             ? dispatch_bwd<kF16>(dout, qkv, ld_qkv, pd, out32, lse, dqkv, ld_dqkv, dpd, workspace,
                                  nkc, B, S, H, D, f, scale, st)
             : dispatch_bwd<kBf16>(dout, qkv, ld_qkv, pd, out32, lse, dqkv, ld_dqkv, dpd, workspace,
                                   nkc, B, S, H, D, f, scale, st);
}

int krsi_relpos_bwd_bf16(const void* dout, const void* qkv, int64_t ld_qkv, const float* pd,
                         const float* out32, const float* lse, void* dqkv, int64_t ld_dqkv,
                         float* dpd, void* workspace, size_t workspace_bytes, int32_t B, int32_t S,
                         int32_t H, int32_t D, float scale, void* stream) {
  return krsi_relpos_bwd(dout, qkv, ld_qkv, pd, out32, lse, dqkv, ld_dqkv, dpd, workspace,
                         workspace_bytes, B, S, H, D, scale, KRSI_DTYPE_BF16, stream);
}

}  // extern "C"
