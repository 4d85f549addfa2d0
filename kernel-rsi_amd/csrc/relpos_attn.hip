// Relative-position-bias flash attention (non-causal), forward and backward,
// for gfx950 on bf16 MFMA (v_mfma_f32_32x32x16_bf16), fp32 softmax.
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
//     the copy stride puts the 8 lanes of one read phase on distinct banks.
//   * Online softmax keeps the exact running max per 64-key step (the step
//     maximum gives p = 1, exact in bf16, as in the reference); the fp32
//     accumulators are rescaled only when some lane's max moved. The row sum
//     adds the bf16 p the PV product uses (v_dot2c_f32_bf16, two per op).
//   * dpd is reduced along the diagonals j - i inside the dQ kernel: each
//     (wave, half-wave) adds its fp32 ds into a private LDS ring indexed by
//     diagonal. Within one register the 32 lanes of a half-wave hit distinct
//     slots and a wave's LDS operations complete in order, so a plain
//     read-modify-write is exact and deterministic. Diagonals that can get no
//     further contribution are folded in a fixed order into one partial row per
//     query block; a last kernel sums the partial rows over batch and query
//     blocks in a fixed order. No [B, H, S, S] buffer exists.
#include <math.h>

#include "krsi_device.h"
#include "krsi_internal.h"

namespace krsi {
namespace {

constexpr int kStep = 64;  // streamed positions per iteration
constexpr float kLog2e = 1.4426950408889634f;

template <int DP>
struct Geo {
  static constexpr int KS = DP / 16;         // K steps of 16 over the head dim
  static constexpr int DB = (DP + 31) / 32;  // 32-wide head-dim blocks of head-dim outputs
  static constexpr int DPV = DB * 32;
  static constexpr int RLD = DPV + 8;        // row-major tile stride (bf16), padded
  static constexpr int CPR = DP / 8;         // 16-byte chunks per staged row
  static constexpr int NCH = kStep * CPR;    // chunks per streamed tile
};

template <int NW>
struct Blk {
  static constexpr int ROWS = 32 * NW;             // queries or keys per workgroup
  static constexpr int NT = 64 * NW;               // threads per workgroup
  static constexpr int WLD = ROWS + kStep + 8;     // bias copy stride, = 8 (mod 32) floats
  static constexpr int WIN = WLD - 3;              // distinct window entries loaded
  static constexpr int BPT = (WIN + NT - 1) / NT;  // window entries per thread
  static constexpr int RING = ROWS <= 128 ? 256 : 512;  // dpd ring (>= ROWS + 2 * kStep - 1)
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
typedef __attribute__((address_space(3))) float lds_f32;

constexpr u32x4 kZero4 = {0u, 0u, 0u, 0u};

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

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, kRsrcWord3);
}
__device__ __forceinline__ u32x4 bload16(rsrc_t r, uint32_t voff) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, 0, 0));
}
__device__ __forceinline__ float bload4(rsrc_t r, uint32_t voff) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (int)voff, 0, 0));
}

// MFMA operand whose 8 K values are rows [k0, k0+4) and [k1, k1+4) of column
// c0 + (lane % 16) of a row-major LDS tile (stride ld): two transposed reads,
// in each of which lane s of a 16-lane group supplies row (k + s/4), columns
// c0 + 4 (s % 4) .. +3. The caller passes c0 = block + 16 * ((lane / 16) % 2),
// so lane l receives column block + l % 32.
__device__ __forceinline__ u32x4 tr_operand(const uint16_t* tile, int ld, int k0, int k1, int c0) {
  const int s = threadIdx.x & 15;
  const int off = (s >> 2) * ld + c0 + 4 * (s & 3);
  const s16x4 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(tile + k0 * ld + off));
  const s16x4 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(tile + k1 * ld + off));
  const uint2 ua = __builtin_bit_cast(uint2, a), ub = __builtin_bit_cast(uint2, b);
  return u32x4{ua.x, ua.y, ub.x, ub.y};
}

// Streamed tiles. Chunk c = threadIdx.x + k * NT of a tile is row c / CPR, head-dim
// columns d0 = 8 (c % CPR) .. +7. Its byte offset from the tile's first row is fixed
// per thread; chunks past D (or past the tile) get kOob and read as zero.
template <int DP, int NT>
struct Tile {
  static constexpr int CPT = (Geo<DP>::NCH + NT - 1) / NT;
};

template <int DP, int NT>
__device__ __forceinline__ void tile_offsets(uint32_t* voff, int64_t ld, int D) {
  using G = Geo<DP>;
#pragma unroll
  for (int k = 0; k < Tile<DP, NT>::CPT; ++k) {
    const int c = threadIdx.x + k * NT;
    const int row = c / G::CPR, d0 = (c - row * G::CPR) * 8;
    voff[k] = opaque((c < G::NCH && d0 < D) ? (uint32_t)(row * ld + d0) * 2u : kOob);
  }
}

// Rows p0..p0+63 of the [S, D] slice whose row 0 is `origin` (row stride ld): the
// resource ends at the last byte of row S-1, so rows >= S read as zero.
template <int DP, int NT>
__device__ __forceinline__ void load_tile(u32x4* regs, const uint32_t* voff, const uint16_t* origin,
                                          int64_t ld, int p0, int S, int D) {
  const rsrc_t r = make_rsrc(origin + (int64_t)p0 * ld, (uint32_t)(((int64_t)(S - 1 - p0) * ld + D) * 2));
#pragma unroll
  for (int k = 0; k < Tile<DP, NT>::CPT; ++k) regs[k] = bload16(r, voff[k]);
}

template <int DP, int NT>
__device__ __forceinline__ void stash_tile(const u32x4* regs, uint16_t* tile) {
  using G = Geo<DP>;
#pragma unroll
  for (int k = 0; k < Tile<DP, NT>::CPT; ++k) {
    const int c = threadIdx.x + k * NT;
    if (c < G::NCH) {
      const int row = c / G::CPR, d0 = (c - row * G::CPR) * 8;
      *reinterpret_cast<u32x4*>(tile + row * G::RLD + d0) = regs[k];
    }
  }
}

// Columns [DP, DPV) of a row-major tile are read by the transposed reads of the
// last head-dim block and never staged: zero them once.
template <int DP, int NT>
__device__ __forceinline__ void zero_pad_cols(uint16_t* tile) {
  using G = Geo<DP>;
  constexpr int W = G::DPV - DP;
  if (W > 0)
    for (int e = threadIdx.x; e < kStep * W; e += NT) tile[(e / W) * G::RLD + DP + e % W] = 0;
}

// Bias window entry x (0 <= x < WIN) holds T[wb + sgn * x] * bmul, zero outside
// [0, 2S - 1) (out-of-range offsets, negative ones included, fall past the
// resource); it is stored at position x + cc of copy cc.
template <int NW>
__device__ __forceinline__ void load_bias(float* regs, const float* pdh, int npd, int wb, int sgn,
                                          float bmul) {
  using K = Blk<NW>;
  const rsrc_t r = make_rsrc(pdh, (uint32_t)npd * 4u);
#pragma unroll
  for (int k = 0; k < K::BPT; ++k) {
    const int x = threadIdx.x + k * K::NT;
    regs[k] = x < K::WIN ? bload4(r, opaque((uint32_t)(wb + sgn * x) * 4u)) * bmul : 0.f;
  }
}

template <int NW>
__device__ __forceinline__ void stash_bias(const float* regs, float* bw) {
  using K = Blk<NW>;
#pragma unroll
  for (int k = 0; k < K::BPT; ++k) {
    const int x = threadIdx.x + k * K::NT;
    if (x < K::WIN) {
#pragma unroll
      for (int cc = 0; cc < 4; ++cc) bw[cc * K::WLD + x + cc] = regs[k];
    }
  }
}

// The 16 bias values of one 32x32 D tile, as the tile's initial accumulator:
// window entries x0 + 8a + b (a, b = 0..3), read from the copy that makes x0
// 16-byte aligned.
template <int NW>
__device__ __forceinline__ f32x16 read_bias16(const float* bw, int x0) {
  const int cc = (-x0) & 3;
  const float* p = bw + cc * Blk<NW>::WLD + x0 + cc;
  f32x16 out;
#pragma unroll
  for (int a = 0; a < 4; ++a) {
    const f32x4 v = *reinterpret_cast<const f32x4*>(p + 8 * a);
#pragma unroll
    for (int b = 0; b < 4; ++b) out[4 * a + b] = v[b];
  }
  return out;
}

// Row sum of bf16 p values: two per v_dot2c_f32_bf16 against (1, 1).
__device__ __forceinline__ float add_bf16_pair(uint32_t pair, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, pair),
                                         __builtin_bit_cast(bf16x2, 0x3f803f80u), acc, false);
}

// ------------------------------------------------------------------- forward
// One 64-key step of the forward for this lane's query: scores (bias folded into
// the accumulator), exact running max, p = exp2(acc c - m), l += bf16(p),
// O^T += V^T P^T. TAIL masks keys >= S (last step only).
template <int DP, int NW, bool TAIL>
__device__ __forceinline__ void fwd_step(const uint16_t* Ks, const uint16_t* Vs, const float* Bw,
                                         const u32x4* qreg, f32x16* oacc, float& m_run, float* l_run,
                                         int j0, int S, int ii, int g, int l32, int c0, float c) {
  using G = Geo<DP>;
  using K = Blk<NW>;
  f32x16 sc[2];
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
    sc[kb] = read_bias16<NW>(Bw, kb * 32 + 4 * g + (K::ROWS - 1) - ii);
#pragma unroll
    for (int s = 0; s < G::KS; ++s)
      sc[kb] = mfma32x32x16(ld16(Ks + (kb * 32 + l32) * G::RLD + 16 * s + 8 * g), qreg[s], sc[kb]);
    if (TAIL) {
#pragma unroll
      for (int r = 0; r < 16; ++r)
        if (j0 + kb * 32 + 8 * (r >> 2) + 4 * g + (r & 3) >= S) sc[kb][r] = -INFINITY;
    }
  }
  float mx = fmaxf(sc[0][0], sc[1][0]);
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int r = 1; r < 16; ++r) mx = fmaxf(mx, sc[kb][r]);
  mx = fmaxf(mx, __shfl_xor(mx, 32)) * c;
  // Exact running max, as the reference (relpos_attention.py:48-50): the step's largest
  // score maps to p = 1, which bf16 holds exactly. The accumulators are only rescaled when
  // some lane's max moved.
  const bool need = mx > m_run;
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
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
    float p[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) p[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[kb][r], c, negm));
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const u32x4 pb = pack8(&p[8 * u]);
#pragma unroll
      for (int w = 0; w < 4; ++w) l_run[w & 1] = add_bf16_pair(pb[w], l_run[w & 1]);
      const int k0 = kb * 32 + 16 * u + 4 * g;
#pragma unroll
      for (int db = 0; db < G::DB; ++db)
        oacc[db] = mfma32x32x16(tr_operand(Vs, G::RLD, k0, k0 + 8, db * 32 + c0), pb, oacc[db]);
    }
  }
}

template <int DP, int NW>
__global__ __launch_bounds__(64 * NW, 2) void relpos_fwd_kernel(
    const uint16_t* __restrict__ qkv, int64_t ld, const float* __restrict__ pd,
    uint16_t* __restrict__ out, float* __restrict__ out32, float* __restrict__ lse, int S, int H,
    int D, Fold f) {
  using G = Geo<DP>;
  using K = Blk<NW>;
  constexpr int CPT = Tile<DP, K::NT>::CPT;
  __shared__ __attribute__((aligned(16))) uint16_t Ks[kStep * G::RLD];
  __shared__ __attribute__((aligned(16))) uint16_t Vs[kStep * G::RLD];
  __shared__ __attribute__((aligned(16))) float Bw[4 * K::WLD];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, g = lane >> 5, l32 = lane & 31;
  const int bh = blockIdx.y, b = bh / H, h = bh - b * H;
  const int i_wg = blockIdx.x * K::ROWS;
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
  const int c0 = 16 * ((lane >> 4) & 1);
  const float c = f.c;

  zero_pad_cols<DP, K::NT>(Vs);

  u32x4 qreg[G::KS];
#pragma unroll
  for (int s = 0; s < G::KS; ++s) {
    const int d0 = 16 * s + 8 * g;
    qreg[s] = (qvalid && d0 < D) ? fold_operand(ld16(q0 + (int64_t)qi * ld + d0), f) : kZero4;
  }

  f32x16 oacc[G::DB];
#pragma unroll
  for (int db = 0; db < G::DB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) oacc[db][r] = 0.f;
  float m_run = -INFINITY, l_run[2] = {0.f, 0.f};

  uint32_t voff[CPT];
  tile_offsets<DP, K::NT>(voff, ld, D);
  u32x4 kst[CPT], vst[CPT];
  float bst[K::BPT];
  const int T = (S + kStep - 1) / kStep;
  // Window base of step t: entry x is table index wb + x, wb = j0 - i_wg - (ROWS-1) + S-1.
  const int wb0 = S - 1 - i_wg - (K::ROWS - 1);
  load_tile<DP, K::NT>(kst, voff, k0p, ld, 0, S, D);
  load_tile<DP, K::NT>(vst, voff, v0p, ld, 0, S, D);
  load_bias<NW>(bst, pdh, npd, wb0, 1, f.bmul);

  // Stage step t (stash the prefetched tile, then prefetch step t+1).
  auto stage = [&](int t) {
    const int j1 = (t + 1) * kStep;
    __syncthreads();
    stash_tile<DP, K::NT>(kst, Ks);
    stash_tile<DP, K::NT>(vst, Vs);
    stash_bias<NW>(bst, Bw);
    __syncthreads();
    if (t + 1 < T) {
      load_tile<DP, K::NT>(kst, voff, k0p, ld, j1, S, D);
      load_tile<DP, K::NT>(vst, voff, v0p, ld, j1, S, D);
      load_bias<NW>(bst, pdh, npd, wb0 + j1, 1, f.bmul);
    }
  };
  // Full 64-key steps carry no key mask; a partial last step (S % 64 != 0) runs once after
  // the loop, so the loop body holds a single copy of the step.
  const int Tfull = S / kStep;
  for (int t = 0; t < Tfull; ++t) {
    stage(t);
    fwd_step<DP, NW, false>(Ks, Vs, Bw, qreg, oacc, m_run, l_run, t * kStep, S, ii, g, l32, c0, c);
  }
  if (Tfull < T) {
    stage(Tfull);
    fwd_step<DP, NW, true>(Ks, Vs, Bw, qreg, oacc, m_run, l_run, Tfull * kStep, S, ii, g, l32, c0, c);
  }

  const float lh = l_run[0] + l_run[1];
  const float l = lh + __shfl_xor(lh, 32);
  if (qvalid) {
    const int64_t obase = (tok0 + qi) * HD + (int64_t)h * D;
#pragma unroll
    for (int db = 0; db < G::DB; ++db)
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const int d0 = db * 32 + 8 * a + 4 * g;
        if (d0 < D) {
          f32x4 o;
#pragma unroll
          for (int b4 = 0; b4 < 4; ++b4) o[b4] = oacc[db][4 * a + b4] / l;
          *reinterpret_cast<f32x4*>(out32 + obase + d0) = o;
          uint2 ob;
          ob.x = pack_bf16x2(o[0], o[1]);
          ob.y = pack_bf16x2(o[2], o[3]);
          *reinterpret_cast<uint2*>(out + obase + d0) = ob;
        }
      }
    if (g == 0) lse[(int64_t)bh * S + qi] = m_run + log2f(l);
  }
}

// ------------------------------------------------ backward: delta, dQ and dpd
// Diagonal ring of the dQ kernel: RING slots indexed by diagonal mod RING, plus a
// 32-slot overflow zone that aliases slots 0..31, so the 16 updates of one D tile
// (diagonals base + 8a + b, a, b < 4) use one base register and immediate offsets.
// Folding a diagonal reads (and clears) both of its slots.
template <int NW>
__device__ __forceinline__ float ring_take(float (*ring)[Blk<NW>::RING + 32], int slot, bool clear) {
  constexpr int RING = Blk<NW>::RING;
  float v = 0.f;
#pragma unroll
  for (int k = 0; k < 2 * NW; ++k) {
    v += ring[k][slot];
    if (clear) ring[k][slot] = 0.f;
    if (slot < 32) {
      v += ring[k][slot + RING];
      if (clear) ring[k][slot + RING] = 0.f;
    }
  }
  return v;
}

// One 64-key step of the dQ kernel for this lane's query: p = exp2(acc c - lse),
// ds = p (dp - delta), ds into the diagonal ring, dQ^T += K^T dS^T. Invalid
// query lanes carry lse = +inf, so their p is 0 without a mask; TAIL masks keys
// >= S (last step only).
template <int DP, int NW, bool TAIL>
__device__ __forceinline__ void dq_step(const uint16_t* Ks, const uint16_t* Vs, const float* Bw,
                                        float* myring, const u32x4* qreg, const u32x4* doreg,
                                        f32x16* dq, float neg_lse, float delta, int j0, int S, int ii,
                                        int g, int l32, int c0, float c) {
  using G = Geo<DP>;
  using K = Blk<NW>;
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
    const int x0 = kb * 32 + 4 * g + (K::ROWS - 1) - ii;
    f32x16 acc = read_bias16<NW>(Bw, x0), accp;
#pragma unroll
    for (int r = 0; r < 16; ++r) accp[r] = 0.f;
#pragma unroll
    for (int s = 0; s < G::KS; ++s) {
      acc = mfma32x32x16(ld16(Ks + (kb * 32 + l32) * G::RLD + 16 * s + 8 * g), qreg[s], acc);
      accp = mfma32x32x16(ld16(Vs + (kb * 32 + l32) * G::RLD + 16 * s + 8 * g), doreg[s], accp);
    }
    float ds[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      float p = __builtin_amdgcn_exp2f(__builtin_fmaf(acc[r], c, neg_lse));
      if (TAIL && j0 + kb * 32 + 8 * (r >> 2) + 4 * g + (r & 3) >= S) p = 0.f;
      ds[r] = p * (accp[r] - delta);
    }
    // Diagonal of D-register r: j - i + ROWS - 1 - i_wg = j0 + x0 + 8a + b. Within one
    // register the 32 lanes of a half hit 32 distinct diagonals of their own ring, and LDS
    // operations of a wave complete in order, so a plain read-modify-write per register is
    // exact (LDS float atomics cost ~30x more here). Lanes ii and ii+1 reach the same
    // diagonal through neighbouring registers, so the read-modify-writes must stay in
    // register order: the accesses are volatile, which forbids batching the reads ahead of
    // the writes (the compiler only sees that one lane's 16 slots are distinct).
    volatile lds_f32* rp = (volatile lds_f32*)myring + ((j0 + x0) & (K::RING - 1));
#pragma unroll
    for (int r = 0; r < 16; ++r) rp[8 * (r >> 2) + (r & 3)] = rp[8 * (r >> 2) + (r & 3)] + ds[r];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const u32x4 dsb = pack8(&ds[8 * u]);
      const int k0 = kb * 32 + 16 * u + 4 * g;
#pragma unroll
      for (int db = 0; db < G::DB; ++db)
        dq[db] = mfma32x32x16(tr_operand(Ks, G::RLD, k0, k0 + 8, db * 32 + c0), dsb, dq[db]);
    }
  }
}

template <int DP, int NW>
__global__ __launch_bounds__(64 * NW, (DP <= 96 ? 2 : 1)) void relpos_bwd_dq_kernel(
    const uint16_t* __restrict__ qkv, int64_t ld, const float* __restrict__ pd,
    const uint16_t* __restrict__ dout, const float* __restrict__ out32,
    const float* __restrict__ lse, float* __restrict__ delta_ws, float* __restrict__ part,
    uint16_t* __restrict__ dqkv, int64_t ldd, int S, int H, int D, Fold f, float scale) {
  using G = Geo<DP>;
  using K = Blk<NW>;
  constexpr int CPT = Tile<DP, K::NT>::CPT;
  constexpr int RING = K::RING;
  __shared__ __attribute__((aligned(16))) uint16_t Ks[kStep * G::RLD];
  __shared__ __attribute__((aligned(16))) uint16_t Vs[kStep * G::RLD];
  __shared__ __attribute__((aligned(16))) float Bw[4 * K::WLD];
  __shared__ float ring[2 * NW][RING + 32];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, g = lane >> 5, l32 = lane & 31;
  const int bh = blockIdx.y, b = bh / H, h = bh - b * H;
  const int i_wg = blockIdx.x * K::ROWS;
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
  const int RS = S + K::ROWS;         // partial row stride
  const int rlen = S + K::ROWS - 1;   // diagonals one query block touches
  float* prow = part + ((int64_t)bh * gridDim.x + blockIdx.x) * RS;
  const int c0 = 16 * ((lane >> 4) & 1);
  const float c = f.c;

  zero_pad_cols<DP, K::NT>(Ks);
  for (int e = tid; e < 2 * NW * (RING + 32); e += K::NT) (&ring[0][0])[e] = 0.f;

  // Register-resident operands and per-query statistics.
  u32x4 qreg[G::KS], doreg[G::KS];
  float dsum = 0.f;
  const int64_t obase = (tok0 + qi) * HD + (int64_t)h * D;
#pragma unroll
  for (int s = 0; s < G::KS; ++s) {
    const int d0 = 16 * s + 8 * g;
    const bool ok = qvalid && d0 < D;
    qreg[s] = ok ? fold_operand(ld16(q0 + (int64_t)qi * ld + d0), f) : kZero4;
    doreg[s] = ok ? ld16(dout + obase + d0) : kZero4;
    if (ok) {
      const f32x4 o0 = *reinterpret_cast<const f32x4*>(out32 + obase + d0);
      const f32x4 o1 = *reinterpret_cast<const f32x4*>(out32 + obase + d0 + 4);
      float df[8];
      unpack8(doreg[s], df);
#pragma unroll
      for (int e = 0; e < 4; ++e) dsum += df[e] * o0[e];
#pragma unroll
      for (int e = 0; e < 4; ++e) dsum += df[4 + e] * o1[e];
    }
  }
  const float delta = dsum + __shfl_xor(dsum, 32);
  // -inf makes p = exp2(acc c - lse) exactly 0 on lanes past S (their acc is finite).
  const float neg_lse = qvalid ? -lse[(int64_t)bh * S + qi] : -INFINITY;
  if (qvalid && g == 0) delta_ws[(int64_t)bh * S + qi] = delta;

  f32x16 dq[G::DB];
#pragma unroll
  for (int db = 0; db < G::DB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) dq[db][r] = 0.f;

  float* myring = ring[wave * 2 + g];
  uint32_t voff[CPT];
  tile_offsets<DP, K::NT>(voff, ld, D);
  u32x4 kst[CPT], vst[CPT];
  float bst[K::BPT];
  const int T = (S + kStep - 1) / kStep;
  const int wb0 = S - 1 - i_wg - (K::ROWS - 1);
  load_tile<DP, K::NT>(kst, voff, k0p, ld, 0, S, D);
  load_tile<DP, K::NT>(vst, voff, v0p, ld, 0, S, D);
  load_bias<NW>(bst, pdh, npd, wb0, 1, f.bmul);

  // Stage step t (stash the prefetched tile, prefetch step t+1, fold finished diagonals).
  auto stage = [&](int t) {
    const int j1 = (t + 1) * kStep;
    __syncthreads();
    stash_tile<DP, K::NT>(kst, Ks);
    stash_tile<DP, K::NT>(vst, Vs);
    stash_bias<NW>(bst, Bw);
    __syncthreads();
    if (t + 1 < T) {
      load_tile<DP, K::NT>(kst, voff, k0p, ld, j1, S, D);
      load_tile<DP, K::NT>(vst, voff, v0p, ld, j1, S, D);
      load_bias<NW>(bst, pdh, npd, wb0 + j1, 1, f.bmul);
    }
    // Diagonals r in [64(t-1), 64t) received their last contribution in
    // iteration t-1: fold the rings in order into the partial row.
    if (t > 0 && wave == 0) {
      const int r = (t - 1) * kStep + lane;
      prow[r] = ring_take<NW>(ring, r & (RING - 1), true);
    }
  };
  // Full 64-key steps carry no key mask; a partial last step runs once after the loop.
  const int Tfull = S / kStep;
  for (int t = 0; t < Tfull; ++t) {
    stage(t);
    dq_step<DP, NW, false>(Ks, Vs, Bw, myring, qreg, doreg, dq, neg_lse, delta, t * kStep, S, ii,
                           g, l32, c0, c);
  }
  if (Tfull < T) {
    stage(Tfull);
    dq_step<DP, NW, true>(Ks, Vs, Bw, myring, qreg, doreg, dq, neg_lse, delta, Tfull * kStep, S,
                          ii, g, l32, c0, c);
  }

  __syncthreads();
  for (int r = (T - 1) * kStep + tid; r < rlen; r += K::NT) prow[r] = ring_take<NW>(ring, r & (RING - 1), false);

  if (qvalid) {
    const int64_t qbase = (tok0 + qi) * ldd + (int64_t)h * D;
#pragma unroll
    for (int db = 0; db < G::DB; ++db)
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const int d0 = db * 32 + 8 * a + 4 * g;
        if (d0 < D) {
          uint2 ob;
          ob.x = pack_bf16x2(dq[db][4 * a] * scale, dq[db][4 * a + 1] * scale);
          ob.y = pack_bf16x2(dq[db][4 * a + 2] * scale, dq[db][4 * a + 3] * scale);
          *reinterpret_cast<uint2*>(dqkv + qbase + d0) = ob;
        }
      }
  }
}

// ---------------------------------------------------------- backward: dK, dV
template <int DP, int NW>
__global__ __launch_bounds__(64 * NW, (DP <= 64 ? 2 : 1)) void relpos_bwd_dkdv_kernel(
    const uint16_t* __restrict__ qkv, int64_t ld, const float* __restrict__ pd,
    const uint16_t* __restrict__ dout, const float* __restrict__ lse,
    const float* __restrict__ delta_ws, uint16_t* __restrict__ dqkv, int64_t ldd, int S, int H,
    int D, Fold f, float scale) {
  using G = Geo<DP>;
  using K = Blk<NW>;
  constexpr int CPT = Tile<DP, K::NT>::CPT;
  __shared__ __attribute__((aligned(16))) uint16_t Qs[kStep * G::RLD];
  __shared__ __attribute__((aligned(16))) uint16_t Os[kStep * G::RLD];
  __shared__ __attribute__((aligned(16))) float Lq[kStep];
  __shared__ __attribute__((aligned(16))) float Dq[kStep];
  __shared__ __attribute__((aligned(16))) float Bw[4 * K::WLD];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, g = lane >> 5, l32 = lane & 31;
  const int bh = blockIdx.y, b = bh / H, h = bh - b * H;
  const int j_wg = blockIdx.x * K::ROWS;
  const int kk = wave * 32 + l32;
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
  const int c0 = 16 * ((lane >> 4) & 1);
  const float c = f.c;

  zero_pad_cols<DP, K::NT>(Qs);
  zero_pad_cols<DP, K::NT>(Os);

  u32x4 kreg[G::KS], vreg[G::KS];
#pragma unroll
  for (int s = 0; s < G::KS; ++s) {
    const int d0 = 16 * s + 8 * g;
    const bool ok = kvalid && d0 < D;
    kreg[s] = ok ? fold_operand(ld16(q0 + HD + (int64_t)kj * ld + d0), f) : kZero4;
    vreg[s] = ok ? ld16(q0 + 2 * HD + (int64_t)kj * ld + d0) : kZero4;
  }

  f32x16 dk[G::DB], dv[G::DB];
#pragma unroll
  for (int db = 0; db < G::DB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) dk[db][r] = dv[db][r] = 0.f;

  uint32_t qoff[CPT], ooff[CPT];
  tile_offsets<DP, K::NT>(qoff, ld, D);
  tile_offsets<DP, K::NT>(ooff, HD, D);
  u32x4 qst[CPT], ost[CPT];
  float bst[K::BPT];
  float sst = 0.f;
  const int T = (S + kStep - 1) / kStep;
  // Per-query statistics of the step: threads 0..63 -lse, 64..127 delta. Rows past S get
  // -lse = -inf, which makes their p = exp2(acc c - lse) exactly 0 (acc is finite there).
  auto stats = [&](int i0) {
    const int q = i0 + (tid & 63);
    if (tid < 128) sst = q < S ? (tid < 64 ? -lse_bh[q] : dl_bh[q]) : (tid < 64 ? -INFINITY : 0.f);
  };
  // Reversed window: entry x holds T[rb - x], rb = (j_wg + ROWS - 1) - i0 + S - 1 the largest
  // diagonal of the step.
  const int rb0 = (j_wg + K::ROWS - 1) + S - 1;
  load_tile<DP, K::NT>(qst, qoff, q0, ld, 0, S, D);
  load_tile<DP, K::NT>(ost, ooff, o0, HD, 0, S, D);
  load_bias<NW>(bst, pdh, npd, rb0, -1, f.bmul);
  stats(0);

  for (int t = 0; t < T; ++t) {
    const int i1 = (t + 1) * kStep;
    __syncthreads();
    stash_tile<DP, K::NT>(qst, Qs);
    stash_tile<DP, K::NT>(ost, Os);
    stash_bias<NW>(bst, Bw);
    if (tid < 64)
      Lq[tid] = sst;
    else if (tid < 128)
      Dq[tid - 64] = sst;
    __syncthreads();
    if (t + 1 < T) {
      load_tile<DP, K::NT>(qst, qoff, q0, ld, i1, S, D);
      load_tile<DP, K::NT>(ost, ooff, o0, HD, i1, S, D);
      load_bias<NW>(bst, pdh, npd, rb0 - i1, -1, f.bmul);
      stats(i1);
    }
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      f32x16 acc = read_bias16<NW>(Bw, (K::ROWS - 1) - kk + qb * 32 + 4 * g), accp;
#pragma unroll
      for (int r = 0; r < 16; ++r) accp[r] = 0.f;
#pragma unroll
      for (int s = 0; s < G::KS; ++s) {
        acc = mfma32x32x16(ld16(Qs + (qb * 32 + l32) * G::RLD + 16 * s + 8 * g), kreg[s], acc);
        accp = mfma32x32x16(ld16(Os + (qb * 32 + l32) * G::RLD + 16 * s + 8 * g), vreg[s], accp);
      }
      float p[16], ds[16];
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const f32x4 nl4 = *reinterpret_cast<const f32x4*>(Lq + qb * 32 + 8 * a + 4 * g);
        const f32x4 d4 = *reinterpret_cast<const f32x4*>(Dq + qb * 32 + 8 * a + 4 * g);
#pragma unroll
        for (int b4 = 0; b4 < 4; ++b4) {
          const int r = 4 * a + b4;
          const float pv = __builtin_amdgcn_exp2f(__builtin_fmaf(acc[r], c, nl4[b4]));
          p[r] = pv;
          ds[r] = pv * (accp[r] - d4[b4]);
        }
      }
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const u32x4 pa = pack8(&p[8 * u]);
        const u32x4 dsa = pack8(&ds[8 * u]);
        const int k0 = qb * 32 + 16 * u + 4 * g;
#pragma unroll
        for (int db = 0; db < G::DB; ++db) {
          dv[db] = mfma32x32x16(pa, tr_operand(Os, G::RLD, k0, k0 + 8, db * 32 + c0), dv[db]);
          dk[db] = mfma32x32x16(dsa, tr_operand(Qs, G::RLD, k0, k0 + 8, db * 32 + c0), dk[db]);
        }
      }
    }
  }

  // D layout: lane = head dim d (n), register r = key 8(r/4) + 4g + r%4 of this wave.
#pragma unroll
  for (int db = 0; db < G::DB; ++db) {
    const int d = db * 32 + l32;
    if (d < D) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = j_wg + wave * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
        if (key < S) {
          uint16_t* rowp = dqkv + (tok0 + key) * ldd + HD + (int64_t)h * D + d;
          rowp[0] = f32_to_bf16(dk[db][r] * scale);
          rowp[HD] = f32_to_bf16(dv[db][r]);
        }
      }
    }
  }
}

// dpd[h, k] = sum over b and query blocks of the partial rows, fixed order.
// Block: 64 diagonals (lane) of head h; the 4 waves take every 4th (b, query
// block) term, then the 4 wave sums are added in wave order.
__global__ __launch_bounds__(256) void relpos_dpd_reduce(const float* __restrict__ part,
                                                         float* __restrict__ dpd, int B, int S,
                                                         int H, int nqb, int rows) {
  __shared__ float s[4][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int k = blockIdx.x * 64 + lane;
  const int h = blockIdx.y;
  const int npd = 2 * S - 1;
  const int RS = S + rows;
  const int rlen = S + rows - 1;
  float acc = 0.f;
  if (k < npd) {
    const int terms = B * nqb;
#pragma unroll 4
    for (int e = wave; e < terms; e += 4) {
      const int b = e / nqb, qb = e - b * nqb;
      const int r = k - S + rows + rows * qb;
      if (r >= 0 && r < rlen) acc += part[((int64_t)(b * H + h) * nqb + qb) * RS + r];
    }
  }
  s[wave][lane] = acc;
  __syncthreads();
  if (wave == 0 && k < npd)
    dpd[(int64_t)h * npd + k] = ((s[0][lane] + s[1][lane]) + s[2][lane]) + s[3][lane];
}

// Waves per workgroup of the three attention kernels.
constexpr int kFwdNW = 4;
constexpr int kDqNW = 4;
constexpr int kDkdvNW = 4;

// Smallest nonzero |scale| * log2(e) the folded bias accepts: pd * log2(e) / c must
// stay finite for any realistic table.
constexpr float kMinScaleLog2 = 8.67361737988403547e-19f;  // 2^-60

int check_attn(const void* qkv, int64_t ld, int B, int S, int H, int D, float scale) {
  if (B <= 0 || S <= 0 || H <= 0 || D <= 0) return KRSI_ERR_BAD_SHAPE;
  if (D % 8 != 0 || D > 128) return KRSI_ERR_UNSUPPORTED;
  if ((int64_t)B * H > 65535 || S > (1 << 24)) return KRSI_ERR_BAD_SHAPE;
  if (ld < 3 * (int64_t)H * D) return KRSI_ERR_BAD_SHAPE;
  // Buffer resources of one (batch, head) slice hold S rows of ld bf16 in < 2^31 bytes.
  if ((int64_t)S * ld * 2 >= ((int64_t)1 << 31)) return KRSI_ERR_UNSUPPORTED;
  if (ld % 8 != 0 || !aligned16(qkv)) return KRSI_ERR_MISALIGNED;
  if (!(scale == scale) || scale > 3.0e38f || scale < -3.0e38f) return KRSI_ERR_BAD_SCALE;
  const float c = fabsf(scale * kLog2e);
  if (c != 0.f && c < kMinScaleLog2) return KRSI_ERR_BAD_SCALE;
  return KRSI_OK;
}

Fold fold_scale(float scale) {
  const float c = scale * kLog2e;
  if (c == 0.f) return Fold{1.f, kLog2e, 0u, 0u};
  const float a = fabsf(c);
  return Fold{a, kLog2e / a, 0xffffffffu, c < 0.f ? 0x80008000u : 0u};
}

int padded_dim(int D) { return (D + 15) / 16 * 16; }

constexpr int kDqRows = Blk<kDqNW>::ROWS;

size_t ws_delta_bytes(int B, int S, int H) { return align256((size_t)B * H * S * sizeof(float)); }
size_t ws_part_bytes(int B, int S, int H) {
  const size_t nqb = (size_t)ceil_div(S, kDqRows);
  return align256((size_t)B * H * nqb * (size_t)(S + kDqRows) * sizeof(float));
}

template <int DP>
void launch_fwd(const void* qkv, int64_t ld, const float* pd, void* out, float* out32, float* lse,
                int B, int S, int H, int D, Fold f, hipStream_t st) {
  using K = Blk<kFwdNW>;
  const dim3 grid((unsigned)ceil_div(S, K::ROWS), (unsigned)(B * H));
  hipLaunchKernelGGL((relpos_fwd_kernel<DP, kFwdNW>), grid, dim3(K::NT), 0, st,
                     (const uint16_t*)qkv, ld, pd, (uint16_t*)out, out32, lse, S, H, D, f);
}

template <int DP>
void launch_bwd(const void* dout, const void* qkv, int64_t ld, const float* pd, const float* out32,
                const float* lse, void* dqkv, int64_t ldd, float* dpd, void* ws, int B, int S, int H,
                int D, Fold f, float scale, hipStream_t st) {
  using KQ = Blk<kDqNW>;
  using KK = Blk<kDkdvNW>;
  float* delta = static_cast<float*>(ws);
  float* part = reinterpret_cast<float*>(static_cast<char*>(ws) + ws_delta_bytes(B, S, H));
  const int nqb = (int)ceil_div(S, KQ::ROWS);
  hipLaunchKernelGGL((relpos_bwd_dq_kernel<DP, kDqNW>), dim3((unsigned)nqb, (unsigned)(B * H)),
                     dim3(KQ::NT), 0, st, (const uint16_t*)qkv, ld, pd, (const uint16_t*)dout, out32,
                     lse, delta, part, (uint16_t*)dqkv, ldd, S, H, D, f, scale);
  hipLaunchKernelGGL((relpos_bwd_dkdv_kernel<DP, kDkdvNW>),
                     dim3((unsigned)ceil_div(S, KK::ROWS), (unsigned)(B * H)), dim3(KK::NT), 0, st,
                     (const uint16_t*)qkv, ld, pd, (const uint16_t*)dout, lse, (const float*)delta,
                     (uint16_t*)dqkv, ldd, S, H, D, f, scale);
  const dim3 rgrid((unsigned)ceil_div(2 * S - 1, 64), (unsigned)H);
  hipLaunchKernelGGL(relpos_dpd_reduce, rgrid, dim3(256), 0, st, (const float*)part, dpd, B, S, H,
                     nqb, KQ::ROWS);
}

}  // namespace
}  // namespace krsi

extern "C" {

int krsi_relpos_fwd_bf16(const void* qkv, int64_t ld_qkv, const float* pd, void* out, float* out32,
                         float* lse, int32_t B, int32_t S, int32_t H, int32_t D, float scale,
                         void* stream) {
  using namespace krsi;
  if (!qkv || !pd || !out || !out32 || !lse) return KRSI_ERR_NULL_POINTER;
  int rc = check_attn(qkv, ld_qkv, B, S, H, D, scale);
  if (rc != KRSI_OK) return rc;
  if (!aligned16(out) || !aligned16(out32)) return KRSI_ERR_MISALIGNED;
  const Fold f = fold_scale(scale);
  hipStream_t st = as_stream(stream);
  switch (padded_dim(D)) {
#define KRSI_CASE(DPV_)                                                                \
  case DPV_:                                                                           \
    launch_fwd<DPV_>(qkv, ld_qkv, pd, out, out32, lse, B, S, H, D, f, st);             \
    break;
    KRSI_CASE(16) KRSI_CASE(32) KRSI_CASE(48) KRSI_CASE(64) KRSI_CASE(80) KRSI_CASE(96)
    KRSI_CASE(112) KRSI_CASE(128)
#undef KRSI_CASE
    default:
      return KRSI_ERR_UNSUPPORTED;
  }
  return launch_status();
}

size_t krsi_relpos_bwd_workspace_bytes(int32_t B, int32_t S, int32_t H, int32_t D) {
  using namespace krsi;
  (void)D;
  if (B <= 0 || S <= 0 || H <= 0) return 0;
  return ws_delta_bytes(B, S, H) + ws_part_bytes(B, S, H);
}

int krsi_relpos_bwd_bf16(const void* dout, const void* qkv, int64_t ld_qkv, const float* pd,
                         const float* out32, const float* lse, void* dqkv, int64_t ld_dqkv,
                         float* dpd, void* workspace, size_t workspace_bytes, int32_t B, int32_t S,
                         int32_t H, int32_t D, float scale, void* stream) {
  using namespace krsi;
  if (!dout || !qkv || !pd || !out32 || !lse || !dqkv || !dpd) return KRSI_ERR_NULL_POINTER;
  int rc = check_attn(qkv, ld_qkv, B, S, H, D, scale);
  if (rc != KRSI_OK) return rc;
  if (ld_dqkv < 3 * (int64_t)H * D) return KRSI_ERR_BAD_SHAPE;
  if (ld_dqkv % 8 != 0 || !aligned16(dqkv) || !aligned16(dout) || !aligned16(out32))
    return KRSI_ERR_MISALIGNED;
  if (!workspace || workspace_bytes < krsi_relpos_bwd_workspace_bytes(B, S, H, D))
    return KRSI_ERR_WORKSPACE;
  if (!aligned16(workspace)) return KRSI_ERR_MISALIGNED;
  const Fold f = fold_scale(scale);
  hipStream_t st = as_stream(stream);
  switch (padded_dim(D)) {
#define KRSI_CASE(DPV_)                                                                      \
  case DPV_:                                                                                 \
    launch_bwd<DPV_>(dout, qkv, ld_qkv, pd, out32, lse, dqkv, ld_dqkv, dpd, workspace, B, S, \
                     H, D, f, scale, st);                                                    \
    break;
    KRSI_CASE(16) KRSI_CASE(32) KRSI_CASE(48) KRSI_CASE(64) KRSI_CASE(80) KRSI_CASE(96)
    KRSI_CASE(112) KRSI_CASE(128)
#undef KRSI_CASE
    default:
      return KRSI_ERR_UNSUPPORTED;
  }
  return launch_status();
}

}  // extern "C"
