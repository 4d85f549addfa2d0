/*
 * krsi.h - C ABI of libkrsi_hip.so, the gfx950 (MI355X) kernels behind the
 * kernel-rsi fused library: RMSNorm, GEGLU and relative-position-bias flash
 * attention, forward and backward.
 *
 * Conventions shared by every entry point:
 *   - All tensor pointers are DEVICE pointers; the caller owns all memory.
 *     The library never allocates, frees or synchronises, so every call can be
 *     captured into a HIP graph.
 *   - `stream` is a hipStream_t (NULL = the legacy default stream). Launches
 *     are asynchronous on that stream.
 *   - Every argument is validated before the first launch; on error nothing
 *     has been launched. The return value is KRSI_OK (0) or one of the
 *     KRSI_ERR_* codes; krsi_error_string() names it.
 *   - Activations (x, w, g, y, dx, dw; u, out, du; qkv, dout, out, dqkv) are
 *     row-major in one dtype chosen by a KRSI_DTYPE_* argument: bf16 and fp16
 *     as raw 16-bit patterns, or fp32. Every rounding point the reference
 *     applies in its input dtype (`.to(x.dtype)`, products of two tensors of
 *     that dtype) is applied in that dtype, round-to-nearest-even. Statistics
 *     (rstd, lse, out32, pd, dpd) are always fp32. The *_bf16 entry points are
 *     the same functions with dtype fixed to KRSI_DTYPE_BF16.
 *   - Stateless and reentrant: any host thread may call, ordering is by stream.
 *     The one exception is krsi_rmsnorm_bwd_noalloc, whose calls share a static
 *     per-device scratch array (see there).
 */
#ifndef KRSI_H_
#define KRSI_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KRSI_ABI_VERSION 3

/* Activation dtypes. The reference's Triton kernels are dtype-generic, and so is
 * every entry point here. */
#define KRSI_DTYPE_BF16 0
#define KRSI_DTYPE_F16 1
#define KRSI_DTYPE_F32 2

enum krsi_status {
  KRSI_OK = 0,
  KRSI_ERR_NULL_POINTER = 1,    /* a required pointer is NULL */
  KRSI_ERR_BAD_SHAPE = 2,       /* a size is <= 0 or out of the supported range */
  KRSI_ERR_MISALIGNED = 3,      /* a pointer or leading dimension breaks 16-byte alignment */
  KRSI_ERR_WORKSPACE = 4,       /* workspace missing or smaller than *_workspace_bytes() */
  KRSI_ERR_UNSUPPORTED = 5,     /* a mode, dtype or head dim this build does not implement */
  KRSI_ERR_LAUNCH = 6,          /* the HIP runtime rejected a kernel launch */
  KRSI_ERR_BAD_SCALE = 7,       /* scale or eps is not finite */
  KRSI_ERR_TOO_LARGE = 8        /* beyond the static scratch of a no-allocation entry point */
};

int krsi_abi_version(void);
const char* krsi_error_string(int status);

/* ------------------------------------------------------------------ RMSNorm
 * Replaces library/rmsnorm.py:54-59 (_fwd: the _rms_fwd launch, :22-31).
 *   rstd[r] = 1 / sqrt(sum_c x[r,c]^2 / n + eps)            (fp32)
 *   y[r,c]  = T( w[c] * T(x[r,c] * rstd[r]) )                 T = dtype
 * x, y: [rows, n] contiguous; w: [n]; all three of `dtype`; rstd: [rows] fp32.
 * Limits: 1 <= n <= 16384, rows >= 1 (rows == 0 is a no-op).        */
int krsi_rmsnorm_fwd(const void* x, const void* w, void* y, float* rstd, int64_t rows,
                     int32_t n, float eps, int32_t dtype, void* stream);
int krsi_rmsnorm_fwd_bf16(const void* x, const void* w, void* y, float* rstd,
                          int64_t rows, int32_t n, float eps, void* stream);

/* Replaces library/rmsnorm.py:62-68 (_bwd: _rms_bwd :34-51 plus the torch
 * `dwp.sum(0).to(w.dtype)` reduction of the per-program partials).
 *   nrm   = T(x * rstd);  dn = float(T(g * w))                       T = dtype
 *   dx    = rstd*dn - x*rstd^3 * sum_c(dn*x)/n                        (T out)
 *   dw[c] = T( sum_r g[r,c] * nrm[r,c] )      fp32 accumulation, fixed order
 * workspace: at least krsi_rmsnorm_bwd_workspace_bytes(rows, n) bytes of
 * device memory (fp32 per-block partials; the size is the same for every
 * dtype); its contents on entry are ignored. */
size_t krsi_rmsnorm_bwd_workspace_bytes(int64_t rows, int32_t n);
int krsi_rmsnorm_bwd(const void* g, const void* x, const void* w, const float* rstd, void* dx,
                     void* dw, void* workspace, size_t workspace_bytes, int64_t rows, int32_t n,
                     int32_t dtype, void* stream);
int krsi_rmsnorm_bwd_bf16(const void* g, const void* x, const void* w, const float* rstd,
                          void* dx, void* dw, void* workspace, size_t workspace_bytes,
                          int64_t rows, int32_t n, void* stream);

/* No counterpart in the reference. It exists for callers that cannot allocate:
 * code under HIP graph capture, serving loops and harnesses that forbid
 * hipMalloc. It is krsi_rmsnorm_bwd (same arguments, kernels and bitwise
 * results) without the workspace arguments. The partial rows go to a static
 * 16 MiB device array of the library:
 *   - each GPU holds its own copy from library load until the process ends;
 *   - the copy used is the current device's (the stream must belong to it);
 *   - its address is looked up once per device on the first call.
 * Limit: krsi_rmsnorm_bwd_workspace_bytes(rows, n) <= 16 MiB. That holds for
 * every row count when n <= 8192, and for fewer rows above that (n = 16384:
 * rows <= 256). Larger problems return KRSI_ERR_TOO_LARGE before anything is
 * launched.
 * Allocates nothing: no hipMalloc, hipFree or allocating library call.
 * Calls that overlap on one GPU (several streams or host threads) share the
 * array and race; serialise them. The array keeps the last call's contents.
 * None of them needs to start at zero. */
int krsi_rmsnorm_bwd_noalloc(const void* g, const void* x, const void* w, const float* rstd,
                             void* dx, void* dw, int64_t rows, int32_t n, int32_t dtype,
                             void* stream);

/* -------------------------------------------------------------------- GEGLU
 * Replaces library/geglu.py:55-61 (_fwd: _geglu_fwd :27-35).
 * u: [rows, 2f] contiguous, a = u[:, :f], b = u[:, f:]; out: [rows, f]; both of
 * `dtype` (T):
 *   out = T( T(gelu(a)) * b )
 * approximate: 1 = tanh form (the reference's only form, geglu.py:20-24),
 *              0 = exact erf form (torch.nn.functional.gelu default).      */
int krsi_geglu_fwd(const void* u, void* out, int64_t rows, int32_t f, int32_t approximate,
                   int32_t dtype, void* stream);
int krsi_geglu_fwd_bf16(const void* u, void* out, int64_t rows, int32_t f,
                        int32_t approximate, void* stream);

/* Replaces library/geglu.py:64-68 (_bwd: _geglu_bwd :38-52).
 * g: [rows, f]; du: [rows, 2f] = [da | db]; all of `dtype` (T):
 *   db = T( g * T(gelu(a)) );  da = T( float(T(g*b)) * gelu'(a) )          */
int krsi_geglu_bwd(const void* g, const void* u, void* du, int64_t rows, int32_t f,
                   int32_t approximate, int32_t dtype, void* stream);
int krsi_geglu_bwd_bf16(const void* g, const void* u, void* du, int64_t rows, int32_t f,
                        int32_t approximate, void* stream);

/* Merged gate|up projection with the GEGLU forward as its epilogue (the merged GEMM
 * whose output library/geglu.py:3-5 takes as u), without writing u to memory:
 *   u   = T(x w^T)      x: [rows, k], w: [2f, k] = [W_gate; W_up] (nn.Linear layout)
 *   out = T( T(gelu(u[:, :f])) * u[:, f:] )                        out: [rows, f]
 * with the rounding points of krsi_geglu_fwd applied to the GEMM output rounded to T.
 * dtype: KRSI_DTYPE_BF16 or KRSI_DTYPE_F16 (T). Limits: k % 64 == 0, f % 64 == 0,
 * 128 * k * 2 < 2^31; x and w 16-byte aligned, contiguous. */
int krsi_geglu_linear_fwd(const void* x, const void* w, void* out, int64_t rows, int32_t k,
                          int32_t f, int32_t approximate, int32_t dtype, void* stream);

/* ------------------------------------------------- relative-position attention
 * Replaces library/relpos_attention.py:132-140 (_forward: _fwd :26-59).
 * dtype (T): KRSI_DTYPE_BF16 or KRSI_DTYPE_F16 run on 16-bit MFMA, and P is rounded
 * to T before the P V product, as the reference rounds it to v's dtype (:53).
 * KRSI_DTYPE_F32 runs on fp32 MFMA with every product in fp32. P is not
 * rounded, since v's dtype is fp32.
 * qkv: [B*S, ld_qkv] of T, unit column stride; token t = b*S + s holds
 *      q at columns [h*D, h*D+D), k at [H*D + h*D, ...), v at [2*H*D + h*D, ...).
 * pd:  [H, 2S-1] fp32, bias[h,i,j] = pd[h, j - i + S - 1].
 * out: [B*S, H*D] of T; out32: same, fp32; lse: [B*H, S] fp32 in the log2
 *      domain (lse = log2 sum_j 2^{(q.k*scale + bias) * log2(e)}). out32 and lse
 *      are what the backward needs; both may be NULL (not one alone) when no
 *      backward follows, and then only out is written (no counterpart in the
 *      reference, whose forward always writes both).
 * Limits: D % 8 == 0 and 8 <= D <= 128, ld_qkv >= 3*H*D, rows of a multiple
 *         of 16 bytes (ld_qkv % 8 == 0 for 16-bit T, % 4 for fp32), S >= 1,
 *         and for 16-bit T S * ld_qkv * 2 < 2^31 bytes (UNSUPPORTED otherwise),
 *         scale finite, and for 16-bit T scale == 0 or |scale| * log2(e) >=
 *         2^-60 (BAD_SCALE otherwise: the 16-bit kernels fold the bias into the
 *         score accumulator as pd * log2(e) / |scale * log2(e)|; the fp32 kernels
 *         add it directly and take any finite scale). Non-causal.            */
int krsi_relpos_fwd(const void* qkv, int64_t ld_qkv, const float* pd, void* out, float* out32,
                    float* lse, int32_t B, int32_t S, int32_t H, int32_t D, float scale,
                    int32_t dtype, void* stream);
int krsi_relpos_fwd_bf16(const void* qkv, int64_t ld_qkv, const float* pd, void* out,
                         float* out32, float* lse, int32_t B, int32_t S, int32_t H,
                         int32_t D, float scale, void* stream);

/* Replaces library/relpos_attention.py:143-157 (_backward_impl: the delta
 * reduction, _bwd_dkdv :62-94, _bwd_dq :97-126 and the torch diagonal sum of
 * dbias into dpd). No [B,H,S,S] buffer: dpd is reduced in-kernel along the
 * diagonals j - i, into per-block partials summed in a fixed order.
 * dout: [B*S, H*D] of T contiguous; dqkv: [B*S, ld_dqkv] of T (same column
 * layout as qkv, every q/k/v column written); dpd: [H, 2S-1] fp32 (overwritten).
 * P and dS are rounded to T before their products (:88-92, :125); for fp32
 * that is no rounding. ld_dqkv rows are a multiple of 16 bytes too.
 * workspace: krsi_relpos_bwd_workspace_bytes(B,S,H,D) bytes (grows as B H S^2
 * / 32: the dpd partial rows of every 128-key block) for the fastest path, or
 * anything down to krsi_relpos_bwd_workspace_min_bytes(B,S,H,D) (grows as
 * B H S: one block's rows). A smaller workspace runs the dK/dV kernel over as
 * many key blocks per launch as it holds, each launch's rows summed into dpd
 * before the next; dqkv is bitwise the same, dpd is the same sum in another
 * order (differences at fp32 rounding). Smaller than the minimum:
 * KRSI_ERR_WORKSPACE. The minimum has no counterpart in the reference (whose
 * backward materialises dbias [B,H,S,S]); it is for long-context callers that
 * must bound the backward's memory.                                          */
size_t krsi_relpos_bwd_workspace_bytes(int32_t B, int32_t S, int32_t H, int32_t D);
size_t krsi_relpos_bwd_workspace_min_bytes(int32_t B, int32_t S, int32_t H, int32_t D);
int krsi_relpos_bwd(const void* dout, const void* qkv, int64_t ld_qkv, const float* pd,
                    const float* out32, const float* lse, void* dqkv, int64_t ld_dqkv, float* dpd,
                    void* workspace, size_t workspace_bytes, int32_t B, int32_t S, int32_t H,
                    int32_t D, float scale, int32_t dtype, void* stream);
int krsi_relpos_bwd_bf16(const void* dout, const void* qkv, int64_t ld_qkv, const float* pd,
                         const float* out32, const float* lse, void* dqkv, int64_t ld_dqkv,
                         float* dpd, void* workspace, size_t workspace_bytes, int32_t B,
                         int32_t S, int32_t H, int32_t D, float scale, void* stream);

/* ------------------------------------ bucketed relative-position table (T5)
 * The steps either side of the attention when pd comes from a bucketed table
 * (an nn.Embedding [num_buckets, H] indexed by the bucket of j - i, as in T5).
 * The reference names this step without code (LESSONS.md:35: sum dBias along
 * the diagonals into [H, 2S-1], then into the buckets, with no scatter); the
 * attention backward above produces dpd [H, 2S-1], these finish the chain.
 * bucket: [2S-1] int32 device array, bucket[r] for distance j - i = r - (S-1)
 * (any map; T5's is built by the Python layer with the T5 formula).
 *
 * Gather: pd[h, r] = table[bucket[r] * H + h]; table [num_buckets, H] fp32,
 * pd [H, 2S-1] fp32. A bucket outside [0, num_buckets) writes NaN.        */
int krsi_relpos_bucket_gather(const float* table, const int32_t* bucket, float* pd, int32_t S,
                              int32_t H, int32_t num_buckets, void* stream);

/* Bucket sum (the gather's backward): dtable[b * H + h] = sum of dpd[h, r]
 * over r with bucket[r] == b, added in a fixed order (bitwise reproducible,
 * no atomics); every entry of dtable [num_buckets, H] is written.          */
int krsi_relpos_bucket_sum(const float* dpd, const int32_t* bucket, float* dtable, int32_t S,
                           int32_t H, int32_t num_buckets, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* KRSI_H_ */
