"""ctypes binding of libkrsi_hip.so (the C ABI declared in include/krsi.h) and the
host wrappers that validate tensors, allocate outputs and workspaces with the
torch caching allocator, and launch on torch's current stream.

There is no CPU or torch fallback: a call without the built library, or with
tensors that are not on a GPU, raises. The library is loaded lazily, after
torch, so that it binds to the HIP runtime torch has already loaded.
"""
from __future__ import annotations

import ctypes
import functools
import os
import threading
from pathlib import Path

import torch

ABI_VERSION = 3
LIB_PATH = Path(__file__).resolve().parent.parent / "libkrsi_hip.so"
# Cap in bytes on the attention backward's workspace (None: no cap, the fastest path). The
# dpd partial rows grow as B H S^2 / 32 bytes; under a cap the backward takes the key blocks
# in chunks (several dK/dV launches), never below one block's rows. Read from
# KRSI_RELPOS_BWD_WORKSPACE_MAX at import; assignable.
def _env_bytes(name: str) -> int | None:
    raw = os.environ.get(name, "").strip()
    if not raw:
        return None
    try:
        v = int(raw)
    except ValueError:
        raise ValueError(f"{name}={raw!r}: expected a byte count (integer)") from None
    return v if v > 0 else None


RELPOS_BWD_WORKSPACE_MAX: int | None = _env_bytes("KRSI_RELPOS_BWD_WORKSPACE_MAX")

# Names and signatures of every entry point of include/krsi.h.
_P, _I32, _I64, _F32, _SZ = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_float, ctypes.c_size_t
SIGNATURES = {
    "krsi_abi_version": (ctypes.c_int, []),
    "krsi_error_string": (ctypes.c_char_p, [ctypes.c_int]),
    "krsi_rmsnorm_fwd": (ctypes.c_int, [_P, _P, _P, _P, _I64, _I32, _F32, _I32, _P]),
    "krsi_rmsnorm_fwd_bf16": (ctypes.c_int, [_P, _P, _P, _P, _I64, _I32, _F32, _P]),
    "krsi_rmsnorm_bwd_workspace_bytes": (_SZ, [_I64, _I32]),
    "krsi_rmsnorm_bwd": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, _P, _SZ, _I64, _I32, _I32, _P]),
    "krsi_rmsnorm_bwd_bf16": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, _P, _SZ, _I64, _I32, _P]),
    "krsi_rmsnorm_bwd_noalloc": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, _I64, _I32, _I32, _P]),
    "krsi_geglu_fwd": (ctypes.c_int, [_P, _P, _I64, _I32, _I32, _I32, _P]),
    "krsi_geglu_fwd_bf16": (ctypes.c_int, [_P, _P, _I64, _I32, _I32, _P]),
    "krsi_geglu_bwd": (ctypes.c_int, [_P, _P, _P, _I64, _I32, _I32, _I32, _P]),
    "krsi_geglu_bwd_bf16": (ctypes.c_int, [_P, _P, _P, _I64, _I32, _I32, _P]),
    "krsi_geglu_linear_fwd": (ctypes.c_int, [_P, _P, _P, _I64, _I32, _I32, _I32, _I32, _P]),
    "krsi_relpos_fwd": (ctypes.c_int, [_P, _I64, _P, _P, _P, _P, _I32, _I32, _I32, _I32, _F32, _I32, _P]),
    "krsi_relpos_fwd_bf16": (ctypes.c_int, [_P, _I64, _P, _P, _P, _P, _I32, _I32, _I32, _I32, _F32, _P]),
    "krsi_relpos_bwd_workspace_bytes": (_SZ, [_I32, _I32, _I32, _I32]),
    "krsi_relpos_bwd_workspace_min_bytes": (_SZ, [_I32, _I32, _I32, _I32]),
    "krsi_relpos_bwd": (ctypes.c_int, [_P, _P, _I64, _P, _P, _P, _P, _I64, _P, _P, _SZ,
                                       _I32, _I32, _I32, _I32, _F32, _I32, _P]),
    "krsi_relpos_bwd_bf16": (ctypes.c_int, [_P, _P, _I64, _P, _P, _P, _P, _I64, _P, _P, _SZ,
                                            _I32, _I32, _I32, _I32, _F32, _P]),
    "krsi_relpos_bucket_gather": (ctypes.c_int, [_P, _P, _P, _I32, _I32, _I32, _P]),
    "krsi_relpos_bucket_sum": (ctypes.c_int, [_P, _P, _P, _I32, _I32, _I32, _P]),
}

# KRSI_DTYPE_* codes of the activation dtypes.
DTYPE_CODES = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}
_ATTN_DTYPES = (torch.bfloat16, torch.float16, torch.float32)

_lib = None
_lock = threading.Lock()


class KrsiError(RuntimeError):
    """A nonzero status from libkrsi_hip.so."""


def lib() -> ctypes.CDLL:
    """The loaded library (loaded and checked on first use)."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not LIB_PATH.is_file():
                    raise ImportError(f"{LIB_PATH} is not built; run `python kernel-rsi_amd/build.py` "
                                      "(or __graft_entry__.build()) first")
                handle = ctypes.CDLL(str(LIB_PATH))
                for name, (res, args) in SIGNATURES.items():
                    fn = getattr(handle, name)
                    fn.restype, fn.argtypes = res, args
                if handle.krsi_abi_version() != ABI_VERSION:
                    raise ImportError(f"{LIB_PATH}: ABI version {handle.krsi_abi_version()} != {ABI_VERSION}")
                _lib = handle
    return _lib


def _check(rc: int) -> None:
    if rc != 0:
        raise KrsiError(lib().krsi_error_string(rc).decode())


# torch's current-stream handle as an int. The raw accessor (the one torch's own Triton
# launchers use) skips building a Stream object: 0.1 against 1.9 us per call.
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(t: torch.Tensor) -> int:
    if _raw_stream is not None:
        return _raw_stream(t.device.index)
    return torch.cuda.current_stream(t.device).cuda_stream


@functools.lru_cache(maxsize=256)
def _rmsnorm_ws_bytes(rows: int, n: int) -> int:
    return lib().krsi_rmsnorm_bwd_workspace_bytes(rows, n)


@functools.lru_cache(maxsize=256)
def _relpos_ws_bytes(B: int, S: int, H: int, D: int) -> int:
    return lib().krsi_relpos_bwd_workspace_bytes(B, S, H, D)


@functools.lru_cache(maxsize=256)
def _relpos_ws_min_bytes(B: int, S: int, H: int, D: int) -> int:
    return lib().krsi_relpos_bwd_workspace_min_bytes(B, S, H, D)


def _on_gpu(*ts: torch.Tensor) -> None:
    for t in ts:
        if not t.is_cuda:
            raise ValueError("krsi kernels run on the GPU only: got a tensor on "
                             f"{t.device} (there is no CPU path)")
    dev = ts[0].device
    for t in ts[1:]:
        if t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} and {t.device}")


def _dtype(name: str, t: torch.Tensor, like: torch.Tensor | None = None,
           allowed: tuple = tuple(DTYPE_CODES)) -> int:
    """KRSI_DTYPE_* code of t, which must be one of `allowed` and, if given, of like's dtype."""
    if t.dtype not in allowed:
        names = ", ".join(str(d) for d in allowed)
        raise TypeError(f"{name} must be one of {names}, got {t.dtype}")
    if like is not None and t.dtype != like.dtype:
        raise TypeError(f"{name} must have the dtype of the activations ({like.dtype}), got {t.dtype}")
    return DTYPE_CODES[t.dtype]


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


# ------------------------------------------------------------------- RMSNorm
def rmsnorm_fwd(x2d: torch.Tensor, w: torch.Tensor, eps: float) -> tuple[torch.Tensor, torch.Tensor]:
    """y, rstd for a contiguous [rows, N] x2d and [N] weight of one dtype (bf16, fp16 or fp32)."""
    _on_gpu(x2d, w)
    dt = _dtype("x2d", x2d)
    _dtype("weight", w, like=x2d)
    if x2d.dim() != 2 or not x2d.is_contiguous():
        raise ValueError("x2d must be a contiguous 2D tensor [rows, N]")
    rows, n = x2d.shape
    if w.shape != (n,):
        raise ValueError(f"weight shape {tuple(w.shape)} != ({n},)")
    w = w.contiguous()
    y = torch.empty_like(x2d)
    rstd = torch.empty(rows, device=x2d.device, dtype=torch.float32)
    if rows:
        _check(lib().krsi_rmsnorm_fwd(_ptr(x2d), _ptr(w), _ptr(y), _ptr(rstd), rows, n,
                                      float(eps), dt, _stream(x2d)))
    return y, rstd


def rmsnorm_bwd(g: torch.Tensor, x2d: torch.Tensor, w: torch.Tensor,
                rstd: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """dx and dw (fp32-accumulated) of rmsnorm, in the dtype of x2d."""
    _on_gpu(g, x2d, w, rstd)
    g = g.contiguous()
    w = w.contiguous()
    rows, n = x2d.shape
    if g.shape != x2d.shape:
        raise ValueError(f"grad shape {tuple(g.shape)} != {tuple(x2d.shape)}")
    dt = _dtype("x2d", x2d)
    _dtype("weight", w, like=x2d)
    _dtype("grad", g, like=x2d)
    dx = torch.empty_like(x2d)
    dw = torch.empty(n, device=x2d.device, dtype=w.dtype)
    nbytes = _rmsnorm_ws_bytes(rows, n)
    ws = torch.empty(max(nbytes, 1), device=x2d.device, dtype=torch.uint8)
    _check(lib().krsi_rmsnorm_bwd(_ptr(g), _ptr(x2d), _ptr(w), _ptr(rstd), _ptr(dx), _ptr(dw),
                                  _ptr(ws), nbytes, rows, n, dt, _stream(x2d)))
    return dx, dw


# --------------------------------------------------------------------- GEGLU
_APPROX = {"tanh": 1, "none": 0}


def _approx(approximate: str) -> int:
    if approximate not in _APPROX:
        raise ValueError(f"approximate must be 'tanh' or 'none', got {approximate!r}")
    return _APPROX[approximate]


def geglu_fwd(u: torch.Tensor, approximate: str = "tanh") -> torch.Tensor:
    _on_gpu(u)
    dt = _dtype("u", u)
    if u.dim() != 2 or not u.is_contiguous() or u.shape[1] % 2:
        raise ValueError("u must be a contiguous [rows, 2F] tensor")
    rows, f2 = u.shape
    out = torch.empty(rows, f2 // 2, device=u.device, dtype=u.dtype)
    if rows and f2:
        _check(lib().krsi_geglu_fwd(_ptr(u), _ptr(out), rows, f2 // 2, _approx(approximate), dt,
                                    _stream(u)))
    return out


def geglu_bwd(g: torch.Tensor, u: torch.Tensor, approximate: str = "tanh") -> torch.Tensor:
    _on_gpu(g, u)
    g = g.contiguous()
    dt = _dtype("u", u)
    _dtype("grad", g, like=u)
    rows, f2 = u.shape
    if g.shape != (rows, f2 // 2):
        raise ValueError(f"grad shape {tuple(g.shape)} != {(rows, f2 // 2)}")
    du = torch.empty_like(u)
    if rows and f2:
        _check(lib().krsi_geglu_bwd(_ptr(g), _ptr(u), _ptr(du), rows, f2 // 2,
                                    _approx(approximate), dt, _stream(u)))
    return du


def geglu_linear_fwd(x: torch.Tensor, w: torch.Tensor, approximate: str = "tanh") -> torch.Tensor:
    """gelu(x @ w[:F].T) * (x @ w[F:].T) for x [rows, K] and the merged weight w [2F, K] in one
    kernel (bf16 or fp16; K and F multiples of 64)."""
    _on_gpu(x, w)
    dt = _dtype("x", x, allowed=(torch.bfloat16, torch.float16))
    _dtype("weight", w, like=x)
    if x.dim() != 2 or w.dim() != 2 or w.shape[1] != x.shape[1] or w.shape[0] % 2:
        raise ValueError(f"need x [rows, K] and w [2F, K], got {tuple(x.shape)} and {tuple(w.shape)}")
    rows, k = x.shape
    f = w.shape[0] // 2
    if k % 64 or f % 64:
        raise ValueError(f"geglu_linear needs K and F multiples of 64, got K={k}, F={f}")
    x, w = x.contiguous(), w.contiguous()
    out = torch.empty(rows, f, device=x.device, dtype=x.dtype)
    if rows:
        _check(lib().krsi_geglu_linear_fwd(_ptr(x), _ptr(w), _ptr(out), rows, k, f, _approx(approximate), dt,
                                           _stream(x)))
    return out


# ------------------------------------------------ relative-position attention
def _check_relpos(qkv: torch.Tensor, pd: torch.Tensor, B: int, S: int, H: int, D: int) -> int:
    _on_gpu(qkv, pd)
    dt = _dtype("qkv", qkv, allowed=_ATTN_DTYPES)
    if pd.dtype != torch.float32:
        raise TypeError(f"pd must be torch.float32, got {pd.dtype}")
    if qkv.dim() != 2 or qkv.stride(1) != 1:
        raise ValueError("qkv must be a 2D [B*S, >=3*H*D] tensor with unit column stride")
    if qkv.shape[0] != B * S or qkv.shape[1] < 3 * H * D:
        raise ValueError(f"qkv shape {tuple(qkv.shape)} does not hold B*S={B * S} rows of 3*H*D={3 * H * D}")
    if tuple(pd.shape) != (H, 2 * S - 1):
        raise ValueError(f"pd shape {tuple(pd.shape)} != {(H, 2 * S - 1)}")
    if D % 8 or not 8 <= D <= 128:
        raise ValueError(f"head dim D={D} unsupported: needs D % 8 == 0 and 8 <= D <= 128")
    return dt


def relpos_fwd(qkv: torch.Tensor, pd: torch.Tensor, B: int, S: int, H: int, D: int,
               scale: float, stats: bool = True):
    """out (qkv's dtype), out32 (fp32) [B*S, H*D] and lse [B*H, S] (log2 domain). With
    stats=False (a forward no backward follows) the kernels store out only: out32 and lse
    come back as None."""
    dt = _check_relpos(qkv, pd, B, S, H, D)
    pd = pd.contiguous()
    out = torch.empty(B * S, H * D, device=qkv.device, dtype=qkv.dtype)
    out32 = torch.empty(B * S, H * D, device=qkv.device, dtype=torch.float32) if stats else None
    lse = torch.empty(B * H, S, device=qkv.device, dtype=torch.float32) if stats else None
    _check(lib().krsi_relpos_fwd(_ptr(qkv), qkv.stride(0), _ptr(pd), _ptr(out), _ptr(out32),
                                 _ptr(lse), B, S, H, D, float(scale), dt, _stream(qkv)))
    return out, out32, lse


def relpos_bwd(dout: torch.Tensor, qkv: torch.Tensor, pd: torch.Tensor, out32: torch.Tensor,
               lse: torch.Tensor, B: int, S: int, H: int, D: int, scale: float,
               workspace_max: int | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """dqkv (same shape and strides as a contiguous qkv) and dpd [H, 2S-1] fp32.

    workspace_max (default RELPOS_BWD_WORKSPACE_MAX) caps the workspace in bytes; it is
    raised to the library's minimum (one key block's dpd partial rows) when below it."""
    dt = _check_relpos(qkv, pd, B, S, H, D)
    _on_gpu(dout, out32, lse)
    dout = dout.contiguous()
    _dtype("grad", dout, like=qkv)
    pd = pd.contiguous()
    # Every column of dqkv is written (q, k and v slots of each head); columns
    # past 3*H*D of a wider qkv are zero, as the gradient of a slice.
    dqkv = torch.empty(qkv.shape, device=qkv.device, dtype=qkv.dtype)
    if qkv.shape[1] > 3 * H * D:
        dqkv[:, 3 * H * D:].zero_()
    dpd = torch.empty(H, 2 * S - 1, device=qkv.device, dtype=torch.float32)
    nbytes = _relpos_ws_bytes(B, S, H, D)
    cap = RELPOS_BWD_WORKSPACE_MAX if workspace_max is None else workspace_max
    if cap is not None and cap < nbytes:
        nbytes = max(int(cap), _relpos_ws_min_bytes(B, S, H, D))
    ws = torch.empty(nbytes, device=qkv.device, dtype=torch.uint8)
    _check(lib().krsi_relpos_bwd(_ptr(dout), _ptr(qkv), qkv.stride(0), _ptr(pd), _ptr(out32),
                                 _ptr(lse), _ptr(dqkv), dqkv.stride(0), _ptr(dpd), _ptr(ws), nbytes,
                                 B, S, H, D, float(scale), dt, _stream(qkv)))
    return dqkv, dpd


# ------------------------------------------ bucketed relative-position table
def _check_bucket(bucket: torch.Tensor, S: int) -> None:
    if bucket.dtype != torch.int32 or bucket.dim() != 1 or bucket.numel() != 2 * S - 1:
        raise ValueError(f"bucket must be a [2S-1] = [{2 * S - 1}] int32 tensor, got "
                         f"{bucket.dtype} {tuple(bucket.shape)}")


def relpos_bucket_gather(table: torch.Tensor, bucket: torch.Tensor, S: int) -> torch.Tensor:
    """pd [H, 2S-1] fp32 with pd[h, r] = table[bucket[r], h]; table [num_buckets, H] fp32."""
    _on_gpu(table, bucket)
    if table.dtype != torch.float32 or table.dim() != 2:
        raise TypeError(f"table must be a [num_buckets, H] float32 tensor, got {table.dtype} "
                        f"{tuple(table.shape)}")
    _check_bucket(bucket, S)
    table, bucket = table.contiguous(), bucket.contiguous()
    nb, H = table.shape
    pd = torch.empty(H, 2 * S - 1, device=table.device, dtype=torch.float32)
    _check(lib().krsi_relpos_bucket_gather(_ptr(table), _ptr(bucket), _ptr(pd), S, H, nb,
                                           _stream(table)))
    return pd


def relpos_bucket_sum(dpd: torch.Tensor, bucket: torch.Tensor, S: int, num_buckets: int) -> torch.Tensor:
    """dtable [num_buckets, H] fp32: the sums of dpd [H, 2S-1] over each bucket's distances."""
    _on_gpu(dpd, bucket)
    if dpd.dtype != torch.float32 or dpd.dim() != 2 or dpd.shape[1] != 2 * S - 1:
        raise ValueError(f"dpd must be an [H, {2 * S - 1}] float32 tensor, got {dpd.dtype} {tuple(dpd.shape)}")
    _check_bucket(bucket, S)
    dpd, bucket = dpd.contiguous(), bucket.contiguous()
    H = dpd.shape[0]
    dtable = torch.empty(num_buckets, H, device=dpd.device, dtype=torch.float32)
    _check(lib().krsi_relpos_bucket_sum(_ptr(dpd), _ptr(bucket), _ptr(dtable), S, H, num_buckets,
                                        _stream(dpd)))
    return dtable
