"""The C-ABI boundary without a GPU: the library loads, exports every entry point of
include/krsi.h with the declared signature, binds to torch's HIP runtime, reports errors
for invalid arguments before launching anything, and the Python layer has no CPU path."""
import re
from pathlib import Path

import pytest
import torch

import _hip

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "krsi.h"
NULL = None
FAKE = 0x10000  # a 16-byte aligned non-null address; never dereferenced on these paths


def declared():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:int|size_t|const char\*)\s+(krsi_\w+)\s*\(", text, re.M)))


def test_header_declares_the_python_binding_set():
    assert declared() == sorted(_hip.SIGNATURES)


def test_library_loads_and_exports_every_symbol():
    lib = _hip.lib()
    for name in declared():
        assert hasattr(lib, name), name
    assert lib.krsi_abi_version() == _hip.ABI_VERSION


def test_single_hip_runtime_in_process():
    _hip.lib()
    maps = Path("/proc/self/maps").read_text()
    paths = {m for m in re.findall(r"\S*libamdhip64\.so\S*", maps)}
    assert len(paths) <= 1, paths


def test_error_strings():
    lib = _hip.lib()
    for code in range(0, 9):
        s = lib.krsi_error_string(code).decode()
        assert s and ("krsi" in s or code == 0)
    assert "unknown" in lib.krsi_error_string(99).decode()


def test_workspace_sizes():
    lib = _hip.lib()
    a = lib.krsi_rmsnorm_bwd_workspace_bytes(32768, 4096)
    assert a > 0 and a % 256 == 0
    assert lib.krsi_rmsnorm_bwd_workspace_bytes(0, 4096) == 0
    assert lib.krsi_rmsnorm_bwd_workspace_bytes(10, 0) == 0
    b = lib.krsi_relpos_bwd_workspace_bytes(4, 4096, 16, 64)
    # delta [B,H,S] + one fp32 partial row of S+128 diagonals per 128-query block
    assert b >= 4 * 16 * 4096 * 4 + 4 * 16 * 32 * (4096 + 128) * 4
    assert lib.krsi_relpos_bwd_workspace_bytes(0, 4096, 16, 64) == 0
    # The smallest workspace: delta and the partial rows of one 128-key block.
    m = lib.krsi_relpos_bwd_workspace_min_bytes(4, 4096, 16, 64)
    assert m == 4 * 16 * 4096 * 4 + 4 * 16 * (4096 + 128) * 4
    assert lib.krsi_relpos_bwd_workspace_min_bytes(4, 4096, 0, 64) == 0
    # One key block in all (S <= 128): the minimum is the full size up to its 256-byte padding.
    full, low = lib.krsi_relpos_bwd_workspace_bytes(3, 100, 5, 64), lib.krsi_relpos_bwd_workspace_min_bytes(3, 100, 5, 64)
    assert low <= full < low + 256


def test_validation_before_launch():
    lib = _hip.lib()
    E = {"NULL": 1, "SHAPE": 2, "ALIGN": 3, "WS": 4, "UNSUP": 5, "SCALE": 7}
    # RMSNorm
    assert lib.krsi_rmsnorm_fwd_bf16(FAKE, FAKE, FAKE, FAKE, 4, 0, 1e-6, NULL) == E["SHAPE"]
    assert lib.krsi_rmsnorm_fwd_bf16(FAKE, FAKE, FAKE, FAKE, 4, 16385, 1e-6, NULL) == E["SHAPE"]
    assert lib.krsi_rmsnorm_fwd_bf16(NULL, FAKE, FAKE, FAKE, 4, 64, 1e-6, NULL) == E["NULL"]
    assert lib.krsi_rmsnorm_fwd_bf16(FAKE, FAKE, FAKE, FAKE, 4, 64, float("nan"), NULL) == E["SCALE"]
    assert lib.krsi_rmsnorm_fwd_bf16(NULL, NULL, NULL, NULL, 0, 64, 1e-6, NULL) == 0   # empty: no-op
    assert lib.krsi_rmsnorm_bwd_bf16(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 16, 64, 64, NULL) == E["WS"]
    assert lib.krsi_rmsnorm_bwd_bf16(FAKE, FAKE, FAKE, FAKE, FAKE, NULL, FAKE, 1 << 30, 64, 64, NULL) == E["NULL"]
    # GEGLU
    assert lib.krsi_geglu_fwd_bf16(FAKE, FAKE, 4, 0, 1, NULL) == E["SHAPE"]
    assert lib.krsi_geglu_fwd_bf16(FAKE, FAKE, 4, 8, 2, NULL) == E["UNSUP"]
    assert lib.krsi_geglu_bwd_bf16(FAKE, NULL, FAKE, 4, 8, 0, NULL) == E["NULL"]
    # Attention
    args = dict(B=2, S=16, H=2, D=64)

    def fwd(qkv=FAKE, ld=384, pd=FAKE, out=FAKE, B=2, S=16, H=2, D=64, scale=0.125):
        return lib.krsi_relpos_fwd_bf16(qkv, ld, pd, out, FAKE, FAKE, B, S, H, D, scale, NULL)

    assert fwd(D=12, ld=72) == E["UNSUP"]
    assert fwd(D=136, ld=816) == E["UNSUP"]
    assert fwd(S=0) == E["SHAPE"]
    assert fwd(ld=380) == E["SHAPE"]
    assert fwd(ld=388) == E["ALIGN"]
    assert fwd(qkv=FAKE + 2) == E["ALIGN"]
    assert fwd(scale=float("inf")) == E["SCALE"]
    assert fwd(scale=1e-25) == E["SCALE"]    # |scale| log2(e) below 2^-60 (folded bias overflow)
    # fp32 adds the bias directly, so a tiny scale passes the scale check and the call stops
    # at the next one (a misaligned out), before any launch.
    assert lib.krsi_relpos_fwd(FAKE, 384, FAKE, FAKE + 2, FAKE, FAKE, 2, 16, 2, 64, 1e-20, 2, NULL) == E["ALIGN"]
    assert lib.krsi_relpos_fwd(FAKE, 384, FAKE, FAKE + 2, FAKE, FAKE, 2, 16, 2, 64, 1e-20, 0, NULL) == E["SCALE"]
    assert fwd(S=1 << 20, ld=1024) == E["UNSUP"]  # one (batch, head) slice >= 2^31 bytes
    assert fwd(pd=NULL) == E["NULL"]
    # out32 and lse are optional together (a forward with no backward), not one without the other.
    assert lib.krsi_relpos_fwd_bf16(FAKE, 384, FAKE, FAKE, NULL, FAKE, 2, 16, 2, 64, 0.125, NULL) == E["NULL"]
    assert lib.krsi_relpos_fwd_bf16(FAKE, 384, FAKE, FAKE, FAKE, NULL, 2, 16, 2, 64, 0.125, NULL) == E["NULL"]
    assert lib.krsi_relpos_fwd_bf16(FAKE, 384, FAKE, FAKE, NULL, NULL, 2, 16, 0, 64, 0.125, NULL) == E["SHAPE"]
    assert fwd(B=40000, H=2) == E["SHAPE"]   # B*H above the grid limit
    ws = lib.krsi_relpos_bwd_workspace_min_bytes(args["B"], args["S"], args["H"], args["D"])
    assert lib.krsi_relpos_bwd_bf16(FAKE, FAKE, 384, FAKE, FAKE, FAKE, FAKE, 384, FAKE, FAKE, ws - 1,
                                    2, 16, 2, 64, 0.125, NULL) == E["WS"]
    assert lib.krsi_relpos_bwd_bf16(FAKE, FAKE, 384, FAKE, FAKE, FAKE, FAKE, 200, FAKE, FAKE, ws,
                                    2, 16, 2, 64, 0.125, NULL) == E["SHAPE"]


def test_noalloc_backward_validates_before_touching_the_device():
    """krsi_rmsnorm_bwd_noalloc checks its arguments, and that the problem fits its static
    16 MiB scratch, before any HIP call (FAKE pointers: nothing is dereferenced)."""
    lib = _hip.lib()
    f = lib.krsi_rmsnorm_bwd_noalloc
    TOO_LARGE = 8
    assert f(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 4, 0, 0, NULL) == 2          # n = 0
    assert f(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 4, 16385, 0, NULL) == 2      # n above 16384
    assert f(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 4, 64, 7, NULL) == 5         # unknown dtype
    assert f(FAKE, FAKE, FAKE, FAKE, FAKE, NULL, 4, 64, 0, NULL) == 1         # dw NULL
    assert f(NULL, FAKE, FAKE, FAKE, FAKE, FAKE, 4, 64, 0, NULL) == 1         # g NULL
    limit = 16 << 20
    for rows, n in ((32768, 16384), (1 << 20, 12288), (257, 16384)):
        assert lib.krsi_rmsnorm_bwd_workspace_bytes(rows, n) > limit
        for dt in (0, 1, 2):
            assert f(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, rows, n, dt, NULL) == TOO_LARGE
    # The stated limit: every row count fits for n <= 8192, and n = 16384 fits up to 256 rows.
    for rows, n in ((1 << 24, 8192), (256, 16384), (32768, 4096)):
        assert lib.krsi_rmsnorm_bwd_workspace_bytes(rows, n) <= limit
    assert "16 MiB" in lib.krsi_error_string(TOO_LARGE).decode()


def test_geglu_linear_validates_before_launch():
    lib = _hip.lib()
    f = lib.krsi_geglu_linear_fwd
    assert f(FAKE, FAKE, FAKE, 4, 64, 64, 1, 2, NULL) == 5        # fp32: not built
    assert f(FAKE, FAKE, FAKE, 4, 64, 64, 2, 0, NULL) == 5        # unknown GELU form
    assert f(FAKE, FAKE, FAKE, 4, 96, 64, 1, 0, NULL) == 5        # K % 64 != 0
    assert f(FAKE, FAKE, FAKE, 4, 64, 96, 1, 0, NULL) == 5        # F % 64 != 0
    assert f(FAKE, FAKE, FAKE, 4, 1 << 23, 64, 1, 0, NULL) == 5   # a stage's offsets past 2^31
    assert f(FAKE, FAKE, FAKE, -1, 64, 64, 1, 0, NULL) == 2
    assert f(NULL, FAKE, FAKE, 4, 64, 64, 1, 0, NULL) == 1
    assert f(FAKE + 2, FAKE, FAKE, 4, 64, 64, 1, 0, NULL) == 3
    assert f(NULL, NULL, NULL, 0, 64, 64, 1, 0, NULL) == 0         # no rows: no-op


def test_dtype_argument_validated_before_launch():
    """The generic entry points take KRSI_DTYPE_* (0 bf16, 1 fp16, 2 fp32); an unknown code,
    or fp32 for attention, is UNSUPPORTED before anything is launched (FAKE pointers)."""
    lib = _hip.lib()
    UNSUP, NULLP = 5, 1
    for dt in (-1, 3, 99):
        assert lib.krsi_rmsnorm_fwd(FAKE, FAKE, FAKE, FAKE, 4, 64, 1e-6, dt, NULL) == UNSUP
        assert lib.krsi_rmsnorm_bwd(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 1 << 30, 4, 64, dt, NULL) == UNSUP
        assert lib.krsi_geglu_fwd(FAKE, FAKE, 4, 8, 1, dt, NULL) == UNSUP
        assert lib.krsi_geglu_bwd(FAKE, FAKE, FAKE, 4, 8, 1, dt, NULL) == UNSUP
    for dt in (3, -1):
        assert lib.krsi_relpos_fwd(FAKE, 384, FAKE, FAKE, FAKE, FAKE, 2, 16, 2, 64, 0.125, dt, NULL) == UNSUP
        assert lib.krsi_relpos_bwd(FAKE, FAKE, 384, FAKE, FAKE, FAKE, FAKE, 384, FAKE, FAKE, 1 << 30,
                                   2, 16, 2, 64, 0.125, dt, NULL) == UNSUP
    # Known dtypes reach the usual checks (here: a NULL pointer), still before any launch.
    for dt in (0, 1, 2):
        assert lib.krsi_rmsnorm_fwd(NULL, FAKE, FAKE, FAKE, 4, 64, 1e-6, dt, NULL) == NULLP
        assert lib.krsi_geglu_fwd(NULL, FAKE, 4, 8, 1, dt, NULL) == NULLP
    for dt in (0, 1, 2):
        assert lib.krsi_relpos_fwd(FAKE, 384, NULL, FAKE, FAKE, FAKE, 2, 16, 2, 64, 0.125, dt, NULL) == NULLP
    # fp32 qkv rows need a 16-byte multiple (ld % 4); 16-bit rows ld % 8. The 2^31-byte slice
    # limit of the 16-bit kernels' buffer resources does not apply to fp32.
    ALIGN = 3
    assert lib.krsi_relpos_fwd(FAKE, 386, FAKE, FAKE, FAKE, FAKE, 2, 16, 2, 64, 0.125, 2, NULL) == ALIGN
    assert lib.krsi_relpos_fwd(FAKE, 388, FAKE, FAKE, FAKE, FAKE, 2, 16, 2, 64, 0.125, 0, NULL) == ALIGN
    assert lib.krsi_relpos_fwd(FAKE, 1024, FAKE, FAKE, FAKE, FAKE, 1, 1 << 20, 2, 64, 0.125, 0, NULL) == UNSUP
    # The workspace size does not depend on the dtype: one size serves all three.
    assert lib.krsi_rmsnorm_bwd_workspace_bytes(1000, 16384) >= 512 * 16384 * 4
    assert _hip.DTYPE_CODES == {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}


def test_bucket_entry_points_validate_before_launch():
    lib = _hip.lib()
    SHAPE, NULLP = 2, 1
    assert lib.krsi_relpos_bucket_gather(FAKE, FAKE, FAKE, 0, 4, 32, NULL) == SHAPE
    assert lib.krsi_relpos_bucket_gather(FAKE, FAKE, FAKE, 16, 0, 32, NULL) == SHAPE
    assert lib.krsi_relpos_bucket_gather(FAKE, FAKE, FAKE, 16, 4, 0, NULL) == SHAPE
    assert lib.krsi_relpos_bucket_gather(NULL, FAKE, FAKE, 16, 4, 32, NULL) == NULLP
    assert lib.krsi_relpos_bucket_sum(FAKE, NULL, FAKE, 16, 4, 32, NULL) == NULLP
    assert lib.krsi_relpos_bucket_sum(FAKE, FAKE, FAKE, 16, 70000, 32, NULL) == SHAPE


def test_python_layer_has_no_cpu_path():
    import geglu
    import relpos_attention
    import rmsnorm

    x = torch.randn(4, 64, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="GPU"):
        rmsnorm.rmsnorm(x, torch.ones(64, dtype=torch.bfloat16), 1e-6)
    with pytest.raises(ValueError, match="GPU"):
        geglu.geglu(x)
    qkv = torch.randn(8, 3 * 64, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="GPU"):
        relpos_attention.relpos_attention(qkv, torch.zeros(1, 15), 1, 8, 1, 64, 0.125)


def test_missing_library_fails_loudly(tmp_path, monkeypatch):
    monkeypatch.setattr(_hip, "LIB_PATH", tmp_path / "libkrsi_hip.so")
    monkeypatch.setattr(_hip, "_lib", None)
    with pytest.raises(ImportError, match="not built"):
        _hip.lib()


def test_product_never_imports_the_oracle():
    for p in (ROOT / "kernel-rsi_amd").rglob("*.py"):
        if p.name == "build.py":
            continue
        assert "oracle" not in p.read_text(), p


def test_modules_keep_the_reference_interface():
    import inspect

    import geglu
    import relpos_attention
    import rmsnorm

    assert list(inspect.signature(rmsnorm.rmsnorm).parameters) == ["x2d", "w", "eps"]
    assert list(inspect.signature(rmsnorm.reference).parameters) == ["x2d", "w", "eps"]
    assert list(inspect.signature(geglu.geglu).parameters)[0] == "u"
    assert list(inspect.signature(relpos_attention.relpos_attention).parameters) == \
        ["qkv", "pd", "B", "S", "H", "D", "scale"]
    for m in (rmsnorm, geglu, relpos_attention):
        assert callable(m.selftest) and callable(m.reference)


def test_workspace_cap_from_environment(monkeypatch):
    """KRSI_RELPOS_BWD_WORKSPACE_MAX: unset, empty or <= 0 means no cap; a non-integer is
    refused with the variable's name in the message."""
    for raw, want in (("", None), ("0", None), ("-5", None), (" 4096 ", 4096)):
        monkeypatch.setenv("KRSI_RELPOS_BWD_WORKSPACE_MAX", raw)
        assert _hip._env_bytes("KRSI_RELPOS_BWD_WORKSPACE_MAX") == want
    monkeypatch.setenv("KRSI_RELPOS_BWD_WORKSPACE_MAX", "64MB")
    with pytest.raises(ValueError, match="KRSI_RELPOS_BWD_WORKSPACE_MAX"):
        _hip._env_bytes("KRSI_RELPOS_BWD_WORKSPACE_MAX")
