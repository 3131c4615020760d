"""CPU checks of the C-ABI library: it loads, exports every declared symbol, and rejects
bad arguments with an error message before touching the GPU."""

import ctypes
import re
from pathlib import Path

import pytest

from bongard_amd import _lib

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "bongard_fp8.h"


def _declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"\b(bf8_[a-z0-9_]+)\s*\(", text)
    return sorted(set(names))


def test_library_loads_and_exports_header_symbols():
    L = _lib.lib()
    declared = _declared_functions()
    assert len(declared) >= 14
    for name in declared:
        assert hasattr(L, name), f"{name} declared in the header but not exported"
    assert set(declared) == set(_lib.SIGNATURES), "ctypes table and header disagree"
    assert L.bf8_abi_version() == _lib.ABI_VERSION


def test_bad_arguments_report_errors_without_gpu():
    L = _lib.lib()
    null = ctypes.c_void_p(0)
    rc = L.bf8_gemm(null, 0, 16, null, 0, 16, 32, 32, 24, null, null, 4, None, 1, null, null,
                    0, 32, null, 0, null)
    assert rc == 1
    assert b"multiples of 16" in L.bf8_last_error()
    rc = L.bf8_cast_bf16(null, 4, 16, null, 0, null, null, null)
    assert rc == 1 and b"scale is NULL" in L.bf8_last_error()
    rc = L.bf8_scale_from_partials(null, 1, 7, null, null)
    assert rc == 1 and b"bad fmt" in L.bf8_last_error()
    rc = L.bf8_gemm_geglu(null, 16, null, 16, 4, 100, 16, null, null, 0, null, 100, null, null,
                          null)
    assert rc == 1 and b"multiple of 128" in L.bf8_last_error()
    with pytest.raises(_lib.Fp8LibError, match="bf8_gemm"):
        _lib.check(L.bf8_gemm(null, 0, 16, null, 0, 16, 32, 32, 24, null, null, 4, None, 1,
                              null, null, 0, 32, null, 0, null), "bf8_gemm")


def test_partials_counts():
    L = _lib.lib()
    assert L.bf8_amax_partials(0) == 1
    assert L.bf8_amax_partials(512 * 2560) >= 1
    # capped at the number of partials a consumer block reduces inline (8 per CU)
    assert L.bf8_amax_partials(1 << 30) == 1024
    assert L.bf8_cast_amax_partials(1 << 15, 1 << 15, 0) == 512
    assert L.bf8_geglu_partials(4096, 10240) == 16 * 80
    assert L.bf8_gemm_workspace(4096, 2560, 10240) >= 0


def test_plan_override_env(monkeypatch):
    """BONGARD_FP8_GEMM_TILE forces the tile (and K split) of the next calls; the gated-GELU
    partial count follows the forced tile, and a K split sizes the fp32 workspace."""
    L = _lib.lib()
    monkeypatch.setenv("BONGARD_FP8_GEMM_TILE", "128x128")
    assert L.bf8_geglu_partials(300, 384) == 3 * 6
    assert L.bf8_gemm_workspace(512, 2560, 10240) == 0
    monkeypatch.setenv("BONGARD_FP8_GEMM_TILE", "256x256:4")
    assert L.bf8_geglu_partials(300, 384) == 2 * 3
    assert L.bf8_gemm_workspace(512, 2560, 10240) == 4 * 512 * 2560 * 4
    # 80 gate + 80 up columns per tile: a gated-GELU variant for I % 80 == 0 only
    monkeypatch.setenv("BONGARD_FP8_GEMM_TILE", "256x160")
    assert L.bf8_geglu_partials(512, 10240) == 2 * 128
    assert L.bf8_geglu_partials(300, 640) == 2 * 8
    assert L.bf8_geglu_partials(300, 384) != 2 * 5  # 384 % 80 != 0: the automatic plan


def test_tail_split_plans(monkeypatch):
    """Tail-split plans (whole 256x256 tiles, the partial last round's tiles split along K)
    size their workspace as [tail tiles x pieces][256][256] fp32: c5's dX and dW_gu GEMMs
    take one automatically; c2's down projection (160 tiles, one round) does not;
    BONGARD_FP8_GEMM_TILE=256x256:t forces one where the shape has a tail."""
    L = _lib.lib()
    tile = 256 * 256 * 4
    monkeypatch.delenv("BONGARD_FP8_GEMM_TILE", raising=False)
    assert L.bf8_gemm_workspace(8192, 2560, 20480) == 64 * 4 * tile   # 320 tiles: 256 + 64
    assert L.bf8_gemm_workspace(20480, 2560, 8192) == 32 * 8 * tile   # 800 tiles: 768 + 32
    assert L.bf8_gemm_workspace(4096, 2560, 10240) == 0
    monkeypatch.setenv("BONGARD_FP8_GEMM_TILE", "256x256:t")
    assert L.bf8_gemm_workspace(4160, 3848, 4112) == 16 * 7 * tile   # 33 K steps in 7 pieces
    assert L.bf8_gemm_workspace(4096, 4096, 4096) == 0                # 256 tiles: no tail


def test_quantize_many_rejects_bad_arguments():
    """The multi-tensor quantization checks its lists on the host (no launch)."""
    L = _lib.lib()
    null = ctypes.c_void_p(0)
    n = (ctypes.c_int64 * 9)(*([64] * 9))
    assert L.bf8_quantize_many_partials(2, n) == 2
    assert L.bf8_quantize_many_partials(9, n) == 0
    buf = ctypes.create_string_buffer(1 << 12)
    ptr = ctypes.c_void_p((ctypes.addressof(buf) + 255) // 256 * 256)
    ptrs = (ctypes.c_void_p * 2)(ptr, ptr)
    rc = L.bf8_quantize_many_bf16(0, ptrs, n, (ctypes.c_int * 2)(0, 0), ptrs, ptrs, ptr, null)
    assert rc == 1 and b"count 0" in L.bf8_last_error()
    rc = L.bf8_quantize_many_bf16(2, ptrs, n, (ctypes.c_int * 2)(0, 7), ptrs, ptrs, ptr, null)
    assert rc == 1 and b"bad fmt 7" in L.bf8_last_error()
    odd = (ctypes.c_void_p * 2)(ptr, ctypes.c_void_p(ptr.value + 8))
    rc = L.bf8_quantize_many_bf16(2, odd, n, (ctypes.c_int * 2)(0, 0), ptrs, ptrs, ptr, null)
    assert rc == 1 and b"16-byte aligned" in L.bf8_last_error()
    nometa = (ctypes.c_void_p * 2)(ptr, null)
    rc = L.bf8_quantize_many_bf16(2, ptrs, n, (ctypes.c_int * 2)(0, 0), ptrs, nometa, ptr, null)
    assert rc == 1 and b"meta is NULL" in L.bf8_last_error()


def test_quantize_mx_many_rejects_bad_arguments():
    L = _lib.lib()
    null = ctypes.c_void_p(0)
    buf = ctypes.create_string_buffer(1 << 12)
    ptr = ctypes.c_void_p((ctypes.addressof(buf) + 255) // 256 * 256)
    ptrs = (ctypes.c_void_p * 2)(ptr, ptr)
    rows = (ctypes.c_int64 * 2)(32, 32)
    fm = (ctypes.c_int * 2)(0, 0)
    rc = L.bf8_quantize_mx_many_bf16(9, ptrs, rows, rows, fm, ptrs, ptrs, null)
    assert rc == 1 and b"count 9" in L.bf8_last_error()
    rc = L.bf8_quantize_mx_many_bf16(2, ptrs, rows, (ctypes.c_int64 * 2)(32, 48), fm, ptrs,
                                     ptrs, null)
    assert rc == 1 and b"cols % 32" in L.bf8_last_error()
    rc = L.bf8_quantize_mx_many_bf16(2, ptrs, rows, rows, fm, ptrs, (ctypes.c_void_p * 2)(ptr, null),
                                     null)
    assert rc == 1 and b"is NULL" in L.bf8_last_error()


def test_quantizing_geglu_and_scale_fold_reject_bad_arguments():
    """The epilogue-quantizing gate/up entries and the delayed scale fold check their
    arguments on the host (no launch): missing H8, a transposed copy with M % 32 != 0,
    bad history slots."""
    L = _lib.lib()
    null = ctypes.c_void_p(0)
    buf = ctypes.create_string_buffer(1 << 12)
    ptr = ctypes.c_void_p((ctypes.addressof(buf) + 255) // 256 * 256)
    # bf8_gemm_geglu_quant: H8 is required
    rc = L.bf8_gemm_geglu_quant(ptr, 32, ptr, 32, 32, 128, 32, ptr, ptr, 0, ptr, null, 128,
                                null, null, null, ptr, null)
    assert rc == 1 and b"H8 is NULL" in L.bf8_last_error()
    # ... and H8t needs M % 32 == 0
    rc = L.bf8_gemm_geglu_quant(ptr, 32, ptr, 32, 40, 128, 32, ptr, ptr, 0, ptr, null, 128,
                                ptr, ptr, null, ptr, null)
    assert rc == 1 and b"M % 32" in L.bf8_last_error()
    # MX variant: I must be a multiple of 128, H8 required
    rc = L.bf8_gemm_geglu_mx_quant(ptr, 32, ptr, 4, ptr, 32, ptr, 4, 32, 100, 32, null, 128,
                                   ptr, ptr, 4, null, null, 0, null, null)
    assert rc == 1 and b"multiple of 128" in L.bf8_last_error()
    rc = L.bf8_gemm_geglu_mx_quant(ptr, 32, ptr, 4, ptr, 32, ptr, 4, 32, 128, 32, null, 128,
                                   null, null, 4, null, null, 0, null, null)
    assert rc == 1 and b"H8 is NULL" in L.bf8_last_error()
    # delayed scale fold: slot outside the history
    rc = L.bf8_delayed_scale_fold(ptr, 16, 16, null, 0, 0, null, null)
    assert rc == 1 and b"outside" in L.bf8_last_error()
    rc = L.bf8_delayed_scale_fold(ptr, 16, 0, null, 5, 0, null, null)
    assert rc == 1 and b"previous partials" in L.bf8_last_error()


def test_kmajor_workspace_covers_transposed_b(monkeypatch):
    """A K-major GEMM whose 256x256 plan would leave most CUs idle (a small output) may run
    on B transposed into its workspace: the workspace query then covers N x K bytes plus
    the row-major plan's own; large shapes keep the K-major plan (c5's GEMMs: same
    workspace as bf8_gemm, which plans them alike), and a forced tile keeps it too."""
    L = _lib.lib()
    monkeypatch.delenv("BONGARD_FP8_GEMM_TILE", raising=False)
    for M, N, K in [(512, 2560, 2048), (1024, 2560, 2560), (304, 320, 1040)]:
        assert L.bf8_gemm_kmajor_workspace(M, N, K) >= N * K
    for M, N, K in [(8192, 2560, 20480), (20480, 2560, 8192), (8192, 10240, 2560),
                    (2560, 10240, 8192)]:
        assert L.bf8_gemm_kmajor_workspace(M, N, K) == L.bf8_gemm_workspace(M, N, K)
    monkeypatch.setenv("BONGARD_FP8_GEMM_TILE", "256x256w8")
    assert L.bf8_gemm_kmajor_workspace(512, 2560, 2048) == 0


def test_nvfp4_and_bf16_geglu_entries_reject_bad_arguments():
    """The NVFP4 quantizer variants (producer partials, dequantized rowwise copy) and the
    bf16 gated-GELU GEMM check their arguments on the host, before any launch."""
    L = _lib.lib()
    null = ctypes.c_void_p(0)
    buf = ctypes.create_string_buffer(1 << 12)
    ptr = ctypes.c_void_p((ctypes.addressof(buf) + 255) // 256 * 256)
    odd = ctypes.c_void_p(ptr.value + 8)
    # producer partials: at least one, and the rowwise blocks need cols % 16 == 0
    rc = L.bf8_quantize_nvfp4_partials_bf16(ptr, 16, 32, ptr, 0, ptr, ptr, null, null, ptr, null)
    assert rc == 1 and b"partials is NULL or empty" in L.bf8_last_error()
    rc = L.bf8_quantize_nvfp4_partials_bf16(ptr, 16, 24, ptr, 4, ptr, ptr, null, null, ptr, null)
    assert rc == 1 and b"cols % 16" in L.bf8_last_error()
    rc = L.bf8_quantize_nvfp4_partials_bf16(ptr, 16, 32, ptr, 4, null, null, null, null, ptr,
                                            null)
    assert rc == 1 and b"both NULL" in L.bf8_last_error()
    # dequantized rowwise copy: deq required and 16-byte aligned, columnwise rows % 16
    rc = L.bf8_quantize_nvfp4_dequant_bf16(ptr, 16, 32, ptr, 0, null, null, null, ptr, null)
    assert rc == 1 and b"needs deq" in L.bf8_last_error()
    rc = L.bf8_quantize_nvfp4_dequant_bf16(ptr, 16, 32, ptr, 0, odd, null, null, ptr, null)
    assert rc == 1 and b"16-byte" in L.bf8_last_error()
    rc = L.bf8_quantize_nvfp4_dequant_bf16(ptr, 24, 32, ptr, 0, ptr, ptr, ptr, ptr, null)
    assert rc == 1 and b"rows % 16" in L.bf8_last_error()
    rc = L.bf8_quantize_nvfp4_dequant_bf16(ptr, 16, 32, ptr, -1, ptr, null, null, ptr, null)
    assert rc == 1 and b"partials is NULL" in L.bf8_last_error()
    # bf16 gated-GELU GEMM: K % 8, and I a multiple of 128
    rc = L.bf8_gemm_geglu_bf16(ptr, 36, ptr, 36, 32, 128, 36, ptr, ptr, ptr, 128, null, ptr,
                               null)
    assert rc == 1 and b"bf8_gemm_geglu_bf16" in L.bf8_last_error()
    rc = L.bf8_gemm_geglu_bf16(ptr, 32, ptr, 32, 32, 100, 32, ptr, ptr, ptr, 128, null, ptr,
                               null)
    assert rc == 1 and b"multiple of 128" in L.bf8_last_error()
