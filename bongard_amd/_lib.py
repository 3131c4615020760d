"""ctypes binding of libbongard_fp8.so (the C ABI in include/bongard_fp8.h).

Loading never touches the GPU. There is no CPU fallback: if the library is not built,
every FP8 op raises.
"""

import ctypes
from ctypes import c_float, c_int, c_int64, c_size_t, c_uint32, c_void_p, POINTER
from pathlib import Path

LIB_PATH = Path(__file__).resolve().with_name("libbongard_fp8.so")
ABI_VERSION = 18

# name -> (restype, argtypes); mirrors include/bongard_fp8.h one to one.
SIGNATURES = {
    "bf8_last_error": (ctypes.c_char_p, []),
    "bf8_abi_version": (c_int, []),
    "bf8_amax_partials": (c_int64, [c_int64]),
    "bf8_amax_bf16": (c_int, [c_void_p, c_int64, c_void_p, c_void_p]),
    "bf8_scale_from_partials": (c_int, [c_void_p, c_int64, c_int, c_void_p, c_void_p]),
    "bf8_cast_partials_bf16": (c_int, [c_void_p, c_int64, c_int64, c_void_p, c_int64, c_int,
                                       c_void_p, c_void_p, c_void_p, c_void_p]),
    "bf8_cast_bf16": (c_int, [c_void_p, c_int64, c_int64, c_void_p, c_int, c_void_p, c_void_p,
                              c_void_p]),
    "bf8_quantize_bf16": (c_int, [c_void_p, c_int64, c_int64, c_int, c_void_p, c_void_p,
                                  c_void_p, c_void_p, c_void_p]),
    "bf8_quantize_bf16_noalloc": (c_int, [c_void_p, c_int64, c_int64, c_int, c_void_p, c_void_p,
                                          c_void_p, c_void_p]),
    "bf8_quantize_many_partials": (c_int64, [c_int, POINTER(c_int64)]),
    "bf8_quantize_many_bf16": (c_int, [c_int, POINTER(c_void_p), POINTER(c_int64),
                                       POINTER(c_int), POINTER(c_void_p), POINTER(c_void_p),
                                       c_void_p, c_void_p]),
    "bf8_quantize_mx_many_bf16": (c_int, [c_int, POINTER(c_void_p), POINTER(c_int64),
                                          POINTER(c_int64), POINTER(c_int), POINTER(c_void_p),
                                          POINTER(c_void_p), c_void_p]),
    "bf8_gemm_workspace": (c_size_t, [c_int64, c_int64, c_int64]),
    "bf8_gemm": (c_int, [c_void_p, c_int, c_int64, c_void_p, c_int, c_int64, c_int64, c_int64,
                         c_int64, c_void_p, c_void_p, c_int, POINTER(c_int64), c_int, c_void_p,
                         c_void_p, c_int, c_int64, c_void_p, c_size_t, c_void_p]),
    "bf8_gemm_kmajor_workspace": (c_size_t, [c_int64, c_int64, c_int64]),
    "bf8_gemm_kmajor": (c_int, [c_void_p, c_int, c_int64, c_int, c_void_p, c_int, c_int64, c_int64,
                                c_int64, c_int64, c_void_p, c_void_p, c_void_p, c_int, c_int64,
                                c_void_p, c_size_t, c_void_p]),
    "bf8_geglu_partials": (c_int64, [c_int64, c_int64]),
    "bf8_gemm_geglu": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_int64, c_int64, c_int64,
                               c_void_p, c_void_p, c_int, c_void_p, c_int64, c_void_p, c_void_p,
                               c_void_p]),
    "bf8_geglu_partials_elementwise": (c_int64, [c_int64, c_int64]),
    "bf8_geglu_bf16": (c_int, [c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_void_p]),
    "bf8_geglu_bwd_partials": (c_int64, [c_int64, c_int64]),
    "bf8_geglu_bwd": (c_int, [c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_void_p,
                              c_void_p]),
    "bf8_delayed_scale_begin": (c_int, [c_void_p, c_int, c_int, c_void_p]),
    "bf8_delayed_scale_end": (c_int, [c_void_p, c_int, c_void_p, c_int64, c_void_p]),
    "bf8_cast_amax_partials": (c_int64, [c_int64, c_int64, c_int]),
    "bf8_cast_delayed_bf16": (c_int, [c_void_p, c_int64, c_int64, c_void_p, c_int, c_int,
                                      c_void_p, c_int64, c_int, c_void_p, c_void_p, c_void_p,
                                      c_void_p, c_void_p]),
    "bf8_cast_delayed_many_bf16": (c_int, [c_int, c_void_p, c_void_p, c_void_p, c_void_p,
                                           c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                           c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    "bf8_geglu_bwd_delayed_partials": (c_int64, [c_int64, c_int64]),
    "bf8_geglu_bwd_delayed": (c_int, [c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_int,
                                      c_int, c_void_p, c_int64, c_int, c_void_p, c_void_p,
                                      c_void_p, c_void_p, c_void_p]),
    "bf8_axiswise_workspace": (c_size_t, [c_int64, c_int64]),
    "bf8_quantize_axiswise_bf16": (c_int, [c_void_p, c_int64, c_int64, c_int, c_void_p, c_void_p,
                                           c_void_p, c_void_p, c_void_p, c_size_t, c_void_p]),
    "bf8_gemm_axiswise": (c_int, [c_void_p, c_int, c_int64, c_void_p, c_int, c_int64, c_int64,
                                  c_int64, c_int64, c_void_p, c_int, c_void_p, c_int, c_void_p,
                                  c_void_p, c_int, c_int64, c_void_p, c_size_t, c_void_p]),
    "bf8_mx_scale_ld": (c_int64, [c_int64]),
    "bf8_quantize_mx_bf16": (c_int, [c_void_p, c_int64, c_int64, c_int, c_void_p, c_void_p,
                                     c_void_p, c_void_p, c_void_p]),
    "bf8_gemm_mx_workspace": (c_size_t, [c_int64, c_int64, c_int64]),
    "bf8_quantize_nvfp4_bf16": (c_int, [c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_void_p,
                                        c_void_p, c_void_p, c_void_p, c_void_p]),
    "bf8_quantize_nvfp4_partials_bf16": (c_int, [c_void_p, c_int64, c_int64, c_void_p, c_int64,
                                                 c_void_p, c_void_p, c_void_p, c_void_p,
                                                 c_void_p, c_void_p]),
    "bf8_quantize_nvfp4_dequant_bf16": (c_int, [c_void_p, c_int64, c_int64, c_void_p, c_int64,
                                                c_void_p, c_void_p, c_void_p, c_void_p,
                                                c_void_p]),
    "bf8_dequant_nvfp4": (c_int, [c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_void_p]),
    "bf8_gemm_bf16_workspace": (c_size_t, [c_int64, c_int64, c_int64]),
    "bf8_gemm_bf16": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_int64, c_int64, c_int64,
                              c_void_p, c_void_p, c_void_p, c_int, c_int64, c_void_p, c_size_t,
                              c_void_p]),
    "bf8_gemm_geglu_bf16": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_int64, c_int64,
                                    c_int64, c_void_p, c_void_p, c_void_p, c_int64, c_void_p,
                                    c_void_p, c_void_p]),
    "bf8_gemm_mx": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int64, c_void_p,
                            c_int64, c_int64, c_int64, c_int64, c_void_p, c_void_p, c_int,
                            c_int64, c_void_p, c_size_t, c_void_p]),
    "bf8_gemm_geglu_mx": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int64,
                                  c_void_p, c_int64, c_int64, c_int64, c_int64, c_void_p,
                                  c_int64, c_void_p, c_void_p]),
    "bf8_gemm_geglu_mx_quant": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_void_p,
                                        c_int64, c_void_p, c_int64, c_int64, c_int64, c_int64,
                                        c_void_p, c_int64, c_void_p, c_void_p, c_int64,
                                        c_void_p, c_void_p, c_int64, c_void_p, c_void_p]),
    "bf8_delayed_scale_fold": (c_int, [c_void_p, c_int, c_int, c_void_p, c_int64, c_int,
                                       c_void_p, c_void_p]),
    "bf8_gemm_geglu_quant": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_int64, c_int64,
                                     c_int64, c_void_p, c_void_p, c_int, c_void_p, c_void_p,
                                     c_int64, c_void_p, c_void_p, c_void_p, c_void_p,
                                     c_void_p]),
    "bf8_rmsnorm_partials": (c_int64, [c_int64]),
    "bf8_rmsnorm_bf16": (c_int, [c_void_p, c_int64, c_int64, c_void_p, c_float, c_int,
                                 c_void_p, c_void_p, c_void_p, c_void_p]),
    "bf8_rmsnorm_bwd_workspace": (c_size_t, [c_int64, c_int64]),
    "bf8_rmsnorm_bwd_bf16": (c_int, [c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_float,
                                     c_int, c_void_p, c_void_p, c_void_p, c_size_t, c_void_p]),
}

_lib = None


class Fp8LibError(RuntimeError):
    """A libbongard_fp8 entry point returned a non-zero status."""


def lib():
    """The loaded library; raises if it has not been built (no fallback exists)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH.name} is not built; run `python -m bongard_amd.build` "
                "(the FP8 path has no CPU or PyTorch fallback)")
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        version = handle.bf8_abi_version()
        if version != ABI_VERSION:
            raise RuntimeError(f"{LIB_PATH.name} ABI {version} != expected {ABI_VERSION}; rebuild")
        _lib = handle
    return _lib


def check(rc, what):
    if rc != 0:
        msg = lib().bf8_last_error().decode(errors="replace")
        raise Fp8LibError(f"{what} failed ({rc}): {msg}")
