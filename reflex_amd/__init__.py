"""reflex_amd: MI355X-native GGUF quantized-matmul path (Q4_K / Q6_K / Q8_0).

The compute lives in ``librfxq.so`` (HIP C++ host code + an embedded gfx950
code object, see ``build.py``); its C ABI is ``include/rfxq.h``. This package
loads it with ctypes and mirrors the reference's Rust call surface for the
path (``reflex_amd.quant``). There is no CPU fallback: if the library is not
built, or the device is not a gfx950, calls raise.
"""
from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "librfxq.so")

_lib = None


class RfxqWeight(ctypes.Structure):
    """``rfxq_weight`` (include/rfxq.h)."""

    _fields_ = [
        ("ggml_type", ctypes.c_uint32),
        ("in_features", ctypes.c_uint32),
        ("out_features", ctypes.c_uint32),
        ("expert_count", ctypes.c_uint32),
        ("data", ctypes.c_void_p),
        ("len", ctypes.c_uint64),
    ]


class RfxqGemvItem(ctypes.Structure):
    _fields_ = [("x", ctypes.c_void_p), ("w", ctypes.POINTER(RfxqWeight)), ("y", ctypes.c_void_p)]


class RfxqOptions(ctypes.Structure):
    """``rfxq_options`` (include/rfxq.h)."""

    _fields_ = [
        ("quant_mma", ctypes.c_int32),
        ("quant_mma_splits", ctypes.c_uint32),
        ("quant_mma_max_rows", ctypes.c_uint32),
        ("quant_mma_tile", ctypes.c_uint32),
        ("mmq_f16", ctypes.c_int32),
        ("fused_max_rows", ctypes.c_uint32),
    ]


class RfxqGemmPolicy(ctypes.Structure):
    """``rfxq_gemm_policy`` (include/rfxq.h)."""

    _fields_ = [(n, ctypes.c_uint32) for n in ("path", "tile_m", "tile_n", "splits", "sb_per_split")]


# name -> (restype, argtypes); every symbol declared in include/rfxq.h
_P, _U32, _U64, _I = ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_int
_WP = ctypes.POINTER(RfxqWeight)
SIGNATURES = {
    "rfxq_last_error": (ctypes.c_char_p, []),
    "rfxq_last_error_code": (_I, []),
    "rfxq_init": (_I, [_I]),
    "rfxq_get_options": (_I, [ctypes.POINTER(RfxqOptions)]),
    "rfxq_set_options": (_I, [ctypes.POINTER(RfxqOptions)]),
    "rfxq_gemm_policy_for": (_I, [_U32, _U32, _U32, _U32, _U32, ctypes.POINTER(RfxqGemmPolicy)]),
    "rfxq_block_dims": (_I, [_U32, ctypes.POINTER(_U32), ctypes.POINTER(_U32)]),
    "rfxq_dequantize": (_I, [_U32, _P, _U64, _P, _I, _P]),
    "rfxq_gemv_to": (_I, [_P, _U64, _WP, _P, _P]),
    "rfxq_gemv_rows": (_I, [_P, _U64, _WP, _U32, _P, _P]),
    "rfxq_gemv_gather": (_I, [_P, _U64, _WP, _P, _U32, _P, _P]),
    "rfxq_gemv_batch": (_I, [ctypes.POINTER(RfxqGemvItem), _U32, _P]),
    "rfxq_gemv_plan_create": (_I, [ctypes.POINTER(RfxqGemvItem), _U32, _I, ctypes.POINTER(_P)]),
    "rfxq_gemv_plan_run": (_I, [_P, _P]),
    "rfxq_gemv_plan_destroy": (None, [_P]),
    "rfxq_gemm_batch": (_I, [ctypes.POINTER(RfxqGemvItem), _U32, _U32, _P]),
    "rfxq_gemm_plan_create": (_I, [ctypes.POINTER(RfxqGemvItem), _U32, _U32, _I, ctypes.POINTER(_P)]),
    "rfxq_gemm_plan_run": (_I, [_P, _P]),
    "rfxq_gemm_plan_destroy": (None, [_P]),
    "rfxq_quantize_q8_1": (_I, [_P, _U32, _U32, _P, _P, _P]),
    "rfxq_gemm_workspace_size": (_U64, [_WP, _U32]),
    "rfxq_gemm": (_I, [_P, _U64, _WP, _U32, _P, _P, _U64, _P]),
    "rfxq_gemm_no_alloc": (_I, [_P, _U64, _WP, _U32, _P, _P]),
    "rfxq_mmq_block_dots": (_I, [_P, _P, _U32, _WP, _P, _P]),
    "rfxq_route_top_k": (_I, [_P, _U32, _U32, _I, _P, _P]),
    "rfxq_quant_expert_weight": (_I, [_WP, _U32, _WP]),
    "rfxq_expert_gemv": (_I, [_P, _U64, _WP, _U32, _P, _P]),
    "rfxq_expert_gemm": (_I, [_P, _U64, _WP, _U32, _U32, _P, _P, _U64, _P]),
    "rfxq_moe_gather": (_I, [_P, _P, _P, _U32, _U32, _P]),
    "rfxq_moe_scatter_add": (_I, [_P, _P, _P, _P, _U32, _U32, _P]),
    "rfxq_silu_and_mul": (_I, [_P, _P, _P, _U64, _P]),
    "rfxq_moe_ffn_grouped": (_I, [_P, _U32, _U32, _P, _U32, _U32, _I, ctypes.c_float, _WP, _WP, _WP, _P, _P]),
    "rfxq_act_q8_1_size": (_U64, [_U32, _U32]),
    "rfxq_gguf_open": (_I, [ctypes.c_char_p, _P]),
    "rfxq_gguf_close": (None, [_P]),
    "rfxq_gguf_version": (_U32, [_P]),
    "rfxq_gguf_tensor_count": (_U64, [_P]),
    "rfxq_gguf_find_tensor": (_I, [_P, ctypes.c_char_p, _P]),
    "rfxq_gguf_tensor_info": (_I, [_P, _U64, _P, _P, _P, _P, _P]),
    "rfxq_gguf_tensor_data": (_I, [_P, _U64, _P, _P]),
    "rfxq_gguf_meta_u64": (_I, [_P, ctypes.c_char_p, _P]),
    "rfxq_gguf_meta_f64": (_I, [_P, ctypes.c_char_p, _P]),
    "rfxq_gguf_meta_str": (_I, [_P, ctypes.c_char_p, _P]),
    "rfxq_gguf_meta_array_len": (_I, [_P, ctypes.c_char_p, _P]),
    "rfxq_gguf_arena_size": (_U64, [_P, _P, _U32]),
    "rfxq_gguf_upload": (_I, [_P, _P, _U32, _P, _U64, _P, _P]),
    "rfxq_moe_route_device": (_I, [_P, _U32, _U32, _U32, _I, ctypes.c_float, _P, _P, _P]),
    "rfxq_moe_ffn_grouped_device": (_I, [_P, _U32, _U32, _P, _U32, _U32, _I, ctypes.c_float, _WP, _WP, _WP, _P,
                                         _P]),
    "rfxq_quantize_act_q8_1": (_I, [_P, _U32, _U32, _P, _P]),
    "rfxq_rmsnorm_q8_1": (_I, [_P, _P, _U32, _U32, ctypes.c_float, _P, _P, _P]),
    "rfxq_silu_and_mul_q8_1": (_I, [_P, _P, _U32, _U32, _P, _P, _P]),
    "rfxq_gemm_q8_1": (_I, [_P, _U32, _WP, _P, _P, _U64, _P]),
    "rfxq_gemm_gate_up_silu_q8_1": (_I, [_P, _U32, _WP, _WP, _P, _P, _P, _U64, _P]),
    "rfxq_gemm_gate_up_silu_workspace_size": (_U64, [_WP, _U32]),
    "rfxq_gemm_q8_1_batch": (_I, [_P, _U32, _U32, _P]),
    "rfxq_gemm_q8_1_plan_create": (_I, [_P, _U32, _U32, _I, ctypes.POINTER(_P)]),
}


def lib() -> ctypes.CDLL:
    """Load librfxq.so (built by ``python -m reflex_amd.build``); raises if absent."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built; run `python -m reflex_amd.build` "
                               "(there is no CPU fallback for this path)")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


from .quant import *  # noqa: E402,F401,F403
