"""ctypes binding of libeimoe.so (the C ABI declared in include/eimoe.h).

The library is built in-tree (``python -m easyinfra_amd.build``).  There is no
fallback: if it is missing, every op raises.
"""
from __future__ import annotations

import ctypes
from ctypes import c_int, c_float, c_longlong, c_size_t, c_void_p, c_char_p, POINTER
from pathlib import Path

LIB_PATH = Path(__file__).resolve().with_name("libeimoe.so")

EIMOE_OK = 0
ERR_NULL, ERR_SHAPE, ERR_ALIGN, ERR_DTYPE, ERR_WORKSPACE, ERR_HIP = -1, -2, -3, -4, -5, -6
F32, BF16, FP8 = 0, 1, 2
RENORMALIZE, Y_F32, W8A8, ROUTING_IN, H_SPLIT, FP32 = 1, 2, 4, 8, 16, 32
LOGITS_BF16 = 1   # eimoe_moe_prologue flag
TILE_AUTO, TILE_256x256, TILE_128x128, TILE_32x128, TILE_16x64, TILE_STREAM, TILE_64x128 = 0, 1, 2, 3, 4, 5, 6
MAX_TOPK, MAX_EXPERTS, MAX_SEGMENTS = 32, 512, 1024

_i32p = POINTER(ctypes.c_int32)
_f32p = POINTER(ctypes.c_float)

# name -> (restype, argtypes); mirrors include/eimoe.h
SIGNATURES = {
    "eimoe_abi_version": (c_int, []),
    "eimoe_last_error": (c_char_p, []),
    "eimoe_release_streams": (c_int, []),
    "eimoe_router_topk": (c_int, [c_void_p, c_int, c_int, c_int, c_int, c_void_p, c_void_p, c_void_p]),
    "eimoe_router_grouped_topk": (c_int, [c_void_p, c_int, c_int, c_int, c_int, c_int, c_void_p, c_int, c_float,
                                          c_void_p, c_void_p, c_void_p]),
    "eimoe_eplb_map": (c_int, [c_void_p, c_int, c_int, c_void_p, c_int, c_int, c_void_p, c_void_p, c_void_p]),
    "eimoe_moe_prologue_workspace_bytes": (c_size_t, [c_int, c_int, c_int]),
    "eimoe_moe_prologue": (c_int, [c_void_p, c_void_p, c_void_p, c_float, c_void_p, c_int, c_int, c_int, c_int,
                                   c_void_p, c_void_p, c_void_p, c_void_p, c_size_t, c_void_p]),
    "eimoe_align_workspace_bytes": (c_size_t, [c_int, c_int, c_int]),
    "eimoe_align": (c_int, [c_void_p, c_int, c_int, c_int, c_int, c_void_p, c_void_p, c_void_p, c_void_p,
                            c_void_p, c_void_p, c_size_t, c_void_p]),
    "eimoe_route_align": (c_int, [c_void_p, c_int, c_int, c_int, c_int, c_int, c_int, c_void_p, c_void_p,
                                  c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    "eimoe_counts_to_offsets": (c_int, [c_void_p, c_int, c_void_p, c_void_p]),
    "eimoe_gather": (c_int, [c_void_p, c_int, c_int, c_void_p, c_void_p, c_int, c_void_p, c_void_p]),
    "eimoe_gemm_gate_up_silu": (c_int, [c_void_p, c_void_p, c_int, c_int, c_void_p, c_int, c_void_p, c_int, c_int,
                                        c_void_p, c_int, c_int, c_int, c_void_p, c_int, c_void_p]),
    "eimoe_gemm_down": (c_int, [c_void_p, c_int, c_void_p, c_int, c_void_p, c_int, c_void_p, c_int, c_int, c_int,
                                c_void_p, c_int, c_int, c_int, c_void_p]),
    "eimoe_gemm_gate_up_silu_w8a8": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_void_p, c_void_p, c_int,
                                             c_int, c_void_p, c_int, c_int, c_int, c_void_p, c_int, c_void_p]),
    "eimoe_gemm_down_w8a8": (c_int, [c_void_p, c_void_p, c_int, c_void_p, c_void_p, c_int, c_void_p, c_int, c_int,
                                     c_int, c_void_p, c_int, c_int, c_int, c_void_p]),
    "eimoe_grouped_gemm": (c_int, [c_void_p, c_void_p, c_int, c_int, c_void_p, c_int, c_void_p, c_longlong, c_int,
                                   c_int,
                                   c_void_p, c_int, c_int, c_int, c_void_p, c_int, c_int, c_void_p]),
    "eimoe_grouped_gemm_ptrs": (c_int, [c_void_p, c_void_p, c_int, c_int, c_void_p, c_int, c_int, c_int, c_void_p,
                                        c_int, c_int, c_int, c_void_p, c_int, c_int, c_void_p]),
    "eimoe_combine": (c_int, [c_void_p, c_int, c_int, c_longlong, c_void_p, c_void_p, c_int, c_int, c_int,
                              c_void_p, c_int, c_void_p, c_int, c_void_p]),
    "eimoe_quantize_rows_fp8": (c_int, [c_void_p, c_int, c_longlong, c_int, c_void_p, c_void_p, c_void_p]),
    "eimoe_fused_moe_workspace_bytes": (c_size_t, [c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int]),
    "eimoe_fused_moe_down_split": (c_int, [c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int]),
    "eimoe_fused_moe": (c_int, [c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int, c_void_p, c_void_p, c_int,
                                c_void_p, c_void_p, c_int, c_int, c_void_p, c_void_p, c_int, c_int, c_void_p, c_int,
                                c_void_p, c_size_t, c_void_p, c_void_p, c_void_p]),
    "eimoe_fused_moe_static_bytes": (c_size_t, []),
    "eimoe_fused_moe_static": (c_int, [c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int, c_void_p, c_void_p,
                                       c_int, c_void_p, c_void_p, c_int, c_int, c_void_p, c_void_p, c_int, c_int,
                                       c_void_p, c_int, c_void_p, c_void_p, c_void_p]),
}

_lib = None


class EimoeError(RuntimeError):
    def __init__(self, code: int, fn: str, msg: str):
        super().__init__(f"{fn} failed ({code}): {msg}")
        self.code = code


def lib() -> ctypes.CDLL:
    """Load libeimoe.so once and declare its signatures; raise if it is not built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is not built; run `python -m easyinfra_amd.build` "
                               "(the HIP path has no fallback)")
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        if handle.eimoe_abi_version() != 1:
            raise RuntimeError("libeimoe.so ABI version mismatch")
        _lib = handle
    return _lib


def call(name: str, *args) -> int:
    rc = getattr(lib(), name)(*args)
    if rc != EIMOE_OK:
        raise EimoeError(rc, name, (lib().eimoe_last_error() or b"").decode())
    return rc


def last_error() -> str:
    return (lib().eimoe_last_error() or b"").decode()
