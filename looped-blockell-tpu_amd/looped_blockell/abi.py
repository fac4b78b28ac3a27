"""ctypes binding of the C ABI in include/lbk.h (liblbk.so).

This is the binding a non-torch caller would use; it mirrors the header one to
one.  Pointers are plain integers (device addresses), streams are raw HIP
stream handles.  ``check`` turns a status code into a RuntimeError carrying
``lbk_status_string``.
"""

from __future__ import annotations

import ctypes as C
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liblbk.so")

LBK_OK = 0
LBK_ERR_NULL = 1
LBK_ERR_TILE = 2
LBK_ERR_SHAPE = 3
LBK_ERR_ALIGN = 4
LBK_ERR_WORKSPACE = 5
LBK_ERR_LAUNCH = 6
LBK_ERR_ARG = 7
LBK_ERR_COLUMN = 8
LBK_ERR_TOO_LARGE = 9


class Bell(C.Structure):
    """``lbk_bell``: one Block-ELL weight with bf16 tiles [B_in, B_out]."""

    _fields_ = [("values", C.c_void_p), ("col_idx", C.c_void_p),
                ("R", C.c_int32), ("K", C.c_int32), ("B", C.c_int32)]


class BellTernary(C.Structure):
    """``lbk_bell_ternary``: packed 2-bit tiles, fp32 block scales, column indices."""

    _fields_ = [("packed", C.c_void_p), ("scales", C.c_void_p), ("col_idx", C.c_void_p),
                ("R", C.c_int32), ("K", C.c_int32), ("B", C.c_int32)]


class TernaryAcc(C.Structure):
    """``lbk_ternary_acc``: optional accumulator exports of the ternary SwiGLU (device pointers)."""

    _fields_ = [("acc_gate", C.c_void_p), ("acc_up", C.c_void_p), ("acc_down", C.c_void_p),
                ("gate_pre", C.c_void_p), ("up_pre", C.c_void_p)]


LBK_MAX_CORE_BLOCKS = 8


class CoreBlock(C.Structure):
    """``lbk_core_block``: one core block of the looped core (norm scale, SwiGLU weights, biases)."""

    _fields_ = [("norm_scale", C.c_void_p), ("gate", Bell), ("up", Bell), ("down", Bell),
                ("b_gate", C.c_void_p), ("b_up", C.c_void_p), ("b_down", C.c_void_p)]


# (name, restype, argtypes) for every entry point of include/lbk.h
_P = C.c_void_p
_I64 = C.c_int64
_I32 = C.c_int32
_SZ = C.c_size_t
_F = C.c_float
_PB = C.POINTER(Bell)
_PT = C.POINTER(BellTernary)
SIGNATURES = {
    "lbk_status_string": (C.c_char_p, [C.c_int]),
    "lbk_version": (C.c_int, []),
    "lbk_check_columns": (C.c_int, [_P, _I64, _I32, _P, _P]),
    "lbk_topology_alive_counts": (C.c_int, [_P, _I32, _I32, _P, _P, _P]),
    "lbk_topology_compact_bf16": (C.c_int, [_P, _P, _P, _I32, _I32, _I32, _I32, _P, _P, _P, _P]),
    "lbk_column_importance": (C.c_int, [_P, _P, _I32, _I32, _P, _I32, _I32, _I32, _P, _P]),
    "lbk_column_permutation": (C.c_int, [_P, _I32, _P, _P]),
    "lbk_apply_permutation_bf16": (C.c_int, [_P, _P, _P, _I32, _I32, _I32, _P, _I32, _I32, _P, _P, _P, _P]),
    "lbk_k_active_macros": (C.c_int, [_P, _P, _I32, _I32, _I32, _P, _P]),
    "lbk_gather_rows": (C.c_int, [_P, _I64, _I64, _P, _I64, _P, _P]),
    "lbk_transposed_index": (C.c_int, [_P, _I32, _I32, _I32, _P, _P, _P]),
    "lbk_block_ell_matmul_bwd_workspace_bytes": (C.c_size_t, [_I64, _I32, _PB]),
    "lbk_block_ell_matmul_bwd_bf16": (C.c_int, [_P, _P, _I64, _I32, _PB, _P, _P, _P, C.c_size_t, _P]),
    "lbk_dense_to_block_ell": (C.c_int, [_P, _I64, _I32, _I32, _I32, _I32, _P, _I32, _P, _P]),
    "lbk_block_ell_to_dense": (C.c_int, [_P, _P, _I32, _I32, _I32, _I32, _I32, _P, _I64, _P]),
    "lbk_block_ell_topk_columns": (C.c_int, [_P, _I64, _I32, _I32, _I32, _I32, _I32, _P, _P]),
    "lbk_ternary_check_codes": (C.c_int, [_P, _I64, _P, _P]),
    "lbk_block_ell_matmul_bf16": (C.c_int, [_P, _I64, _I32, _I64, _PB, _P, _P, _I64, _P]),
    "lbk_block_ell_matmul_workspace_bytes": (_SZ, [_I64, _I32, _PB]),
    "lbk_block_ell_matmul_ws_bf16": (C.c_int, [_P, _I64, _I32, _PB, _P, _P, _P, _SZ, _P]),
    "lbk_block_ell_matmul_prepacked_bytes": (_SZ, [_I32, _PB]),
    "lbk_block_ell_matmul_prepack_bf16": (C.c_int, [_I32, _PB, _P, _SZ, _P]),
    "lbk_block_ell_matmul_prepacked_bf16": (C.c_int, [_P, _I64, _I32, _PB, _P, _SZ, _P, _P, _P]),
    "lbk_swiglu_workspace_bytes": (_SZ, [_I64, _I32, _PB, _PB, _PB, C.c_int]),
    "lbk_swiglu_fwd_bf16": (C.c_int, [_P, _I64, _I32, _PB, _PB, _PB, C.c_int, _P, _P, _P, _P, _P, _SZ, _P]),
    "lbk_noalloc_scratch_bytes": (_SZ, []),
    "lbk_noalloc_init": (C.c_int, []),
    "lbk_swiglu_forward_path": (C.c_int, [_I64, _I32, _PB, _PB, _PB, C.c_int]),
    "lbk_swiglu_fwd_bf16_noalloc": (C.c_int, [_P, _I64, _I32, _PB, _PB, _PB, C.c_int, _P, _P]),
    "lbk_swiglu_fwd_bias_bf16": (C.c_int, [_P, _I64, _I32, _PB, _PB, _PB, _P, _P, _P, C.c_int, _P, _P, _P, _P, _P,
                                           _SZ, _P]),
    "lbk_diagonal_injection_bwd_workspace_bytes": (_SZ, [_I64, _I32]),
    "lbk_diagonal_injection_bwd_bf16": (C.c_int, [_P, _P, _P, _P, _P, _I64, _I32, _P, _P, _P, _P, _P, _SZ, _P]),
    "lbk_swiglu_prepacked_bytes": (_SZ, [_I32, _PB, _PB, _PB]),
    "lbk_swiglu_prepack_bf16": (C.c_int, [_I32, _PB, _PB, _PB, _P, _SZ, _P]),
    "lbk_swiglu_prepacked_workspace_bytes": (_SZ, [_I64, _I32, _PB, _PB, _PB, C.c_int]),
    "lbk_swiglu_fwd_prepacked_bf16": (C.c_int, [_P, _I64, _I32, _PB, _PB, _PB, _P, _SZ, _P, _P, _P, C.c_int, _P,
                                                _P, _P, _P, _P, _SZ, _P]),
    "lbk_swiglu_bwd_workspace_bytes": (_SZ, [_I64, _I32, _PB, _PB, _PB]),
    "lbk_swiglu_bwd_bias_workspace_bytes": (_SZ, [_I64, _I32, _PB, _PB, _PB]),
    "lbk_swiglu_bwd_bias_bf16": (C.c_int, [_P, _P, _P, _P, _P, _I64, _I32, _PB, _PB, _PB, C.c_int, _P, _P, _P, _P,
                                           _P, _P, _P, _P, _SZ, _P]),
    "lbk_swiglu_bwd_bf16": (C.c_int, [_P, _P, _P, _P, _P, _I64, _I32, _PB, _PB, _PB, C.c_int, _P, _P, _P, _P, _P,
                                      _SZ, _P]),
    "lbk_rmsnorm_bf16": (C.c_int, [_P, _I64, _I32, _P, _F, _P, _P]),
    "lbk_rmsnorm_bwd_workspace_bytes": (_SZ, [_I64, _I32]),
    "lbk_rmsnorm_bwd_bf16": (C.c_int, [_P, _P, _I64, _I32, _P, _F, _P, _P, _P, _SZ, _P]),
    "lbk_diagonal_injection_bf16": (C.c_int, [_P, _P, _P, _P, _I64, _I32, _P, _P]),
    "lbk_looped_workspace_bytes": (_SZ, [_I64, _I32, _PB, _PB, _PB]),
    "lbk_looped_swiglu_bf16": (C.c_int, [_P, _I64, _I32, _P, _F, _I32, _PB, _PB, _PB, _P, _P, _SZ, _P]),
    "lbk_looped_swiglu_bias_bf16": (C.c_int, [_P, _I64, _I32, _P, _F, _I32, _PB, _PB, _PB, _P, _P, _P, _P, _P, _SZ,
                                              _P]),
    "lbk_looped_swiglu_persistent_bf16": (C.c_int, [_P, _I64, _I32, _P, _F, _I32, _PB, _PB, _PB, _P, _P, _SZ,
                                                    _P]),
    "lbk_looped_swiglu_launches_bf16": (C.c_int, [_P, _I64, _I32, _P, _F, _I32, _PB, _PB, _PB, _P, _P, _SZ, _P]),
    "lbk_looped_core_workspace_bytes": (_SZ, [_I64, _I32, _I32, C.POINTER(CoreBlock)]),
    "lbk_looped_core_bf16": (C.c_int, [_P, _P, _P, _P, _I64, _I32, _I32, C.POINTER(CoreBlock), _F, _I32, _P, _I64,
                                       _P, _P, _SZ, _P]),
    "lbk_looped_core_persistent_bf16": (C.c_int, [_P, _P, _P, _P, _I64, _I32, _I32, C.POINTER(CoreBlock), _F, _I32,
                                                  _P, _I64, _P, _P, _SZ, _P]),
    "lbk_quantize_act_int8": (C.c_int, [_P, _I64, _I32, _I64, _P, _P, _P]),
    "lbk_pack_ternary": (C.c_int, [_P, _I32, _I32, _I32, _P, _P]),
    "lbk_ternary_quantize_weights_bf16": (C.c_int, [_P, _I32, _I32, _I32, _P, _P, _P]),
    "lbk_ternary_matmul": (C.c_int, [_P, _P, _I64, _I32, _PT, _P, _P, _P]),
    "lbk_ternary_swiglu_workspace_bytes": (_SZ, [_I64, _I32, _PT, _PT, _PT]),
    "lbk_swiglu_fwd_ternary": (C.c_int, [_P, _P, _I64, _I32, _PT, _PT, _PT, _P, _P, _P, _P, _P, _P, _SZ, _P]),
    "lbk_swiglu_fwd_ternary_acc": (C.c_int, [_P, _P, _I64, _I32, _PT, _PT, _PT, _P, _P, _P, _P, _P,
                                             C.POINTER(TernaryAcc), _P, _SZ, _P]),
    "lbk_ternary_prepared_bytes": (_SZ, [_I32, _PT, _PT, _PT]),
    "lbk_ternary_prepare": (C.c_int, [_I32, _PT, _PT, _PT, _P, _SZ, _P]),
    "lbk_ternary_prepared_workspace_bytes": (_SZ, [_I64, _I32, _PT, _PT, _PT]),
    "lbk_swiglu_fwd_ternary_prepared": (C.c_int, [_P, _P, _I64, _I32, _PT, _PT, _PT, _P, _SZ, _P, _P, _P, _P, _P,
                                                  C.POINTER(TernaryAcc), _P, _SZ, _P]),
}

_lib = None


def load(path: str = LIB_PATH) -> C.CDLL:
    """Load liblbk.so and attach the prototypes.  Raises if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise ImportError(f"liblbk.so not built at {path}; run looped-blockell-tpu_amd/build.py")
    lib = C.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def status_string(code: int) -> str:
    return load().lbk_status_string(code).decode()


def check(code: int, what: str = "lbk") -> None:
    if code != LBK_OK:
        raise RuntimeError(f"{what}: {status_string(code)} (status {code})")


def exported_symbols() -> list[str]:
    return list(SIGNATURES)
