"""ctypes binding of libcudeep_amd.so (the C-ABI in include/cudeep_amd.h).

The library is the product: if it is missing this module raises, there is
no CPU fallback.  Device memory and streams come from PyTorch-ROCm (plain
pointers cross the boundary); the library itself never sees a torch type.
"""
from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libcudeep_amd.so")

CDX_OK = 0
CDX_ERR_INVALID_ARG = 1
CDX_ERR_UNSUPPORTED = 2
CDX_ERR_HIP = 3
CDX_ERR_WORKSPACE = 4

OP_N, OP_T = 0, 1
EPI_NONE, EPI_RELU, EPI_GELU, EPI_SILU, EPI_SIGMOID = 0, 1, 2, 3, 4
# activation-backward epilogues (cdx_gemm_fused): C = (A B) * act'(aux)
EPI_BWD_RELU, EPI_BWD_GELU, EPI_BWD_SILU, EPI_BWD_SIGMOID = 8, 9, 10, 11
ACT_TANH, ACT_LEAKY_RELU = 5, 6   # elementwise activations only
BIAS_NONE, BIAS_ROW, BIAS_COL = 0, 1, 2
PREC_FP32, PREC_TF32MODE, PREC_TF32MODE4 = 0, 1, 2

_i64 = ctypes.c_int64
_int = ctypes.c_int
_f32 = ctypes.c_float
_vp = ctypes.c_void_p
_sz = ctypes.c_size_t

# name -> (restype, argtypes); every symbol declared in include/cudeep_amd.h
SIGNATURES = {
    "cdx_last_error": (ctypes.c_char_p, []),
    "cdx_version": (ctypes.c_char_p, []),
    "cdx_sgemm_f32": (_int, [_vp, _vp, _vp, _i64, _i64, _i64, _vp]),
    "cdx_gemm_tf32mode": (_int, [_vp, _vp, _vp, _i64, _i64, _i64, _vp]),
    "cdx_gemm_ex": (_int, [_int, _int, _int, _i64, _i64, _i64, _vp, _i64, _vp, _i64,
                           _vp, _i64, _vp, _int, _int, _vp]),
    "cdx_gemm_workspace_size": (_sz, [_int, _int, _int, _i64, _i64, _i64]),
    "cdx_gemm_ex_ws": (_int, [_int, _int, _int, _i64, _i64, _i64, _vp, _i64, _vp, _i64,
                              _vp, _i64, _vp, _int, _int, _vp, _sz, _vp]),
    "cdx_gemm_fused_workspace_size": (_sz, [_int, _int, _int, _i64, _i64, _i64, _int]),
    "cdx_gemm_fused": (_int, [_int, _int, _int, _i64, _i64, _i64, _vp, _i64, _vp, _i64,
                              _vp, _i64, _vp, _int, _int, _vp, _i64, _vp, _vp, _sz, _vp]),
    "cdx_matmul_fused_act": (_int, [_vp, _vp, _vp, _i64, _i64, _i64, _int, _vp]),
    "cdx_hgemm_f16": (_int, [_vp, _vp, _vp, _i64, _i64, _i64, _vp]),
    "cdx_gemm16_ex": (_int, [_int, _int, _int, _i64, _i64, _i64, _vp, _i64, _vp, _i64,
                             _vp, _i64, _vp, _int, _int, _vp]),
    "cdx_dgemm": (_int, [_int, _int, _i64, _i64, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _vp]),
    "cdx_im2col_f32": (_int, [_vp, _vp] + [_i64] * 10 + [_vp]),
    "cdx_conv2d_forward_workspace_size": (_sz, [_i64] * 10),
    "cdx_conv2d_forward_f32": (_int, [_vp, _vp, _vp, _vp] + [_i64] * 11 + [_int, _vp, _sz, _vp]),
    "cdx_conv2d_forward_implicit_f32": (_int, [_vp, _vp, _vp, _vp] + [_i64] * 11 + [_vp]),
    "cdx_sum_reduce_rows_workspace_size": (_sz, [_i64, _i64]),
    "cdx_sum_reduce_rows_f32": (_int, [_vp, _vp, _i64, _i64, _vp, _sz, _vp]),
    "cdx_broadcast_add_row_f32": (_int, [_vp, _vp, _vp, _i64, _i64, _vp]),
    "cdx_activation_forward_f32": (_int, [_vp, _vp, _i64, _int, _f32, _vp]),
    "cdx_activation_backward_f32": (_int, [_vp, _vp, _vp, _i64, _int, _f32, _vp]),
    "cdx_conv2d_winograd_workspace_size": (_sz, [_i64] * 7),
    "cdx_conv2d_forward_winograd_f32": (_int, [_vp, _vp, _vp, _vp] + [_i64] * 7 + [_int, _vp, _sz, _vp]),
    "cdx_col2im_f32": (_int, [_vp, _vp] + [_i64] * 10 + [_vp]),
    "cdx_conv2d_backward_data_workspace_size": (_sz, [_i64] * 11),
    "cdx_conv2d_backward_data_f32": (_int, [_vp, _vp, _vp] + [_i64] * 11 + [_int, _vp, _sz, _vp]),
    "cdx_conv2d_backward_data_winograd_workspace_size": (_sz, [_i64] * 7),
    "cdx_conv2d_backward_data_winograd_f32": (_int, [_vp, _vp, _vp] + [_i64] * 7 + [_int, _vp, _sz, _vp]),
    "cdx_conv2d_backward_weight_workspace_size": (_sz, [_i64] * 11),
    "cdx_conv2d_backward_weight_f32": (_int, [_vp, _vp, _vp] + [_i64] * 11 + [_int, _vp, _sz, _vp]),
    "cdx_conv2d_backward_weight_f32_noalloc": (_int, [_vp, _vp, _vp] + [_i64] * 11 + [_int, _vp]),
    "cdx_conv2d_backward_bias_f32": (_int, [_vp, _vp, _i64, _i64, _i64, _vp]),
    "cdx_conv2d_forward_f64": (_int, [_vp, _vp, _vp, _vp] + [_i64] * 11 + [_vp]),
    "cdx_conv2d_backward_data_f64": (_int, [_vp, _vp, _vp] + [_i64] * 11 + [_vp]),
    "cdx_conv2d_backward_weight_f64": (_int, [_vp, _vp, _vp] + [_i64] * 11 + [_vp]),
    "cdx_conv2d_backward_bias_f64": (_int, [_vp, _vp, _i64, _i64, _i64, _vp]),
    "cdx_strided_copy": (_int, [_vp, _vp, _int, _vp, _vp, _int, _vp]),
    "cdx_fill": (_int, [_vp, _i64, ctypes.c_double, _int, _vp]),
    "cdx_binary": (_int, [_int, _int, _vp, _vp, _vp, _i64, _vp]),
    "cdx_randn": (_int, [_vp, _i64, _int, ctypes.c_uint64, ctypes.c_uint64, _vp]),
    "cdx_sum_workspace_size": (_sz, [_int]),
    "cdx_sum": (_int, [_vp, _vp, _i64, _int, _vp, _sz, _vp]),
    "cdx_broadcast_add_row_f64": (_int, [_vp, _vp, _vp, _i64, _i64, _vp]),
    "cdx_sum_reduce_rows_f64": (_int, [_vp, _vp, _i64, _i64, _vp, _sz, _vp]),
    "cdx_activation_forward_f64": (_int, [_vp, _vp, _i64, _int, _f32, _vp]),
    "cdx_activation_backward_f64": (_int, [_vp, _vp, _vp, _i64, _int, _f32, _vp]),
}

DTYPE_F32, DTYPE_F64, DTYPE_F16, DTYPE_BF16 = 0, 1, 2, 3
BINARY_ADD, BINARY_SUB, BINARY_MUL = 0, 1, 2

_lib = None


class CdxError(RuntimeError):
    """A non-zero status from the C-ABI (message from cdx_last_error)."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"[cdx status {code}] {msg}")
        self.code = code


def lib():
    """Load libcudeep_amd.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} not found: build it with __graft_entry__.build() "
                "(make -C cudeep_amd/csrc); there is no CPU fallback")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(code: int) -> None:
    if code != CDX_OK:
        msg = lib().cdx_last_error().decode(errors="replace")
        raise CdxError(code, msg)


def call(name: str, *args) -> None:
    """Call an int-returning entry point and raise CdxError on failure."""
    check(getattr(lib(), name)(*args))
