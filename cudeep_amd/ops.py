"""Thin tensor-level wrappers over the C-ABI, for callers that hold
PyTorch-ROCm device tensors (tests, bench, the host layer).  PyTorch only
supplies device memory and the current stream; all arithmetic happens in
libcudeep_amd.so.  Every wrapper validates shapes / dtypes / devices on the
host before any launch, so a bad call raises instead of faulting.
"""
from __future__ import annotations

import torch

from . import _lib as L


def _stream():
    return ctypes_stream(torch.cuda.current_stream())


def ctypes_stream(s) -> int:
    return int(s.cuda_stream)


def _need(t: torch.Tensor, name: str, dtype=torch.float32):
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if not t.is_cuda:
        raise ValueError(f"{name} must be a device tensor")
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")


def _ld(t: torch.Tensor, name: str) -> int:
    """Leading dimension of a row-major 2-D view (unit column stride)."""
    if t.dim() != 2:
        raise ValueError(f"{name} must be 2-D")
    if t.stride(1) != 1 and t.size(1) > 1:
        raise ValueError(f"{name} must have unit column stride")
    return max(t.stride(0), t.size(1), 1)


def gemm(A: torch.Tensor, B: torch.Tensor, *, precision: int = L.PREC_FP32,
         transA: bool = False, transB: bool = False, bias: torch.Tensor | None = None,
         bias_mode: int = L.BIAS_NONE, epilogue: int = L.EPI_NONE,
         out: torch.Tensor | None = None) -> torch.Tensor:
    """C = epi(op(A) @ op(B) + bias).  A, B are row-major storage; transA /
    transB select the transpose, so x @ W.T is gemm(x, W, transB=True)."""
    _need(A, "A")
    _need(B, "B")
    M, K = (A.shape[1], A.shape[0]) if transA else (A.shape[0], A.shape[1])
    K2, N = (B.shape[1], B.shape[0]) if transB else (B.shape[0], B.shape[1])
    if K != K2:
        raise ValueError(f"inner dimensions differ: {K} vs {K2}")
    if out is None:
        out = torch.empty((M, N), device=A.device, dtype=torch.float32)
    _need(out, "out")
    if tuple(out.shape) != (M, N):
        raise ValueError("out has the wrong shape")
    bptr = None
    if bias_mode != L.BIAS_NONE:
        if bias is None:
            raise ValueError("bias_mode set but bias is None")
        _need(bias, "bias")
        want = M if bias_mode == L.BIAS_ROW else N
        if bias.numel() != want or not bias.is_contiguous():
            raise ValueError("bias has the wrong size or is not contiguous")
        bptr = bias.data_ptr()
    L.call("cdx_gemm_ex", precision, int(transA), int(transB), M, N, K,
           A.data_ptr(), _ld(A, "A"), B.data_ptr(), _ld(B, "B"),
           out.data_ptr(), _ld(out, "out"), bptr, bias_mode, epilogue, _stream())
    return out


def sgemm(A, B, out=None):
    """C = A @ B, FP32 MFMA (cdx_sgemm_f32); A, B contiguous row-major."""
    _need(A, "A")
    _need(B, "B")
    if A.dim() != 2 or B.dim() != 2 or A.shape[1] != B.shape[0]:
        raise ValueError("sgemm: shape mismatch")
    if not (A.is_contiguous() and B.is_contiguous()):
        raise ValueError("sgemm: operands must be contiguous")
    M, K = A.shape
    N = B.shape[1]
    if out is None:
        out = torch.empty((M, N), device=A.device, dtype=torch.float32)
    L.call("cdx_sgemm_f32", A.data_ptr(), B.data_ptr(), out.data_ptr(), M, N, K, _stream())
    return out


def gemm_tf32mode(A, B, out=None):
    """C = A @ B in TF32 mode (bf16x3 split MFMA, cdx_gemm_tf32mode)."""
    _need(A, "A")
    _need(B, "B")
    if A.dim() != 2 or B.dim() != 2 or A.shape[1] != B.shape[0]:
        raise ValueError("gemm_tf32mode: shape mismatch")
    if not (A.is_contiguous() and B.is_contiguous()):
        raise ValueError("gemm_tf32mode: operands must be contiguous")
    M, K = A.shape
    N = B.shape[1]
    if out is None:
        out = torch.empty((M, N), device=A.device, dtype=torch.float32)
    L.call("cdx_gemm_tf32mode", A.data_ptr(), B.data_ptr(), out.data_ptr(), M, N, K, _stream())
    return out


def dgemm(A, B, transA=False, transB=False, out=None):
    _need(A, "A", torch.float64)
    _need(B, "B", torch.float64)
    M, K = (A.shape[1], A.shape[0]) if transA else (A.shape[0], A.shape[1])
    K2, N = (B.shape[1], B.shape[0]) if transB else (B.shape[0], B.shape[1])
    if K != K2:
        raise ValueError("dgemm: inner dimensions differ")
    if out is None:
        out = torch.empty((M, N), device=A.device, dtype=torch.float64)
    L.call("cdx_dgemm", int(transA), int(transB), M, N, K, A.data_ptr(), _ld(A, "A"),
           B.data_ptr(), _ld(B, "B"), out.data_ptr(), _ld(out, "out"), _stream())
    return out


def conv_out_size(i, k, s, p):
    return (i + 2 * p - k) // s + 1


def im2col(x, KH, KW, stride=(1, 1), padding=(0, 0), out=None):
    _need(x, "input")
    if x.dim() != 4 or not x.is_contiguous():
        raise ValueError("im2col: input must be contiguous NCHW")
    Bn, C, H, W = x.shape
    OH = conv_out_size(H, KH, stride[0], padding[0])
    OW = conv_out_size(W, KW, stride[1], padding[1])
    if OH <= 0 or OW <= 0:
        raise ValueError("im2col: kernel larger than padded input")
    shape = (C * KH * KW, Bn * OH * OW)
    if out is None:
        out = torch.empty(shape, device=x.device, dtype=torch.float32)
    if tuple(out.shape) != shape or not out.is_contiguous():
        raise ValueError("im2col: bad output buffer")
    L.call("cdx_im2col_f32", x.data_ptr(), out.data_ptr(), Bn, C, H, W, KH, KW,
           stride[0], stride[1], padding[0], padding[1], _stream())
    return out


def conv2d_forward(x, w, bias=None, stride=(1, 1), padding=(0, 0),
                   precision=L.PREC_FP32, workspace=None, out=None):
    _need(x, "input")
    _need(w, "weight")
    if x.dim() != 4 or w.dim() != 4 or not x.is_contiguous() or not w.is_contiguous():
        raise ValueError("conv2d: input / weight must be contiguous NCHW / OIHW")
    Bn, C, H, W = x.shape
    OC, C2, KH, KW = w.shape
    if C != C2:
        raise ValueError("conv2d: channel mismatch")
    OH = conv_out_size(H, KH, stride[0], padding[0])
    OW = conv_out_size(W, KW, stride[1], padding[1])
    if OH <= 0 or OW <= 0:
        raise ValueError("conv2d: kernel larger than padded input")
    if bias is not None:
        _need(bias, "bias")
        if bias.numel() != OC or not bias.is_contiguous():
            raise ValueError("conv2d: bias must have out_channels elements")
    if out is None:
        out = torch.empty((Bn, OC, OH, OW), device=x.device, dtype=torch.float32)
    ws_ptr, ws_bytes = None, 0
    if workspace is not None:
        ws_ptr, ws_bytes = workspace.data_ptr(), workspace.numel() * workspace.element_size()
    L.call("cdx_conv2d_forward_f32", x.data_ptr(), w.data_ptr(),
           None if bias is None else bias.data_ptr(), out.data_ptr(), Bn, C, OC, H, W, KH, KW,
           stride[0], stride[1], padding[0], padding[1], precision, ws_ptr, ws_bytes, _stream())
    return out


def conv2d_workspace_bytes(x_shape, w_shape, stride=(1, 1), padding=(0, 0)) -> int:
    Bn, C, H, W = x_shape
    _, _, KH, KW = w_shape
    return int(L.lib().cdx_conv2d_forward_workspace_size(
        Bn, C, H, W, KH, KW, stride[0], stride[1], padding[0], padding[1]))


def sum_reduce_rows(x, out=None):
    _need(x, "input")
    if x.dim() != 2 or not x.is_contiguous():
        raise ValueError("sum_reduce_rows: input must be contiguous 2-D")
    rows, cols = x.shape
    if out is None:
        out = torch.empty((cols,), device=x.device, dtype=torch.float32)
    L.call("cdx_sum_reduce_rows_f32", x.data_ptr(), out.data_ptr(), rows, cols, None, 0, _stream())
    return out


def broadcast_add_row(m, row, out=None):
    _need(m, "matrix")
    _need(row, "row")
    if m.dim() != 2 or not m.is_contiguous() or row.numel() != m.shape[1]:
        raise ValueError("broadcast_add: shape mismatch")
    if out is None:
        out = torch.empty_like(m)
    L.call("cdx_broadcast_add_row_f32", m.data_ptr(), row.contiguous().data_ptr(),
           out.data_ptr(), m.shape[0], m.shape[1], _stream())
    return out


def activation(x, act, out=None):
    _need(x, "input")
    if not x.is_contiguous():
        raise ValueError("activation: input must be contiguous")
    if out is None:
        out = torch.empty_like(x)
    L.call("cdx_activation_forward_f32", x.data_ptr(), out.data_ptr(), x.numel(), act, _stream())
    return out


def activation_backward(grad_out, x, act, out=None):
    _need(grad_out, "grad_output")
    _need(x, "input")
    if grad_out.shape != x.shape or not (x.is_contiguous() and grad_out.is_contiguous()):
        raise ValueError("activation_backward: shape mismatch or non-contiguous")
    if out is None:
        out = torch.empty_like(x)
    L.call("cdx_activation_backward_f32", grad_out.data_ptr(), x.data_ptr(), out.data_ptr(),
           x.numel(), act, _stream())
    return out
