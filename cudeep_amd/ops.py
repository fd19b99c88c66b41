"""Thin tensor-level wrappers over the C-ABI, for callers that hold
PyTorch-ROCm device tensors (tests, bench, the host layer).  PyTorch only
supplies device memory and the current stream; all arithmetic happens in
libcudeep_amd.so.  Every wrapper validates shapes / dtypes / devices on the
host before any launch, so a bad call raises instead of faulting.
"""
from __future__ import annotations

import torch

import ctypes

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


def _scratch(workspace, nbytes, device):
    """(pointer, bytes, keep-alive) of a call's scratch: the caller's
    `workspace`, else a block of torch's stream-ordered caching allocator
    sized by the library's query (no block when the call needs none; a block
    freed here is reused only by work queued after this call on the same
    stream).  Passing scratch in keeps the library off its own
    stream-ordered pool, whose allocate / free pair costs ~5 us between the
    kernels of back-to-back calls."""
    if workspace is not None:
        return workspace.data_ptr(), workspace.numel() * workspace.element_size(), workspace
    n = int(nbytes())
    if n <= 0:
        return None, 0, None
    t = torch.empty(n, dtype=torch.uint8, device=device)
    return t.data_ptr(), n, t


def gemm(A: torch.Tensor, B: torch.Tensor, *, precision: int = L.PREC_FP32,
         transA: bool = False, transB: bool = False, bias: torch.Tensor | None = None,
         bias_mode: int = L.BIAS_NONE, epilogue: int = L.EPI_NONE,
         out: torch.Tensor | None = None,
         workspace: torch.Tensor | None = None, aux: torch.Tensor | None = None,
         colsum: torch.Tensor | None = None) -> torch.Tensor:
    """C = epi(op(A) @ op(B) + bias).  A, B are row-major storage; transA /
    transB select the transpose, so x @ W.T is gemm(x, W, transB=True).
    `workspace` (at least gemm_workspace_bytes(...) bytes) makes the call
    allocation-free (cdx_gemm_ex_ws).  Fusions (cdx_gemm_fused): with an
    EPI_BWD_* epilogue, C = (op(A) @ op(B)) * act'(aux) (aux [M, N]); with
    `colsum` (a float32 [M] tensor), colsum[m] = sum_k op(A)[m, k] in the
    same launch (size the workspace with colsum=True)."""
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
    if workspace is not None:
        _need(workspace, "workspace")
    ws_ptr, ws_bytes, _keep = _scratch(
        workspace, lambda: gemm_workspace_bytes(M, N, K, precision=precision, transA=transA,
                                                transB=transB, colsum=colsum is not None),
        A.device)
    if aux is None and colsum is None:
        L.call("cdx_gemm_ex_ws", precision, int(transA), int(transB), M, N, K,
               A.data_ptr(), _ld(A, "A"), B.data_ptr(), _ld(B, "B"),
               out.data_ptr(), _ld(out, "out"), bptr, bias_mode, epilogue, ws_ptr, ws_bytes,
               _stream())
        return out
    aux_ptr, ldaux = None, 0
    if aux is not None:
        _need(aux, "aux")
        if tuple(aux.shape) != (M, N):
            raise ValueError("aux must be [M, N]")
        aux_ptr, ldaux = aux.data_ptr(), _ld(aux, "aux")
    cs_ptr = None
    if colsum is not None:
        _need(colsum, "colsum")
        if colsum.numel() != M or not colsum.is_contiguous():
            raise ValueError("colsum must be a contiguous [M] tensor")
        cs_ptr = colsum.data_ptr()
    L.call("cdx_gemm_fused", precision, int(transA), int(transB), M, N, K,
           A.data_ptr(), _ld(A, "A"), B.data_ptr(), _ld(B, "B"),
           out.data_ptr(), _ld(out, "out"), bptr, bias_mode, epilogue, aux_ptr, ldaux, cs_ptr,
           ws_ptr, ws_bytes, _stream())
    return out


def gemm_workspace_bytes(M: int, N: int, K: int, *, precision: int = L.PREC_FP32,
                         transA: bool = False, transB: bool = False,
                         colsum: bool = False) -> int:
    """Scratch bytes gemm(..., workspace=) needs for op(A) [M, K] @ op(B) [K, N]
    (with colsum=True: for a call that also forms the row sums of op(A))."""
    if colsum:
        return int(L.lib().cdx_gemm_fused_workspace_size(precision, int(transA), int(transB),
                                                         M, N, K, 1))
    return int(L.lib().cdx_gemm_workspace_size(precision, int(transA), int(transB), M, N, K))


def gemm16(A: torch.Tensor, B: torch.Tensor, *, transA: bool = False, transB: bool = False,
           bias: torch.Tensor | None = None, bias_mode: int = L.BIAS_NONE,
           epilogue: int = L.EPI_NONE, out: torch.Tensor | None = None) -> torch.Tensor:
    """C = epi(op(A) @ op(B) + bias) for float16 or bfloat16 A, B (both the
    same type), fp32 accumulation and fp32 C (cdx_gemm16_ex)."""
    if not isinstance(A, torch.Tensor) or A.dtype not in (torch.float16, torch.bfloat16):
        raise TypeError("A must be a float16 or bfloat16 tensor")
    _need(A, "A", A.dtype)
    _need(B, "B", A.dtype)
    dt = L.DTYPE_F16 if A.dtype == torch.float16 else L.DTYPE_BF16
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
    L.call("cdx_gemm16_ex", dt, int(transA), int(transB), M, N, K,
           A.data_ptr(), _ld(A, "A"), B.data_ptr(), _ld(B, "B"),
           out.data_ptr(), _ld(out, "out"), bptr, bias_mode, epilogue, _stream())
    return out


def hgemm(A, B, out=None):
    """C = A @ B for contiguous float16 A, B, fp32 C (cdx_hgemm_f16)."""
    _need(A, "A", torch.float16)
    _need(B, "B", torch.float16)
    if A.dim() != 2 or B.dim() != 2 or A.shape[1] != B.shape[0]:
        raise ValueError("hgemm: shape mismatch")
    if not (A.is_contiguous() and B.is_contiguous()):
        raise ValueError("hgemm: operands must be contiguous")
    M, K = A.shape
    N = B.shape[1]
    if out is None:
        out = torch.empty((M, N), device=A.device, dtype=torch.float32)
    _need(out, "out")
    L.call("cdx_hgemm_f16", A.data_ptr(), B.data_ptr(), out.data_ptr(), M, N, K, _stream())
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
    ws_ptr, ws_bytes, _keep = _scratch(
        workspace, lambda: conv2d_workspace_bytes(x.shape, w.shape, stride, padding), x.device)
    L.call("cdx_conv2d_forward_f32", x.data_ptr(), w.data_ptr(),
           None if bias is None else bias.data_ptr(), out.data_ptr(), Bn, C, OC, H, W, KH, KW,
           stride[0], stride[1], padding[0], padding[1], precision, ws_ptr, ws_bytes, _stream())
    return out


def conv2d_implicit(x, w, bias=None, stride=(1, 1), padding=(0, 0), out=None):
    """NCHW convolution as an implicit GEMM, no column buffer
    (cdx_conv2d_forward_implicit_f32; FP32 products)."""
    _need(x, "input")
    _need(w, "weight")
    if x.dim() != 4 or w.dim() != 4 or not x.is_contiguous() or not w.is_contiguous():
        raise ValueError("conv2d_implicit: input / weight must be contiguous NCHW / OIHW")
    Bn, C, H, W = x.shape
    OC, C2, KH, KW = w.shape
    if C != C2:
        raise ValueError("conv2d_implicit: channel mismatch")
    OH = conv_out_size(H, KH, stride[0], padding[0])
    OW = conv_out_size(W, KW, stride[1], padding[1])
    if OH <= 0 or OW <= 0:
        raise ValueError("conv2d_implicit: kernel larger than padded input")
    if bias is not None:
        _need(bias, "bias")
        if bias.numel() != OC or not bias.is_contiguous():
            raise ValueError("conv2d_implicit: bias must have out_channels elements")
    if out is None:
        out = torch.empty((Bn, OC, OH, OW), device=x.device, dtype=torch.float32)
    L.call("cdx_conv2d_forward_implicit_f32", x.data_ptr(), w.data_ptr(),
           None if bias is None else bias.data_ptr(), out.data_ptr(), Bn, C, OC, H, W, KH, KW,
           stride[0], stride[1], padding[0], padding[1], _stream())
    return out


def conv2d_winograd(x, w, bias=None, padding=(0, 0), precision=L.PREC_FP32, workspace=None,
                    out=None):
    """3x3 stride-1 NCHW convolution by Winograd F(4x4, 3x3)
    (cdx_conv2d_forward_winograd_f32)."""
    _need(x, "input")
    _need(w, "weight")
    if x.dim() != 4 or w.dim() != 4 or not x.is_contiguous() or not w.is_contiguous():
        raise ValueError("conv2d_winograd: input / weight must be contiguous NCHW / OIHW")
    Bn, C, H, W = x.shape
    OC, C2, KH, KW = w.shape
    if C != C2 or KH != 3 or KW != 3:
        raise ValueError("conv2d_winograd: needs a 3x3 kernel and matching channels")
    OH, OW = H + 2 * padding[0] - 2, W + 2 * padding[1] - 2
    if OH <= 0 or OW <= 0:
        raise ValueError("conv2d_winograd: kernel larger than padded input")
    if bias is not None:
        _need(bias, "bias")
        if bias.numel() != OC or not bias.is_contiguous():
            raise ValueError("conv2d_winograd: bias must have out_channels elements")
    if out is None:
        out = torch.empty((Bn, OC, OH, OW), device=x.device, dtype=torch.float32)
    ws_ptr, ws_bytes, _keep = _scratch(
        workspace, lambda: conv2d_winograd_workspace_bytes(x.shape, OC, padding), x.device)
    L.call("cdx_conv2d_forward_winograd_f32", x.data_ptr(), w.data_ptr(),
           None if bias is None else bias.data_ptr(), out.data_ptr(), Bn, C, OC, H, W,
           padding[0], padding[1], precision, ws_ptr, ws_bytes, _stream())
    return out


def conv2d_winograd_workspace_bytes(x_shape, out_channels, padding=(0, 0)) -> int:
    Bn, C, H, W = x_shape
    return int(L.lib().cdx_conv2d_winograd_workspace_size(Bn, C, out_channels, H, W,
                                                          padding[0], padding[1]))


def conv2d_workspace_bytes(x_shape, w_shape, stride=(1, 1), padding=(0, 0)) -> int:
    Bn, C, H, W = x_shape
    _, _, KH, KW = w_shape
    return int(L.lib().cdx_conv2d_forward_workspace_size(
        Bn, C, H, W, KH, KW, stride[0], stride[1], padding[0], padding[1]))


def sum_reduce_rows(x, out=None, workspace=None):
    """Column sums of a contiguous 2-D tensor; `workspace` (at least
    sum_reduce_rows_workspace_bytes(rows, cols)) makes the call allocation-free."""
    _need(x, "input")
    if x.dim() != 2 or not x.is_contiguous():
        raise ValueError("sum_reduce_rows: input must be contiguous 2-D")
    rows, cols = x.shape
    if out is None:
        out = torch.empty((cols,), device=x.device, dtype=torch.float32)
    if workspace is not None:
        _need(workspace, "workspace")
    ws_ptr, ws_bytes, _keep = _scratch(
        workspace, lambda: sum_reduce_rows_workspace_bytes(rows, cols), x.device)
    L.call("cdx_sum_reduce_rows_f32", x.data_ptr(), out.data_ptr(), rows, cols, ws_ptr, ws_bytes,
           _stream())
    return out


def sum_reduce_rows_workspace_bytes(rows: int, cols: int) -> int:
    return int(L.lib().cdx_sum_reduce_rows_workspace_size(rows, cols))


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


def activation(x, act, out=None, alpha=0.01):
    """act(x) elementwise; act is EPI_RELU / _GELU / _SILU / _SIGMOID, ACT_TANH or
    ACT_LEAKY_RELU (negative slope alpha)."""
    _need(x, "input")
    if not x.is_contiguous():
        raise ValueError("activation: input must be contiguous")
    if out is None:
        out = torch.empty_like(x)
    L.call("cdx_activation_forward_f32", x.data_ptr(), out.data_ptr(), x.numel(), act, alpha,
           _stream())
    return out


def activation_backward(grad_out, x, act, out=None, alpha=0.01):
    _need(grad_out, "grad_output")
    _need(x, "input")
    if grad_out.shape != x.shape or not (x.is_contiguous() and grad_out.is_contiguous()):
        raise ValueError("activation_backward: shape mismatch or non-contiguous")
    if out is None:
        out = torch.empty_like(x)
    L.call("cdx_activation_backward_f32", grad_out.data_ptr(), x.data_ptr(), out.data_ptr(),
           x.numel(), act, alpha, _stream())
    return out


def col2im(col, x_shape, KH, KW, stride=(1, 1), padding=(0, 0), out=None):
    _need(col, "col")
    Bn, C, H, W = x_shape
    OH = conv_out_size(H, KH, stride[0], padding[0])
    OW = conv_out_size(W, KW, stride[1], padding[1])
    if tuple(col.shape) != (C * KH * KW, Bn * OH * OW) or not col.is_contiguous():
        raise ValueError("col2im: col has the wrong shape")
    if out is None:
        out = torch.empty(tuple(x_shape), device=col.device, dtype=torch.float32)
    L.call("cdx_col2im_f32", col.data_ptr(), out.data_ptr(), Bn, C, H, W, KH, KW,
           stride[0], stride[1], padding[0], padding[1], _stream())
    return out


def _conv_geom(x_shape, w_shape, stride, padding):
    Bn, C, H, W = x_shape
    OC, C2, KH, KW = w_shape
    if C != C2:
        raise ValueError("conv2d: channel mismatch")
    OH = conv_out_size(H, KH, stride[0], padding[0])
    OW = conv_out_size(W, KW, stride[1], padding[1])
    if OH <= 0 or OW <= 0:
        raise ValueError("conv2d: kernel larger than padded input")
    return Bn, C, H, W, OC, KH, KW, OH, OW


def conv2d_backward_data(grad_out, w, x_shape, stride=(1, 1), padding=(0, 0),
                         precision=L.PREC_FP32, out=None, workspace=None):
    """`workspace` (at least conv2d_backward_data_workspace_bytes(...) bytes)
    makes the call allocation-free."""
    _need(grad_out, "grad_output")
    _need(w, "weight")
    Bn, C, H, W, OC, KH, KW, OH, OW = _conv_geom(tuple(x_shape), tuple(w.shape), stride, padding)
    if tuple(grad_out.shape) != (Bn, OC, OH, OW) or not grad_out.is_contiguous() \
            or not w.is_contiguous():
        raise ValueError("conv2d_backward_data: bad grad_output / weight")
    if out is None:
        out = torch.empty((Bn, C, H, W), device=w.device, dtype=torch.float32)
    ws_ptr, ws_bytes, _keep = _scratch(
        workspace, lambda: conv2d_backward_data_workspace_bytes(x_shape, w.shape, stride, padding),
        w.device)
    L.call("cdx_conv2d_backward_data_f32", grad_out.data_ptr(), w.data_ptr(), out.data_ptr(),
           Bn, C, OC, H, W, KH, KW, stride[0], stride[1], padding[0], padding[1], precision,
           ws_ptr, ws_bytes, _stream())
    return out


def conv2d_backward_data_workspace_bytes(x_shape, w_shape, stride=(1, 1),
                                         padding=(0, 0)) -> int:
    Bn, C, H, W, OC, KH, KW, _, _ = _conv_geom(tuple(x_shape), tuple(w_shape), stride, padding)
    return int(L.lib().cdx_conv2d_backward_data_workspace_size(
        Bn, C, OC, H, W, KH, KW, stride[0], stride[1], padding[0], padding[1]))


def conv2d_backward_data_winograd(grad_out, w, x_shape, padding=(0, 0), precision=L.PREC_FP32,
                                  workspace=None, out=None):
    """grad_input of a 3x3 stride-1 conv by Winograd F(4x4, 3x3) on the
    transposed convolution (cdx_conv2d_backward_data_winograd_f32)."""
    _need(grad_out, "grad_output")
    _need(w, "weight")
    Bn, C, H, W, OC, KH, KW, OH, OW = _conv_geom(tuple(x_shape), tuple(w.shape), (1, 1), padding)
    if (KH, KW) != (3, 3) or padding[0] > 2 or padding[1] > 2:
        raise ValueError("conv2d_backward_data_winograd: needs a 3x3 kernel and padding <= 2")
    if tuple(grad_out.shape) != (Bn, OC, OH, OW) or not grad_out.is_contiguous() \
            or not w.is_contiguous():
        raise ValueError("conv2d_backward_data_winograd: bad grad_output / weight")
    if out is None:
        out = torch.empty((Bn, C, H, W), device=w.device, dtype=torch.float32)
    ws_ptr, ws_bytes, _keep = _scratch(
        workspace, lambda: conv2d_backward_data_winograd_workspace_bytes(x_shape, OC, padding),
        w.device)
    L.call("cdx_conv2d_backward_data_winograd_f32", grad_out.data_ptr(), w.data_ptr(),
           out.data_ptr(), Bn, C, OC, H, W, padding[0], padding[1], precision,
           ws_ptr, ws_bytes, _stream())
    return out


def conv2d_backward_data_winograd_workspace_bytes(x_shape, out_channels, padding=(0, 0)) -> int:
    Bn, C, H, W = x_shape
    return int(L.lib().cdx_conv2d_backward_data_winograd_workspace_size(
        Bn, C, out_channels, H, W, padding[0], padding[1]))


def conv2d_backward_weight(grad_out, x, w_shape, stride=(1, 1), padding=(0, 0),
                           precision=L.PREC_FP32, out=None, workspace=None):
    """`workspace` (at least conv2d_backward_weight_workspace_bytes(...) bytes)
    makes the call allocation-free."""
    _need(grad_out, "grad_output")
    _need(x, "input")
    Bn, C, H, W, OC, KH, KW, OH, OW = _conv_geom(tuple(x.shape), tuple(w_shape), stride, padding)
    if tuple(grad_out.shape) != (Bn, OC, OH, OW) or not grad_out.is_contiguous() \
            or not x.is_contiguous():
        raise ValueError("conv2d_backward_weight: bad grad_output / input")
    if out is None:
        out = torch.empty(tuple(w_shape), device=x.device, dtype=torch.float32)
    ws_ptr, ws_bytes, _keep = _scratch(
        workspace, lambda: conv2d_backward_weight_workspace_bytes(x.shape, w_shape, stride, padding),
        x.device)
    L.call("cdx_conv2d_backward_weight_f32", grad_out.data_ptr(), x.data_ptr(), out.data_ptr(),
           Bn, C, OC, H, W, KH, KW, stride[0], stride[1], padding[0], padding[1], precision,
           ws_ptr, ws_bytes, _stream())
    return out


def conv2d_backward_weight_workspace_bytes(x_shape, w_shape, stride=(1, 1),
                                           padding=(0, 0)) -> int:
    Bn, C, H, W, OC, KH, KW, _, _ = _conv_geom(tuple(x_shape), tuple(w_shape), stride, padding)
    return int(L.lib().cdx_conv2d_backward_weight_workspace_size(
        Bn, C, OC, H, W, KH, KW, stride[0], stride[1], padding[0], padding[1]))


def conv2d_backward_bias(grad_out, out=None):
    _need(grad_out, "grad_output")
    if grad_out.dim() != 4 or not grad_out.is_contiguous():
        raise ValueError("conv2d_backward_bias: grad_output must be contiguous NCHW")
    Bn, OC, OH, OW = grad_out.shape
    if out is None:
        out = torch.empty((OC,), device=grad_out.device, dtype=torch.float32)
    L.call("cdx_conv2d_backward_bias_f32", grad_out.data_ptr(), out.data_ptr(), Bn, OC, OH * OW,
           _stream())
    return out


def _dtype_code(t):
    if t.dtype == torch.float32:
        return L.DTYPE_F32
    if t.dtype == torch.float64:
        return L.DTYPE_F64
    raise TypeError("only float32 / float64 tensors")


def strided_copy(view):
    """Contiguous copy of a strided device view (cdx_strided_copy)."""
    if not view.is_cuda:
        raise ValueError("device tensor expected")
    code = _dtype_code(view)
    out = torch.empty(tuple(view.shape), device=view.device, dtype=view.dtype)
    nd = view.dim()
    shape = (ctypes.c_int64 * max(nd, 1))(*view.shape)
    strides = (ctypes.c_int64 * max(nd, 1))(*view.stride())
    L.call("cdx_strided_copy", view.data_ptr(), out.data_ptr(), nd, shape, strides, code, _stream())
    return out


def fill(t, value):
    L.call("cdx_fill", t.data_ptr(), t.numel(), float(value), _dtype_code(t), _stream())
    return t


def binary(op, a, b, out=None):
    if a.shape != b.shape or a.dtype != b.dtype or not (a.is_contiguous() and b.is_contiguous()):
        raise ValueError("binary: operands must match and be contiguous")
    if out is None:
        out = torch.empty_like(a)
    L.call("cdx_binary", op, _dtype_code(a), a.data_ptr(), b.data_ptr(), out.data_ptr(),
           a.numel(), _stream())
    return out


def randn(shape, dtype=torch.float32, seed=0, offset=0):
    out = torch.empty(tuple(shape), device="cuda", dtype=dtype)
    L.call("cdx_randn", out.data_ptr(), out.numel(), _dtype_code(out), int(seed), int(offset),
           _stream())
    return out


def total_sum(x):
    if not x.is_contiguous():
        raise ValueError("sum: input must be contiguous")
    out = torch.empty((1,), device=x.device, dtype=x.dtype)
    L.call("cdx_sum", x.data_ptr(), out.data_ptr(), x.numel(), _dtype_code(x), None, 0, _stream())
    return out
