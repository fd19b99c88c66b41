"""CPU oracle for the dense-contraction path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg import this package, and only as the checker (or the
timed CPU baseline).  The product package ``cudeep_amd`` never imports it and
has no CPU fallback.

The arithmetic lives in ``oracle/oracle.c`` (built by ``oracle/Makefile``
into ``liboracle.so``); each C routine cites the reference file:line it
restates.  This module adds numpy wrappers and the error metrics used by the
parity gates:

* ``sgemm_seqfma``   -- reference SGEMM numerics, bit-exact
  (``src/kernels/matmul_kernel.cu:499-520``, ``:632-647``).
* ``dgemm``          -- fp64 yardstick.
* ``gemm_tf32emu``   -- reference TF32 tensor-core GEMM, emulated
  (``matmul_kernel.cu:179-214``; ``ptx_intrinsics.cuh:316-335``, ``:639-649``).
* ``im2col`` / ``transpose_bias`` / ``conv2d_direct64``
  (``src/kernels/conv_kernel.cu:32-65``, ``:74-93``, ``:113-159``).
* ``col2im`` and the backward-conv routes (``conv_kernel.cu:344-545``).
* ``colsum`` (``src/kernels/unary_kernel.cu:204-238``).
* ``gelu`` / ``gelu_grad`` / ``relu`` / ``relu_grad``
  (``src/kernels/activation_kernel.cu:19-52``, ``:256-319``).

The reference itself cannot be built here (CUDA sources with inline PTX, no
CUDA toolchain), so there is no ``oracle/_ref``; the restatements are pinned
by the reference's own known-answer tests and by closed forms (see
``tests/test_oracle.py``).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

_i64 = ctypes.c_int64
_int = ctypes.c_int
_vp = ctypes.c_void_p


def build(force: bool = False) -> str:
    """Compile liboracle.so from oracle.c with the committed Makefile."""
    src = os.path.join(_HERE, "oracle.c")
    if force or not os.path.exists(_LIB_PATH) or \
            os.path.getmtime(_LIB_PATH) < os.path.getmtime(src):
        subprocess.run(["make", "-s", "-C", _HERE, "-B" if force else "all"],
                       check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.orc_sgemm_seqfma_rows.argtypes = [_vp, _vp, _vp, _i64, _i64, _i64,
                                            _int, _int, _i64, _i64, _i64, _i64]
        L.orc_dgemm_rows_f32in.argtypes = [_vp, _vp, _vp, _i64, _i64, _i64,
                                           _int, _int, _i64, _i64, _i64, _i64]
        L.orc_dgemm_f64.argtypes = [_vp, _vp, _vp, _i64, _i64, _i64,
                                    _int, _int, _i64, _i64]
        L.orc_gemm_tf32emu.argtypes = [_vp, _vp, _vp, _i64, _i64, _i64, _int]
        L.orc_gemm_tf32emu_rows.argtypes = [_vp, _vp, _vp, _i64, _i64, _i64, _int,
                                            _i64, _i64]
        L.orc_tf32_round.argtypes = [ctypes.c_float, _int]
        L.orc_tf32_round.restype = ctypes.c_float
        L.orc_im2col.argtypes = [_vp, _vp] + [_i64] * 10
        L.orc_transpose_bias.argtypes = [_vp, _vp, _vp, _i64, _i64, _i64]
        L.orc_conv2d_direct64.argtypes = [_vp, _vp, _vp, _vp] + [_i64] * 11
        L.orc_conv2d_implicit.argtypes = [_vp, _vp, _vp, _vp] + [_i64] * 11
        L.orc_colsum.argtypes = [_vp, _vp, _i64, _i64]
        L.orc_col2im.argtypes = [_vp, _vp] + [_i64] * 10
        L.orc_col2im64.argtypes = [_vp, _vp] + [_i64] * 10
        L.orc_winograd_f43.argtypes = [_vp, _vp, _vp, _vp] + [_i64] * 7 + [_int]
        L.orc_winograd_f43_64.argtypes = [_vp, _vp, _vp, _vp] + [_i64] * 7 + [_int]
        L.orc_gelu_vec.argtypes = [_vp, _vp, _i64]
        L.orc_gelu_grad_vec.argtypes = [_vp, _vp, _i64]
        L.orc_num_threads.restype = _int
        L.orc_set_num_threads.argtypes = [_int]
        _lib = L
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def _c32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def num_threads() -> int:
    return lib().orc_num_threads()


def set_num_threads(n: int) -> None:
    lib().orc_set_num_threads(int(n))


def _op_shape(X, trans):
    r, c = X.shape
    return (c, r) if trans else (r, c)


def sgemm_seqfma(A, B, transA=False, transB=False, rows=None):
    """op(A) @ op(B) with the reference SGEMM's per-output sequential fp32
    FMA chain over ascending k (bit-exact restatement).  ``rows=(r0, r1)``
    computes only output rows [r0, r1)."""
    A, B = _c32(A), _c32(B)
    M, K = _op_shape(A, transA)
    K2, N = _op_shape(B, transB)
    assert K == K2, (A.shape, B.shape, transA, transB)
    r0, r1 = (0, M) if rows is None else rows
    C = np.empty((r1 - r0, N), np.float32)
    lib().orc_sgemm_seqfma_rows(_p(A), _p(B), _p(C), M, N, K, int(transA),
                                int(transB), A.shape[1], B.shape[1], r0, r1)
    return C


def dgemm(A, B, transA=False, transB=False, rows=None):
    """fp64 op(A) @ op(B) of fp32 (or fp64) operands; rows as above."""
    if A.dtype == np.float64 and B.dtype == np.float64 and rows is None:
        A, B = np.ascontiguousarray(A), np.ascontiguousarray(B)
        M, K = _op_shape(A, transA)
        _, N = _op_shape(B, transB)
        C = np.empty((M, N), np.float64)
        lib().orc_dgemm_f64(_p(A), _p(B), _p(C), M, N, K, int(transA),
                            int(transB), A.shape[1], B.shape[1])
        return C
    A, B = _c32(A), _c32(B)
    M, K = _op_shape(A, transA)
    K2, N = _op_shape(B, transB)
    assert K == K2
    r0, r1 = (0, M) if rows is None else rows
    C = np.empty((r1 - r0, N), np.float64)
    lib().orc_dgemm_rows_f32in(_p(A), _p(B), _p(C), M, N, K, int(transA),
                               int(transB), A.shape[1], B.shape[1], r0, r1)
    return C


def tf32_round(x, mode: str = "rz"):
    """Round fp32 values to TF32 (10-bit mantissa); mode 'rz' or 'rne'."""
    x = _c32(x)
    u = x.view(np.uint32).copy()
    finite = (u & 0x7F800000) != 0x7F800000
    if mode == "rne":
        lsb = (u >> 13) & 1
        u = np.where(finite, u + np.uint32(0x0FFF) + lsb, u).astype(np.uint32)
    elif mode != "rz":
        raise ValueError(mode)
    u = np.where(finite, u & np.uint32(0xFFFFE000), u).astype(np.uint32)
    return u.view(np.float32)


def gemm_tf32emu(A, B, mode: str = "rz", rows=None):
    """Emulated reference TF32 tensor-core GEMM (ideal MMA, 8-term k chunks).
    ``rows=(r0, r1)`` computes only output rows [r0, r1)."""
    A, B = _c32(A), _c32(B)
    M, K = A.shape
    _, N = B.shape
    r0, r1 = (0, M) if rows is None else rows
    C = np.empty((r1 - r0, N), np.float32)
    lib().orc_gemm_tf32emu_rows(_p(A), _p(B), _p(C), M, N, K,
                                {"rz": 0, "rne": 1}[mode], r0, r1)
    return C


def conv_out_size(i, k, s, p):
    """conv_kernel.cu:235-236."""
    return (i + 2 * p - k) // s + 1


def im2col(x, KH, KW, SH=1, SW=1, PH=0, PW=0):
    """Bit-exact im2col, layout [IC*KH*KW, B*OH*OW] (conv_kernel.cu:32-65)."""
    x = _c32(x)
    Bn, IC, IH, IW = x.shape
    OH, OW = conv_out_size(IH, KH, SH, PH), conv_out_size(IW, KW, SW, PW)
    col = np.empty((IC * KH * KW, Bn * OH * OW), np.float32)
    lib().orc_im2col(_p(x), _p(col), Bn, IC, IH, IW, KH, KW, SH, SW, PH, PW)
    return col


def transpose_bias(src, OC, batch, spatial, bias=None):
    """[OC, B*S] -> [B, OC, S] (+bias[oc]) (conv_kernel.cu:74-93)."""
    src = _c32(src)
    dst = np.empty((batch, OC, spatial), np.float32)
    b = None if bias is None else _c32(bias)
    lib().orc_transpose_bias(_p(src), _p(dst), None if b is None else _p(b),
                             OC, batch, spatial)
    return dst


def conv2d_direct64(x, w, bias=None, stride=(1, 1), padding=(0, 0)):
    """fp64 direct cross-correlation (conv_kernel.cu:113-159)."""
    x, w = _c32(x), _c32(w)
    Bn, IC, IH, IW = x.shape
    OC, IC2, KH, KW = w.shape
    assert IC == IC2
    SH, SW = stride
    PH, PW = padding
    OH, OW = conv_out_size(IH, KH, SH, PH), conv_out_size(IW, KW, SW, PW)
    out = np.empty((Bn, OC, OH, OW), np.float64)
    b = None if bias is None else _c32(bias)
    lib().orc_conv2d_direct64(_p(x), _p(w), None if b is None else _p(b), _p(out),
                              Bn, IC, OC, IH, IW, KH, KW, SH, SW, PH, PW)
    return out


def conv2d_ref_implicit(x, w, bias=None, stride=(1, 1), padding=(0, 0), batches=None):
    """The reference's implicit-GEMM route restated on the CPU
    (implicit_gemm_conv2d_kernel, conv_kernel.cu:172-215): per output one fp32
    FMA chain starting from the bias, taps ic -> kh -> kw, padding taps
    skipped.  Its error vs fp64 is the yardstick for layers the reference
    sends to that kernel.  `batches` restricts it to those images."""
    x, w = _c32(x), _c32(w)
    if batches is not None:
        x = np.ascontiguousarray(x[list(batches)])
    Bn, IC, IH, IW = x.shape
    OC, IC2, KH, KW = w.shape
    assert IC == IC2
    SH, SW = stride
    PH, PW = padding
    OH, OW = conv_out_size(IH, KH, SH, PH), conv_out_size(IW, KW, SW, PW)
    out = np.empty((Bn, OC, OH, OW), np.float32)
    b = None if bias is None else _c32(bias)
    lib().orc_conv2d_implicit(_p(x), _p(w), None if b is None else _p(b), _p(out),
                              Bn, IC, OC, IH, IW, KH, KW, SH, SW, PH, PW)
    return out


def conv2d_ref_im2col(x, w, bias=None, stride=(1, 1), padding=(0, 0)):
    """The reference's explicit im2col route restated on the CPU
    (conv_kernel.cu:279-334): im2col -> seq-FMA SGEMM W[OC,Kcol]·col ->
    transpose + bias.  Its error vs fp64 is the conv parity yardstick."""
    x, w = _c32(x), _c32(w)
    Bn = x.shape[0]
    OC, IC, KH, KW = w.shape
    col = im2col(x, KH, KW, stride[0], stride[1], padding[0], padding[1])
    flat = sgemm_seqfma(w.reshape(OC, -1), col)
    OH = conv_out_size(x.shape[2], KH, stride[0], padding[0])
    OW = conv_out_size(x.shape[3], KW, stride[1], padding[1])
    out = transpose_bias(flat, OC, Bn, OH * OW, bias)
    return out.reshape(Bn, OC, OH, OW)


def conv2d_winograd(x, w, bias=None, padding=(0, 0), double=False, tf32=None):
    """The reference's Winograd F(4x4, 3x3) route for 3x3 stride-1 convolution
    (conv_kernel.cu:557-789) restated on the CPU: weight / input transforms,
    36 seq-FMA GEMMs over input channels, output transform + bias, in fp32
    (``double=True``: the same algorithm in fp64, equal to direct convolution
    up to rounding).  ``tf32="rz" | "rne"`` rounds the GEMM operands to TF32
    first, as the reference's default TF32 GEMM sees them."""
    x, w = _c32(x), _c32(w)
    Bn, IC, IH, IW = x.shape
    OC, IC2, KH, KW = w.shape
    assert IC == IC2 and KH == 3 and KW == 3
    PH, PW = padding
    OH, OW = IH + 2 * PH - 2, IW + 2 * PW - 2
    out = np.empty((Bn, OC, OH, OW), np.float64 if double else np.float32)
    b = None if bias is None else _c32(bias)
    f = lib().orc_winograd_f43_64 if double else lib().orc_winograd_f43
    mode = {None: 0, "rz": 1, "rne": 2}[tf32]
    f(_p(x), _p(w), None if b is None else _p(b), _p(out), Bn, IC, OC, IH, IW, PH, PW, mode)
    return out


def col2im(col, x_shape, KH, KW, SH=1, SW=1, PH=0, PW=0):
    """fp32 col2im gather, kh then kw ascending (conv_kernel.cu:344-380).
    A float64 ``col`` runs the same gather in double."""
    Bn, IC, IH, IW = x_shape
    if np.asarray(col).dtype == np.float64:
        col = np.ascontiguousarray(col, dtype=np.float64)
        out = np.empty(x_shape, np.float64)
        lib().orc_col2im64(_p(col), _p(out), Bn, IC, IH, IW, KH, KW, SH, SW, PH, PW)
        return out
    col = _c32(col)
    out = np.empty(x_shape, np.float32)
    lib().orc_col2im(_p(col), _p(out), Bn, IC, IH, IW, KH, KW, SH, SW, PH, PW)
    return out


def nchw_to_cm(y):
    """[B, C, H, W] -> [C, B*H*W] (conv_kernel.cu:383-399)."""
    Bn, C = y.shape[:2]
    return np.ascontiguousarray(np.asarray(y).reshape(Bn, C, -1).transpose(1, 0, 2).reshape(C, -1))


def conv2d_backward_data_ref(dy, w, x_shape, stride=(1, 1), padding=(0, 0), mode="fp32"):
    """The reference's backward-data route (conv_kernel.cu:417-478):
    grad_col = W^T [Kc, OC] @ dY [OC, B*S] (seq-FMA for fp32, the TF32
    emulation for mode 'rz' / 'rne'), then fp32 col2im."""
    OC = w.shape[0]
    KH, KW = w.shape[2], w.shape[3]
    wt = np.ascontiguousarray(np.asarray(w, np.float32).reshape(OC, -1).T)
    go = nchw_to_cm(np.asarray(dy, np.float32))
    if mode == "fp32":
        gcol = sgemm_seqfma(wt, go)
    else:
        gcol = gemm_tf32emu(wt, go, mode)
    return col2im(gcol, x_shape, KH, KW, stride[0], stride[1], padding[0], padding[1])


def conv2d_backward_data64(dy, w, x_shape, stride=(1, 1), padding=(0, 0)):
    """fp64 grad_input: fp64 W^T dY then the fp64 col2im gather."""
    OC = w.shape[0]
    KH, KW = w.shape[2], w.shape[3]
    gcol = np.asarray(w, np.float64).reshape(OC, -1).T @ nchw_to_cm(np.asarray(dy, np.float64))
    return col2im(gcol, x_shape, KH, KW, stride[0], stride[1], padding[0], padding[1])


def flip_filter(w):
    """The stride-1 transposed convolution's filter: wf[ic, oc] = w[oc, ic]
    with both spatial axes reversed."""
    return np.ascontiguousarray(np.asarray(w, np.float32)[:, :, ::-1, ::-1].transpose(1, 0, 2, 3))


def conv2d_backward_data_winograd(dy, w, x_shape, padding=(0, 0), double=False, tf32=None):
    """grad_input of a 3x3 stride-1 conv as the Winograd forward of grad_out
    with the flipped filter, padded 2 - P (the reference's Winograd route,
    conv_kernel.cu:557-789, applied to the transposed convolution)."""
    PH, PW = padding
    dx = conv2d_winograd(dy, flip_filter(w), None, padding=(2 - PH, 2 - PW), double=double,
                         tf32=tf32)
    assert dx.shape == tuple(x_shape)
    return dx


def conv2d_backward_weight_ref(dy, x, w_shape, stride=(1, 1), padding=(0, 0), mode="fp32"):
    """The reference's backward-weight route (conv_kernel.cu:486-545):
    dW [OC, Kc] = dY [OC, B*S] @ col^T (seq-FMA, or the TF32 emulation)."""
    OC, IC, KH, KW = w_shape
    col = im2col(x, KH, KW, stride[0], stride[1], padding[0], padding[1])
    go = nchw_to_cm(np.asarray(dy, np.float32))
    if mode == "fp32":
        dw = sgemm_seqfma(go, col, transB=True)
    else:
        dw = gemm_tf32emu(go, np.ascontiguousarray(col.T), mode)
    return dw.reshape(w_shape)


def conv2d_backward_weight64(dy, x, w_shape, stride=(1, 1), padding=(0, 0)):
    OC, IC, KH, KW = w_shape
    col = im2col(x, KH, KW, stride[0], stride[1], padding[0], padding[1])
    go = nchw_to_cm(np.asarray(dy, np.float32))
    return dgemm(go, col, transB=True).reshape(w_shape)


def colsum(x):
    """Serial fp32 column sums (unary_kernel.cu:204-238)."""
    x = _c32(x)
    r, c = x.shape
    out = np.empty((c,), np.float32)
    lib().orc_colsum(_p(x), _p(out), r, c)
    return out


def gelu(x):
    x = np.ascontiguousarray(x, dtype=np.float64)
    y = np.empty_like(x)
    lib().orc_gelu_vec(_p(x), _p(y), x.size)
    return y


def gelu_grad(x):
    x = np.ascontiguousarray(x, dtype=np.float64)
    y = np.empty_like(x)
    lib().orc_gelu_grad_vec(_p(x), _p(y), x.size)
    return y


def relu(x):
    x = np.asarray(x, dtype=np.float64)
    return np.where(x > 0, x, 0.0)


def relu_grad(x):
    return (np.asarray(x) > 0).astype(np.float64)


def sigmoid(x):
    """1 / (1 + exp(-x)) in fp64 (reference act_sigmoid,
    src/kernels/activation_kernel.cu:24-31; GEMM epilogue
    src/kernels/matmul_kernel.cu:1541).  Evaluated as exp(min(x,0)) /
    (1 + exp(-|x|)) so neither tail overflows."""
    x = np.asarray(x, dtype=np.float64)
    e = np.exp(-np.abs(x))
    return np.where(x >= 0, 1.0 / (1.0 + e), e / (1.0 + e))


def sigmoid_grad(x):
    """s (1 - s) (reference backward, activation_kernel.cu:268-274)."""
    s = sigmoid(x)
    return s * sigmoid(-np.asarray(x, dtype=np.float64))


def silu(x):
    """x * sigmoid(x) (reference act_silu, activation_kernel.cu:55-62)."""
    x = np.asarray(x, dtype=np.float64)
    return x * sigmoid(x)


def silu_grad(x):
    """s (1 + x (1 - s)) (reference backward, activation_kernel.cu:297-303)."""
    x = np.asarray(x, dtype=np.float64)
    s = sigmoid(x)
    return s * (1.0 + x * sigmoid(-x))


def tanh(x):
    """tanh in fp64 (reference act_tanh, src/kernels/activation_kernel.cu:33-40)."""
    return np.tanh(np.asarray(x, dtype=np.float64))


def tanh_grad(x):
    """1 - tanh(x)^2 (reference backward, activation_kernel.cu:168-171)."""
    t = tanh(x)
    return 1.0 - t * t


def leaky_relu(x, alpha=0.01):
    """x > 0 ? x : alpha * x (reference act_leaky_relu, activation_kernel.cu:63-66),
    alpha rounded to fp32 as the reference passes it."""
    x = np.asarray(x, dtype=np.float64)
    return np.where(x > 0, x, float(np.float32(alpha)) * x)


def leaky_relu_grad(x, alpha=0.01):
    """1 for x > 0, alpha otherwise (reference backward, activation_kernel.cu:190-191)."""
    return np.where(np.asarray(x) > 0, 1.0, float(np.float32(alpha)))


def activation(x, name):
    """Forward activation by name: relu / gelu / silu / sigmoid / tanh / leaky_relu
    (slope 0.01, the reference's default)."""
    return {"relu": relu, "gelu": gelu, "silu": silu, "sigmoid": sigmoid, "tanh": tanh,
            "leaky_relu": leaky_relu}[name](x)


def activation_grad(x, name):
    """d activation / dx at the pre-activation input x."""
    return {"relu": relu_grad, "gelu": gelu_grad, "silu": silu_grad,
            "sigmoid": sigmoid_grad, "tanh": tanh_grad,
            "leaky_relu": leaky_relu_grad}[name](x)


def rel_fro(C, Cref) -> float:
    """Relative Frobenius error ||C - Cref||_F / ||Cref||_F (in fp64)."""
    C = np.asarray(C, dtype=np.float64)
    Cref = np.asarray(Cref, dtype=np.float64)
    num = np.linalg.norm((C - Cref).ravel())
    den = np.linalg.norm(Cref.ravel())
    return float(num / den) if den > 0 else float(num)
