"""Autograd-aware Tensor over the native ``_cudeep_core.Tensor``.

Public surface of the reference's python/cuDeep/tensor.py for the
dense-contraction path: construction from numpy / lists / raw tensors,
factories, shape queries, reshape / transpose, +, -, *, matmul (@), sum,
relu / gelu, broadcast_add, conv2d, backward.  Differences in how the work
is done (same results, fewer passes):

* ``MatMulOp.backward`` computes dA = dY B^T and dB = A^T dY with
  transposed-operand GEMMs instead of materialising transposes
  (reference tensor.py:430-443 copies both).
* ``linear`` runs x W^T + b (and a ReLU / GELU epilogue) as one fused GEMM
  launch; its backward uses the NN / TN GEMMs and the GPU column sum.
* ``Conv2dOp.backward`` computes the bias gradient on the GPU (reference
  tensor.py:718-721 copies grad_output to the host and sums in NumPy).
"""
from __future__ import annotations

from typing import Optional

import numpy as np

from ._core import (
    DType,
    Tensor as _RawTensor,
    activation_backward as _activation_backward,
    broadcast_add as _broadcast_add,
    conv2d_backward_bias as _conv2d_backward_bias,
    conv2d_backward_data as _conv2d_backward_data,
    conv2d_backward_weight as _conv2d_backward_weight,
    conv2d_forward as _conv2d_forward,
    gelu as _gelu,
    linear_forward as _linear_forward,
    matmul_ex as _matmul_ex,
    relu as _relu,
    sum as _sum,
    sum_reduce_rows as _sum_reduce_rows,
)
from .autograd import Function, backward as _backward


class Tensor:
    """GPU tensor with reverse-mode autograd (reference tensor.py:57-307)."""

    __slots__ = ("_data", "grad", "requires_grad", "_grad_fn", "_ctx", "_prev")

    def __init__(self, data, requires_grad=False, dtype=None):
        if isinstance(data, _RawTensor):
            self._data = data
        elif isinstance(data, np.ndarray):
            arr = np.ascontiguousarray(data)
            if dtype is not None:
                arr = arr.astype(np.float64 if dtype == DType.float64 else np.float32, copy=False)
            elif arr.dtype not in (np.float32, np.float64):
                arr = arr.astype(np.float32)
            self._data = _RawTensor.from_numpy(arr)
        elif isinstance(data, (list, tuple, int, float)):
            np_dt = np.float64 if dtype == DType.float64 else np.float32
            self._data = _RawTensor.from_numpy(np.array(data, dtype=np_dt))
        else:
            raise TypeError(f"Cannot create Tensor from {type(data)}")
        self.grad: Optional[Tensor] = None
        self.requires_grad = requires_grad
        self._grad_fn = None
        self._ctx = None
        self._prev: tuple = ()

    @classmethod
    def _wrap(cls, raw: _RawTensor, requires_grad=False) -> "Tensor":
        t = object.__new__(cls)
        t._data = raw
        t.grad = None
        t.requires_grad = requires_grad
        t._grad_fn = None
        t._ctx = None
        t._prev = ()
        return t

    # ---- factories ----
    @staticmethod
    def zeros(shape, dtype=DType.float32, requires_grad=False) -> "Tensor":
        return Tensor._wrap(_RawTensor.zeros(list(shape), dtype), requires_grad)

    @staticmethod
    def ones(shape, dtype=DType.float32, requires_grad=False) -> "Tensor":
        return Tensor._wrap(_RawTensor.ones(list(shape), dtype), requires_grad)

    @staticmethod
    def randn(shape, dtype=DType.float32, requires_grad=False) -> "Tensor":
        return Tensor._wrap(_RawTensor.randn(list(shape), dtype), requires_grad)

    @staticmethod
    def from_numpy(arr, requires_grad=False) -> "Tensor":
        arr = np.ascontiguousarray(arr)
        if arr.dtype not in (np.float32, np.float64):
            arr = arr.astype(np.float32)
        return Tensor._wrap(_RawTensor.from_numpy(arr), requires_grad)

    @staticmethod
    def full(shape, value, dtype=DType.float32, requires_grad=False) -> "Tensor":
        t = Tensor._wrap(_RawTensor(list(shape), dtype), requires_grad)
        t._data.fill_(float(value))
        return t

    # ---- properties ----
    def shape(self):
        return self._data.shape()

    def dtype(self):
        return self._data.dtype()

    def ndim(self):
        return self._data.ndim()

    def numel(self):
        return self._data.numel()

    def is_contiguous(self):
        return self._data.is_contiguous()

    def numpy(self):
        return self._data.numpy()

    def item(self):
        if self._data.numel() != 1:
            raise ValueError("item() only for single-element tensors")
        return self._data.numpy().item()

    def detach(self) -> "Tensor":
        return Tensor._wrap(self._data, requires_grad=False)

    def contiguous(self) -> "Tensor":
        if self._data.is_contiguous():
            return self
        return Tensor._wrap(self._data.contiguous(), self.requires_grad)

    def clone(self) -> "Tensor":
        return Tensor._wrap(self._data.clone(), self.requires_grad)

    # ---- in-place (no autograd) ----
    def fill_(self, value):
        self._data.fill_(float(value))
        return self

    def zero_(self):
        self._data.zero_()
        return self

    # ---- reshape / transpose ----
    def reshape(self, *shape):
        if len(shape) == 1 and isinstance(shape[0], (list, tuple)):
            shape = list(shape[0])
        return ReshapeOp.apply(self, list(shape))

    def transpose(self, dim0, dim1):
        return TransposeOp.apply(self, dim0, dim1)

    def t(self):
        return self.transpose(0, 1)

    # ---- arithmetic ----
    def __add__(self, other):
        if isinstance(other, (int, float)):
            other = Tensor.full(self.shape(), other, self.dtype())
        return AddOp.apply(self, other)

    def __radd__(self, other):
        return self.__add__(other)

    def __sub__(self, other):
        if isinstance(other, (int, float)):
            other = Tensor.full(self.shape(), other, self.dtype())
        return SubOp.apply(self, other)

    def __rsub__(self, other):
        if isinstance(other, (int, float)):
            other = Tensor.full(self.shape(), other, self.dtype())
        return SubOp.apply(other, self)

    def __mul__(self, other):
        if isinstance(other, (int, float)):
            other = Tensor.full(self.shape(), other, self.dtype())
        return MulOp.apply(self, other)

    def __rmul__(self, other):
        return self.__mul__(other)

    def __neg__(self):
        return self * -1.0

    # ---- matmul / reductions / activations ----
    def matmul(self, other):
        return MatMulOp.apply(self, other)

    def __matmul__(self, other):
        return self.matmul(other)

    def sum(self):
        return SumOp.apply(self)

    def relu(self):
        return ReLUOp.apply(self)

    def gelu(self):
        return GELUOp.apply(self)

    # ---- backward ----
    def backward(self, grad_output=None):
        _backward(self, grad_output)

    def __repr__(self):
        n = self.numel()
        body = repr(self.numpy()) if n <= 10 else f"shape={self.shape()}"
        s = f"Tensor({body}, dtype={self.dtype()}"
        if self.requires_grad:
            s += ", requires_grad=True"
            if self._grad_fn is not None:
                s += f", grad_fn={self._grad_fn.__name__}"
        return s + ")"

    def __len__(self):
        return self.shape()[0]

    def __bool__(self):
        if self.numel() != 1:
            raise RuntimeError("bool() on multi-element tensor is ambiguous")
        return bool(self.item())


def zeros_like(t: Tensor) -> Tensor:
    return Tensor.zeros(t.shape(), t.dtype())


def ones_like(t: Tensor) -> Tensor:
    return Tensor.ones(t.shape(), t.dtype())


def randn_like(t: Tensor) -> Tensor:
    return Tensor.randn(t.shape(), t.dtype())


# ---------------------------------------------------------------------------
# differentiable operations
# ---------------------------------------------------------------------------

class AddOp(Function):
    @staticmethod
    def forward(ctx, a, b):
        return Tensor._wrap(a._data + b._data)

    @staticmethod
    def backward(ctx, g):
        return g, g


class SubOp(Function):
    @staticmethod
    def forward(ctx, a, b):
        return Tensor._wrap(a._data - b._data)

    @staticmethod
    def backward(ctx, g):
        return g, Tensor._wrap(g._data * Tensor.full(g.shape(), -1.0, g.dtype())._data)


class MulOp(Function):
    @staticmethod
    def forward(ctx, a, b):
        ctx.save_for_backward(a, b)
        return Tensor._wrap(a._data * b._data)

    @staticmethod
    def backward(ctx, g):
        a, b = ctx.saved_tensors
        return Tensor._wrap(g._data * b._data), Tensor._wrap(g._data * a._data)


class ReshapeOp(Function):
    @staticmethod
    def forward(ctx, a, shape):
        ctx.save_for_backward(list(a.shape()))
        return Tensor._wrap(a._data.reshape(shape))

    @staticmethod
    def backward(ctx, g):
        (shape,) = ctx.saved_tensors
        return (Tensor._wrap(g._data.reshape(shape)),)


class TransposeOp(Function):
    """A strided view; no data moves (reference tensor.py:475-484)."""

    @staticmethod
    def forward(ctx, a, dim0, dim1):
        ctx.save_for_backward(dim0, dim1)
        return Tensor._wrap(a._data.transpose(dim0, dim1))

    @staticmethod
    def backward(ctx, g):
        dim0, dim1 = ctx.saved_tensors
        return (Tensor._wrap(g._data.transpose(dim0, dim1)),)


class MatMulOp(Function):
    """C = A B (reference tensor.py:422-443).  The native matmul reads
    transposed 2-D views as transposed GEMM operands, so neither the
    forward nor the backward copies a transpose."""

    @staticmethod
    def forward(ctx, a, b):
        ctx.save_for_backward(a, b)
        return Tensor._wrap(a._data.matmul(b._data))

    @staticmethod
    def backward(ctx, g):
        a, b = ctx.saved_tensors
        ga = gb = None
        if a.requires_grad:
            ga = Tensor._wrap(g._data.matmul(b._data.transpose(0, 1)))    # dY B^T
        if b.requires_grad:
            gb = Tensor._wrap(a._data.transpose(0, 1).matmul(g._data))    # A^T dY
        return ga, gb


class SumOp(Function):
    @staticmethod
    def forward(ctx, a):
        ctx.save_for_backward(a)
        return Tensor._wrap(_sum(a._data))

    @staticmethod
    def backward(ctx, g):
        (a,) = ctx.saved_tensors
        return (Tensor.full(a.shape(), g.item(), a.dtype()),)


def _make_activation_op(name, fwd):
    class _Op(Function):
        @staticmethod
        def forward(ctx, a):
            ctx.save_for_backward(a)
            return Tensor._wrap(fwd(a._data))

        @staticmethod
        def backward(ctx, g):
            (a,) = ctx.saved_tensors
            return (Tensor._wrap(_activation_backward(g._data, a._data, name)),)

    _Op.__name__ = f"{name.upper() if name == 'gelu' else name.title()}Op"
    return _Op


ReLUOp = _make_activation_op("relu", _relu)
GELUOp = _make_activation_op("gelu", _gelu)


class BroadcastAddOp(Function):
    """matrix [N, M] + row [M] (reference tensor.py:617-631)."""

    @staticmethod
    def forward(ctx, matrix, row):
        ctx.save_for_backward(matrix, row)
        return Tensor._wrap(_broadcast_add(matrix._data, row._data))

    @staticmethod
    def backward(ctx, g):
        matrix, row = ctx.saved_tensors
        g_row = Tensor._wrap(_sum_reduce_rows(g._data)) if row.requires_grad else None
        return (g if matrix.requires_grad else None), g_row


class LinearOp(Function):
    """y = act(x W^T + b) as one fused GEMM (bias and ReLU / GELU in the
    epilogue).  Backward: dZ = act'(...) dY, dX = dZ W (NN GEMM),
    dW = dZ^T x (TN GEMM), db = column sums of dZ.  For ReLU the mask is
    taken from y (y > 0 exactly where x W^T + b > 0); GELU keeps the
    pre-activation, so it is fused only when no gradient is recorded."""

    @staticmethod
    def forward(ctx, x, weight, bias, activation):
        keep_pre = activation == "gelu"
        raw_b = bias._data if bias is not None else None
        if keep_pre:
            z = _linear_forward(x._data, weight._data, raw_b, "none")
            y = _gelu(z)
            ctx.extra["pre"] = z
        else:
            y = _linear_forward(x._data, weight._data, raw_b, activation)
            ctx.extra["out"] = y
        ctx.save_for_backward(x, weight, bias, activation)
        return Tensor._wrap(y)

    @staticmethod
    def backward(ctx, g):
        x, weight, bias, activation = ctx.saved_tensors
        dz = g._data
        if activation == "relu":
            dz = _activation_backward(dz, ctx.extra["out"], "relu")
        elif activation == "gelu":
            dz = _activation_backward(dz, ctx.extra["pre"], "gelu")
        gx = gw = gb = None
        if x.requires_grad:
            gx = Tensor._wrap(_matmul_ex(dz, weight._data, False, False))
        if weight.requires_grad:
            gw = Tensor._wrap(_matmul_ex(dz, x._data, True, False))
        if bias is not None and bias.requires_grad:
            gb = Tensor._wrap(_sum_reduce_rows(dz))
        return gx, gw, gb


class Conv2dOp(Function):
    """NCHW conv (reference tensor.py:691-723): im2col + one GEMM forward
    with the bias in the epilogue; backward data / weight / bias on the GPU."""

    @staticmethod
    def forward(ctx, input, weight, bias, stride, padding):
        raw_b = bias._data if bias is not None else None
        out = _conv2d_forward(input._data, weight._data, raw_b, list(stride), list(padding))
        ctx.save_for_backward(input, weight, bias, tuple(stride), tuple(padding))
        return Tensor._wrap(out)

    @staticmethod
    def backward(ctx, g):
        input, weight, bias, stride, padding = ctx.saved_tensors
        gi = gw = gb = None
        if input.requires_grad:
            gi = Tensor._wrap(_conv2d_backward_data(g._data, weight._data, list(input.shape()),
                                                    list(stride), list(padding)))
        if weight.requires_grad:
            gw = Tensor._wrap(_conv2d_backward_weight(g._data, input._data, list(weight.shape()),
                                                      list(stride), list(padding)))
        if bias is not None and bias.requires_grad:
            gb = Tensor._wrap(_conv2d_backward_bias(g._data))
        return gi, gw, gb


# ---- functional API (reference tensor.py:727-740) ----

def relu(x):
    return x.relu()


def gelu(x):
    return x.gelu()


def broadcast_add(matrix, row):
    return BroadcastAddOp.apply(matrix, row)


def linear(x, weight, bias=None, activation="none"):
    """y = activation(x W^T + b) in one fused GEMM (activation: none / relu / gelu)."""
    return LinearOp.apply(x, weight, bias, activation)


def conv2d(input, weight, bias=None, stride=(1, 1), padding=(0, 0)):
    if isinstance(stride, int):
        stride = (stride, stride)
    if isinstance(padding, int):
        padding = (padding, padding)
    return Conv2dOp.apply(input, weight, bias, tuple(stride), tuple(padding))
