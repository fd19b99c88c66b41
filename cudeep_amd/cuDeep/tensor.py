"""Autograd-aware Tensor over the native ``_cudeep_core.Tensor``.

The public surface of the reference's python/cuDeep/tensor.py:57-319 for the
dense-contraction path -- construction from NumPy arrays, lists, scalars or
raw tensors; the zeros / ones / randn / from_numpy / full factories; shape
queries; reshape / transpose / t; +, -, * (tensors or scalars), @ / matmul;
sum; relu / gelu; broadcast_add; conv2d; linear; backward -- over a design
of this build:

* a Tensor is a thin handle: the native tensor (``_data``), ``grad``,
  ``requires_grad`` and the graph node that produced it (``_grad_fn``, see
  autograd.py);
* operator overloads go through one table (``_BINARY``) and one scalar
  promotion rule;
* the differentiable operations work without materialised transposes:
  ``MatMulOp.backward`` computes dA = dY B^T and dB = A^T dY with transposed-
  operand GEMMs (reference tensor.py:430-443 copies both), ``linear`` runs
  x W^T + b with its activation as one fused GEMM, and ``Conv2dOp.backward``
  computes the bias gradient on the GPU (reference tensor.py:718-721 sums on
  the host in NumPy).
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
    linear_input_grad as _linear_input_grad,
    linear_weight_grad as _linear_weight_grad,
    matmul_ex as _matmul_ex,
    relu as _relu,
    sum as _sum,
    sum_reduce_rows as _sum_reduce_rows,
)
from .autograd import (
    Function,
    backward as _run_backward,
    fuse_activation_backward_enabled as _fusion_on,
    sole_consumer as _sole_consumer,
)


def _np_dtype(dtype) -> type:
    return np.float64 if dtype == DType.float64 else np.float32


def _to_raw(data, dtype) -> _RawTensor:
    """Native tensor holding `data` (a native tensor is taken as is; NumPy
    data is uploaded as float32 unless it is float64 or dtype asks)."""
    if isinstance(data, _RawTensor):
        return data
    if isinstance(data, Tensor):
        return data._data
    if isinstance(data, np.ndarray):
        if dtype is not None:
            want = _np_dtype(dtype)
        else:
            want = data.dtype.type if data.dtype in (np.float32, np.float64) else np.float32
        return _RawTensor.from_numpy(np.ascontiguousarray(data, dtype=want))
    if isinstance(data, (list, tuple, int, float, np.floating, np.integer)):
        return _RawTensor.from_numpy(np.asarray(data, dtype=_np_dtype(dtype)))
    raise TypeError(f"Tensor(): unsupported data of type {type(data).__name__}")


class Tensor:
    """GPU tensor with reverse-mode autograd."""

    # _act_applied: on a gradient, the Context of the activation whose
    # derivative the gradient already carries (set by the consumer that
    # fused it into its GEMM epilogue; that activation's backward then
    # passes the gradient through).
    __slots__ = ("_data", "grad", "requires_grad", "_grad_fn", "_act_applied")

    def __init__(self, data, requires_grad=False, dtype=None):
        self._data = _to_raw(data, dtype)
        self.grad: Optional[Tensor] = None
        self.requires_grad = bool(requires_grad)
        self._grad_fn = None
        self._act_applied = None

    @classmethod
    def _wrap(cls, raw, requires_grad=False) -> "Tensor":
        """A handle on an existing native tensor (no copy, no conversion)."""
        t = cls.__new__(cls)
        t._data = raw
        t.grad = None
        t.requires_grad = requires_grad
        t._grad_fn = None
        t._act_applied = None
        return t

    def _plus(self, other: "Tensor") -> "Tensor":
        """Unrecorded sum (gradient accumulation)."""
        return Tensor._wrap(self._data + other._data)

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
        return Tensor._wrap(_to_raw(np.asarray(arr), None), requires_grad)

    @staticmethod
    def full(shape, value, dtype=DType.float32, requires_grad=False) -> "Tensor":
        raw = _RawTensor(list(shape), dtype)
        raw.fill_(float(value))
        return Tensor._wrap(raw, requires_grad)

    # ---- queries (forwarded to the native tensor) ----
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
        values = self._data.numpy().reshape(-1)
        if values.size != 1:
            raise ValueError(f"item(): tensor has {values.size} elements, not one")
        return values[0].item()

    def detach(self) -> "Tensor":
        return Tensor._wrap(self._data)

    def contiguous(self) -> "Tensor":
        return self if self.is_contiguous() else Tensor._wrap(self._data.contiguous(),
                                                               self.requires_grad)

    def clone(self) -> "Tensor":
        return Tensor._wrap(self._data.clone(), self.requires_grad)

    # ---- in place, unrecorded ----
    def fill_(self, value):
        self._data.fill_(float(value))
        return self

    def zero_(self):
        self._data.zero_()
        return self

    # ---- views ----
    def reshape(self, *shape):
        dims = list(shape[0]) if len(shape) == 1 and isinstance(shape[0], (list, tuple)) \
            else list(shape)
        return ReshapeOp.apply(self, dims)

    def transpose(self, dim0, dim1):
        return TransposeOp.apply(self, dim0, dim1)

    def t(self):
        return TransposeOp.apply(self, 0, 1)

    # ---- arithmetic: tensors or Python scalars (promoted to a filled tensor) ----
    def _operand(self, other) -> "Tensor":
        if isinstance(other, Tensor):
            return other
        if isinstance(other, (int, float, np.floating, np.integer)):
            return Tensor.full(self.shape(), other, self.dtype())
        return NotImplemented

    def _binary(self, op: str, other, swap: bool = False):
        rhs = self._operand(other)
        if rhs is NotImplemented:
            return NotImplemented
        lhs, rhs = (rhs, self) if swap else (self, rhs)
        return _BINARY[op].apply(lhs, rhs)

    def __add__(self, other):
        return self._binary("+", other)

    def __radd__(self, other):
        return self._binary("+", other, swap=True)

    def __sub__(self, other):
        return self._binary("-", other)

    def __rsub__(self, other):
        return self._binary("-", other, swap=True)

    def __mul__(self, other):
        return self._binary("*", other)

    def __rmul__(self, other):
        return self._binary("*", other, swap=True)

    def __neg__(self):
        return self._binary("*", -1.0)

    def matmul(self, other):
        return MatMulOp.apply(self, other)

    def __matmul__(self, other):
        return MatMulOp.apply(self, other)

    # ---- reductions / activations ----
    def sum(self):
        return SumOp.apply(self)

    def relu(self):
        return ReLUOp.apply(self)

    def gelu(self):
        return GELUOp.apply(self)

    # ---- autograd ----
    def backward(self, grad_output=None):
        _run_backward(self, grad_output)

    def __repr__(self):
        fields = [f"shape={self.shape()}", f"dtype={self.dtype()}"]
        if self.numel() <= 10:
            fields.insert(0, np.array2string(self.numpy(), separator=", "))
        if self._grad_fn is not None:
            fields.append(f"grad_fn={self._grad_fn.__name__}")
        elif self.requires_grad:
            fields.append("requires_grad=True")
        return f"Tensor({', '.join(fields)})"

    def __len__(self):
        dims = self.shape()
        if not dims:
            raise TypeError("len() of a 0-d tensor")
        return dims[0]

    def __bool__(self):
        if self.numel() != 1:
            raise RuntimeError(f"the truth value of a tensor with {self.numel()} elements "
                               "is ambiguous")
        return bool(self.item())


def zeros_like(t: Tensor) -> Tensor:
    return Tensor.zeros(t.shape(), t.dtype())


def ones_like(t: Tensor) -> Tensor:
    return Tensor.ones(t.shape(), t.dtype())


def randn_like(t: Tensor) -> Tensor:
    return Tensor.randn(t.shape(), t.dtype())


# ---------------------------------------------------------------------------
# differentiable operations (backward: one gradient per Tensor argument)
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
        need_a, need_b = ctx.needs_input_grad
        neg = Tensor._wrap(g._data * Tensor.full(g.shape(), -1.0, g.dtype())._data) \
            if need_b else None
        return g, neg


class MulOp(Function):
    @staticmethod
    def forward(ctx, a, b):
        ctx.save_for_backward(a, b)
        return Tensor._wrap(a._data * b._data)

    @staticmethod
    def backward(ctx, g):
        a, b = ctx.saved_tensors
        need_a, need_b = ctx.needs_input_grad
        return (Tensor._wrap(g._data * b._data) if need_a else None,
                Tensor._wrap(g._data * a._data) if need_b else None)


_BINARY = {"+": AddOp, "-": SubOp, "*": MulOp}


class ReshapeOp(Function):
    @staticmethod
    def forward(ctx, a, shape):
        ctx.in_shape = list(a.shape())
        return Tensor._wrap(a._data.reshape(shape))

    @staticmethod
    def backward(ctx, g):
        return Tensor._wrap(g._data.reshape(ctx.in_shape))


class TransposeOp(Function):
    """A strided view; no data moves (reference tensor.py:475-484)."""

    @staticmethod
    def forward(ctx, a, dim0, dim1):
        ctx.dims = (dim0, dim1)
        return Tensor._wrap(a._data.transpose(dim0, dim1))

    @staticmethod
    def backward(ctx, g):
        return Tensor._wrap(g._data.transpose(*ctx.dims))


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
        need_a, need_b = ctx.needs_input_grad
        ga = Tensor._wrap(g._data.matmul(b._data.transpose(0, 1))) if need_a else None  # dY B^T
        gb = Tensor._wrap(a._data.transpose(0, 1).matmul(g._data)) if need_b else None  # A^T dY
        return ga, gb


class SumOp(Function):
    @staticmethod
    def forward(ctx, a):
        ctx.in_shape, ctx.in_dtype = a.shape(), a.dtype()
        return Tensor._wrap(_sum(a._data))

    @staticmethod
    def backward(ctx, g):
        return Tensor.full(ctx.in_shape, g.item(), ctx.in_dtype)


class _ActivationOp(Function):
    """y = act(x) elementwise; backward from the saved input (none when the
    consumer of y already applied act'(x) in its GEMM epilogue)."""

    NAME = ""
    FORWARD = None

    @classmethod
    def forward(cls, ctx, a):
        ctx.save_for_backward(a)
        ctx.activation, ctx.aux = cls.NAME, a._data
        return Tensor._wrap(cls.FORWARD(a._data))

    @classmethod
    def backward(cls, ctx, g):
        if g._act_applied is ctx:
            return g
        (a,) = ctx.saved_tensors
        return Tensor._wrap(_activation_backward(g._data, a._data, cls.NAME))


class ReLUOp(_ActivationOp):
    NAME = "relu"
    FORWARD = staticmethod(_relu)


class GELUOp(_ActivationOp):
    NAME = "gelu"
    FORWARD = staticmethod(_gelu)


class BroadcastAddOp(Function):
    """matrix [N, M] + row [M] (reference tensor.py:617-631)."""

    @staticmethod
    def forward(ctx, matrix, row):
        return Tensor._wrap(_broadcast_add(matrix._data, row._data))

    @staticmethod
    def backward(ctx, g):
        need_m, need_r = ctx.needs_input_grad
        return (g if need_m else None,
                Tensor._wrap(_sum_reduce_rows(g._data)) if need_r else None)


def _fusable_activation(x: Tensor):
    """The Context of the activation that produced x, when a consumer GEMM
    can apply its derivative in the epilogue: x is the direct output of a
    recorded float32 ReLU / GELU (an activation op, or a Linear with that
    activation fused) and the caller is its only consumer in this backward
    pass (GELU's derivative must not multiply a gradient twice, and a sum of
    contributions is formed after the consumers run).  Its ``aux`` is what
    the derivative reads (the input of the activation; for ReLU the output
    serves as well, since y > 0 exactly where x > 0)."""
    node = x._grad_fn
    if node is None or not _fusion_on() or not _sole_consumer(node):
        return None
    ctx = node.ctx
    if getattr(ctx, "activation", "none") not in ("relu", "gelu"):
        return None
    aux = getattr(ctx, "aux", None)
    if aux is None or aux.dtype() != DType.float32 or x.dtype() != DType.float32:
        return None
    return ctx


class LinearOp(Function):
    """y = act(x W^T + b) as one fused GEMM (bias and ReLU / GELU in the
    epilogue).  Backward: dZ = act'(...) dY, dX = dZ W (NN GEMM), and
    dW = dZ^T x with db = column sums of dZ from the same launch (a column of
    ones appended to x).  For ReLU the mask is taken from y (y > 0 exactly
    where x W^T + b > 0); GELU keeps the pre-activation, so its activation is
    a separate launch when recorded.

    When x itself came out of a recorded ReLU / GELU (a Linear with that
    activation, or the activation op), dX is formed with that activation's
    derivative in the GEMM epilogue -- dX = act'(aux) (.) (dZ W) -- and
    marked, so the producer's backward skips its own activation-backward
    launch (the reference runs it as a kernel of its own,
    python/cuDeep/tensor.py:430-443 then activation_kernel.cu:256-319).  The
    epilogue uses the elementwise kernel's formulas, so the gradients are the
    same bits either way.  A gradient that other consumers add to loses the
    mark (the sum is a new tensor), and the producer then applies its
    derivative to the sum, as it must."""

    @staticmethod
    def forward(ctx, x, weight, bias, activation):
        raw_b = bias._data if bias is not None else None
        ctx.activation = activation
        if activation == "gelu":
            ctx.aux = _linear_forward(x._data, weight._data, raw_b, "none")
            y = _gelu(ctx.aux)
        else:
            y = _linear_forward(x._data, weight._data, raw_b, activation)
            ctx.aux = y
        ctx.save_for_backward(x, weight)
        return Tensor._wrap(y)

    @staticmethod
    def backward(ctx, g):
        x, weight = ctx.saved_tensors
        flags = ctx.needs_input_grad
        need_x, need_w = flags[0], flags[1]
        need_b = len(flags) > 2 and flags[2]
        dz = g._data
        if ctx.activation != "none" and g._act_applied is not ctx:
            dz = _activation_backward(dz, ctx.aux, ctx.activation)
        gx = None
        if need_x:
            producer = _fusable_activation(x)
            if producer is not None:
                gx = Tensor._wrap(_linear_input_grad(dz, weight._data, producer.aux,
                                                     producer.activation))
                gx._act_applied = producer
            else:
                gx = Tensor._wrap(_matmul_ex(dz, weight._data, False, False))
        gw = gb = None
        if need_w:
            raw_w, raw_b = _linear_weight_grad(dz, x._data, bool(need_b))
            gw = Tensor._wrap(raw_w)
            gb = Tensor._wrap(raw_b) if need_b else None
        elif need_b:
            gb = Tensor._wrap(_sum_reduce_rows(dz))
        return gx, gw, gb


class Conv2dOp(Function):
    """NCHW conv (reference tensor.py:691-723): forward with the bias in the
    GEMM epilogue; backward data / weight / bias on the GPU."""

    @staticmethod
    def forward(ctx, input, weight, bias, stride, padding):
        raw_b = bias._data if bias is not None else None
        ctx.geom = (list(stride), list(padding))
        ctx.save_for_backward(input, weight)
        return Tensor._wrap(_conv2d_forward(input._data, weight._data, raw_b, list(stride),
                                            list(padding)))

    @staticmethod
    def backward(ctx, g):
        x, w = ctx.saved_tensors
        stride, padding = ctx.geom
        flags = ctx.needs_input_grad
        need_b = len(flags) > 2 and flags[2]
        gx = Tensor._wrap(_conv2d_backward_data(g._data, w._data, list(x.shape()), stride,
                                                padding)) if flags[0] else None
        gw = Tensor._wrap(_conv2d_backward_weight(g._data, x._data, list(w.shape()), stride,
                                                  padding)) if flags[1] else None
        gb = Tensor._wrap(_conv2d_backward_bias(g._data)) if need_b else None
        return gx, gw, gb


# ---- functional API (reference tensor.py:727-740) ----

def relu(x):
    return ReLUOp.apply(x)


def gelu(x):
    return GELUOp.apply(x)


def broadcast_add(matrix, row):
    return BroadcastAddOp.apply(matrix, row)


def linear(x, weight, bias=None, activation="none"):
    """y = activation(x W^T + b) in one fused GEMM (activation: none / relu / gelu)."""
    return LinearOp.apply(x, weight, bias, activation)


def _pair(v):
    return (v, v) if isinstance(v, int) else tuple(v)


def conv2d(input, weight, bias=None, stride=(1, 1), padding=(0, 0)):
    return Conv2dOp.apply(input, weight, bias, _pair(stride), _pair(padding))
