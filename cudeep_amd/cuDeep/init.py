"""Weight initialisers with the reference's names, arguments and
distributions (python/cuDeep/init.py:11-88):

  xavier_uniform_  U(-a, a),  a   = gain * sqrt(6 / (fan_in + fan_out))
  xavier_normal_   N(0, s),   s   = gain * sqrt(2 / (fan_in + fan_out))
  kaiming_uniform_ U(-a, a),  a   = sqrt(2 / (1 + neg_slope^2)) * sqrt(3 / fan)
  kaiming_normal_  N(0, s),   s   = sqrt(2 / (1 + neg_slope^2)) / sqrt(fan)
  uniform_, normal_, zeros_, ones_, constant_

(Glorot & Bengio 2010; He et al. 2015.)  fan_in = size(1) * receptive field,
fan_out = size(0) * receptive field, receptive field = product of the
dimensions after the first two.  Random values come from NumPy's global
generator (so ``np.random.seed`` makes them reproducible, as in the
reference), are drawn on the host and uploaded once, in the tensor's own
dtype.
"""
from __future__ import annotations

import math

import numpy as np

from ._core import DType, Tensor as _RawTensor
from .tensor import Tensor


def _fans(shape) -> tuple:
    dims = list(shape)
    if len(dims) < 2:
        raise ValueError(f"init: fan-in / fan-out need a tensor of 2 or more dimensions, "
                         f"got shape {dims}")
    field = math.prod(dims[2:])
    return dims[1] * field, dims[0] * field


def _relu_family_gain(neg_slope) -> float:
    return math.sqrt(2.0 / (1.0 + float(neg_slope) ** 2))


def _upload(tensor: Tensor, values: np.ndarray) -> Tensor:
    kind = np.float64 if tensor.dtype() == DType.float64 else np.float32
    tensor._data = _RawTensor.from_numpy(np.ascontiguousarray(values, dtype=kind))
    return tensor


def _uniform_fill(tensor: Tensor, lo: float, hi: float) -> Tensor:
    return _upload(tensor, np.random.uniform(lo, hi, tensor.shape()))


def _normal_fill(tensor: Tensor, mean: float, std: float) -> Tensor:
    return _upload(tensor, np.random.normal(mean, std, tensor.shape()))


def xavier_uniform_(tensor: Tensor, gain=1.0):
    fin, fout = _fans(tensor.shape())
    a = gain * math.sqrt(6.0 / (fin + fout))
    return _uniform_fill(tensor, -a, a)


def xavier_normal_(tensor: Tensor, gain=1.0):
    fin, fout = _fans(tensor.shape())
    return _normal_fill(tensor, 0.0, gain * math.sqrt(2.0 / (fin + fout)))


def kaiming_uniform_(tensor: Tensor, a=0, mode="fan_in", nonlinearity="leaky_relu"):
    fan = _fans(tensor.shape())[0 if mode == "fan_in" else 1]
    bound = _relu_family_gain(a) * math.sqrt(3.0 / fan)
    return _uniform_fill(tensor, -bound, bound)


def kaiming_normal_(tensor: Tensor, a=0, mode="fan_in", nonlinearity="leaky_relu"):
    fan = _fans(tensor.shape())[0 if mode == "fan_in" else 1]
    return _normal_fill(tensor, 0.0, _relu_family_gain(a) / math.sqrt(fan))


def uniform_(tensor: Tensor, a=0.0, b=1.0):
    return _uniform_fill(tensor, a, b)


def normal_(tensor: Tensor, mean=0.0, std=1.0):
    return _normal_fill(tensor, mean, std)


def constant_(tensor: Tensor, val):
    tensor._data.fill_(float(val))
    return tensor


def zeros_(tensor: Tensor):
    return constant_(tensor, 0.0)


def ones_(tensor: Tensor):
    return constant_(tensor, 1.0)
