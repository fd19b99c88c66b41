"""Weight initialisers (reference python/cuDeep/init.py:11-88): fan
computation and the Xavier / Kaiming bounds of the reference.  Values are
drawn on the host with numpy's global generator, as the reference does,
and uploaded."""
from __future__ import annotations

import math

import numpy as np

from ._core import DType, Tensor as _RawTensor
from .tensor import Tensor


def _fan_in_out(tensor: Tensor):
    shape = tensor.shape()
    if len(shape) < 2:
        raise ValueError("fan_in/fan_out requires at least 2D tensor")
    fan_in, fan_out = shape[1], shape[0]
    if len(shape) > 2:
        receptive = int(np.prod(shape[2:]))
        fan_in *= receptive
        fan_out *= receptive
    return fan_in, fan_out


def _set(tensor: Tensor, arr: np.ndarray) -> Tensor:
    dt = np.float64 if tensor.dtype() == DType.float64 else np.float32
    tensor._data = _RawTensor.from_numpy(np.ascontiguousarray(arr, dtype=dt))
    return tensor


def xavier_uniform_(tensor: Tensor, gain=1.0):
    fan_in, fan_out = _fan_in_out(tensor)
    bound = gain * math.sqrt(6.0 / (fan_in + fan_out))
    return _set(tensor, np.random.uniform(-bound, bound, tensor.shape()))


def xavier_normal_(tensor: Tensor, gain=1.0):
    fan_in, fan_out = _fan_in_out(tensor)
    std = gain * math.sqrt(2.0 / (fan_in + fan_out))
    return _set(tensor, np.random.normal(0, std, tensor.shape()))


def kaiming_uniform_(tensor: Tensor, a=0, mode="fan_in", nonlinearity="leaky_relu"):
    fan_in, fan_out = _fan_in_out(tensor)
    fan = fan_in if mode == "fan_in" else fan_out
    bound = math.sqrt(2.0 / (1 + a ** 2)) * math.sqrt(3.0 / fan)
    return _set(tensor, np.random.uniform(-bound, bound, tensor.shape()))


def kaiming_normal_(tensor: Tensor, a=0, mode="fan_in", nonlinearity="leaky_relu"):
    fan_in, fan_out = _fan_in_out(tensor)
    fan = fan_in if mode == "fan_in" else fan_out
    std = math.sqrt(2.0 / (1 + a ** 2)) / math.sqrt(fan)
    return _set(tensor, np.random.normal(0, std, tensor.shape()))


def zeros_(tensor: Tensor):
    tensor._data.zero_()
    return tensor


def ones_(tensor: Tensor):
    tensor._data.fill_(1.0)
    return tensor


def constant_(tensor: Tensor, val):
    tensor._data.fill_(float(val))
    return tensor


def uniform_(tensor: Tensor, a=0.0, b=1.0):
    return _set(tensor, np.random.uniform(a, b, tensor.shape()))


def normal_(tensor: Tensor, mean=0.0, std=1.0):
    return _set(tensor, np.random.normal(mean, std, tensor.shape()))
