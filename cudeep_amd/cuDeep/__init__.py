"""cuDeep's public Python API for the dense-contraction path, on MI355X.

Drop-in for the reference package's ``cuDeep`` (python/cuDeep/__init__.py)
as far as Tensor.matmul, nn.Linear and nn.Conv2d (forward and backward)
go: ``from cudeep_amd import cuDeep`` (or put ``cudeep_amd/`` on sys.path
and ``import cuDeep``).  Everything runs in libcudeep_amd.so through the
native ``_cudeep_core`` module; there is no CPU fallback.
"""

__version__ = "0.1.0"

from ._core import (DType, Event, Layout, MemoryPool, Stream, device_info,  # noqa: F401
                    get_conv_algorithm, get_matmul_precision, set_conv_algorithm,
                    set_matmul_precision)
from .tensor import (Tensor, broadcast_add, conv2d, gelu, linear, ones_like,  # noqa: F401
                     randn_like, relu, zeros_like)
from .autograd import no_grad  # noqa: F401
from . import autograd, init, nn  # noqa: F401

__all__ = [
    "Tensor", "DType", "Layout", "Stream", "Event", "MemoryPool", "device_info",
    "zeros_like", "ones_like", "randn_like", "relu", "gelu", "broadcast_add", "conv2d",
    "linear", "no_grad", "nn", "autograd", "init", "set_matmul_precision",
    "get_matmul_precision", "set_conv_algorithm", "get_conv_algorithm",
]
