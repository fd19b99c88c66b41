"""Neural-network modules for the dense-contraction path, with the
reference's names and constructor arguments (python/cuDeep/nn.py:17-189):
Parameter, Module, Linear, Conv2d, ReLU, GELU, Sequential.

Module keeps its parameters and children in ``_parameters`` / ``_modules``
(name -> object, registration order), filled either through
``register_parameter`` / ``register_module`` or by plain attribute
assignment; attribute reads fall back to those tables, so
``layer._parameters["weight"] = t`` and ``layer.weight`` always agree.
Parameter names are dotted paths from one depth-first walk of the module
tree (a module's own parameters, then each child's in order).

``Linear.forward`` is one fused GEMM (x W^T + b, where the reference's
nn.py:110-115 launches a transpose copy, the GEMM and a bias kernel), and
``Sequential`` folds a Linear directly followed by ReLU (always) or GELU
(when no graph is recorded) into that GEMM's epilogue.  Default
initialisation follows the reference: weight ~ N(0, 1), bias = 0
(nn.py:104-108).
"""
from __future__ import annotations

import numpy as np

from ._core import DType, Tensor as _RawTensor
from .autograd import is_grad_enabled
from .tensor import Tensor, broadcast_add, conv2d, linear


class Parameter(Tensor):
    """A Tensor that requires gradients; built from a Tensor it shares that
    tensor's storage."""

    def __init__(self, data):
        super().__init__(data._data if isinstance(data, Tensor) else data, requires_grad=True)

    def __repr__(self):
        return f"Parameter({self.shape()}, {self.dtype()})"


class Module:
    """Base class: a tree of modules owning parameters."""

    def __init__(self):
        object.__setattr__(self, "_parameters", {})
        object.__setattr__(self, "_modules", {})
        object.__setattr__(self, "_training", True)

    # ---- registration ----
    def __setattr__(self, name, value):
        if isinstance(value, Parameter):
            self.__dict__.pop(name, None)
            self._parameters[name] = value
        elif isinstance(value, Module):
            self.__dict__.pop(name, None)
            self._modules[name] = value
        else:
            object.__setattr__(self, name, value)

    def __getattr__(self, name):
        # only reached when ordinary lookup fails
        for table in ("_parameters", "_modules"):
            entries = self.__dict__.get(table)
            if entries is not None and name in entries:
                return entries[name]
        raise AttributeError(f"{type(self).__name__} has no attribute {name!r}")

    def register_parameter(self, name: str, tensor):
        self._parameters[name] = tensor if isinstance(tensor, Parameter) else Parameter(tensor)

    def register_module(self, name: str, module: "Module"):
        self._modules[name] = module

    # ---- traversal ----
    def _walk(self, prefix: str = ""):
        """(dotted prefix, module) for this module and every descendant,
        depth first, in registration order."""
        yield prefix, self
        for name, child in self._modules.items():
            yield from child._walk(f"{prefix}{name}.")

    def named_parameters(self):
        for prefix, mod in self._walk():
            for name, p in mod._parameters.items():
                yield prefix + name, p

    def parameters(self) -> list:
        seen, out = set(), []
        for _, p in self.named_parameters():
            if id(p) not in seen:
                seen.add(id(p))
                out.append(p)
        return out

    # ---- mode ----
    def train(self, mode=True):
        for _, mod in self._walk():
            object.__setattr__(mod, "_training", bool(mode))
        return self

    def eval(self):
        return self.train(False)

    @property
    def training(self):
        return self._training

    # ---- state ----
    def state_dict(self) -> dict:
        return {name: p.numpy() for name, p in self.named_parameters()}

    def load_state_dict(self, sd: dict):
        """Copies each array of `sd` whose name is a parameter of this module
        into that parameter (same shape required); other names are ignored."""
        params = dict(self.named_parameters())
        for name, values in sd.items():
            p = params.get(name)
            if p is None:
                continue
            arr = np.asarray(values)
            if list(arr.shape) != list(p.shape()):
                raise ValueError(f"load_state_dict: {name} has shape {list(arr.shape)}, "
                                 f"the parameter {p.shape()}")
            kind = np.float64 if p.dtype() == DType.float64 else np.float32
            p._data = _RawTensor.from_numpy(np.ascontiguousarray(arr, dtype=kind))

    def zero_grad(self):
        for p in self.parameters():
            p.grad = None

    # ---- call ----
    def forward(self, *args, **kwargs):
        raise NotImplementedError

    def __call__(self, *args, **kwargs):
        return self.forward(*args, **kwargs)


class Linear(Module):
    """y = x W^T + b; weight [out_features, in_features]."""

    def __init__(self, in_features, out_features, bias=True, dtype=DType.float32):
        super().__init__()
        self.in_features = in_features
        self.out_features = out_features
        self.weight = Parameter(Tensor.randn([out_features, in_features], dtype))
        if bias:
            self.bias = Parameter(Tensor.zeros([out_features], dtype))

    def forward(self, x, activation="none"):
        w = self._parameters["weight"]
        b = self._parameters.get("bias")
        if w.dtype() == DType.float64:
            # fp64: the fp64 GEMM on the transposed view, then the bias
            out = x.matmul(w.transpose(0, 1))
            if b is not None:
                out = broadcast_add(out, b)
            if activation == "relu":
                out = out.relu()
            elif activation == "gelu":
                out = out.gelu()
            return out
        return linear(x, w, b, activation)


class Conv2d(Module):
    """2-D convolution, NCHW input, OIHW weight."""

    def __init__(self, in_channels, out_channels, kernel_size, stride=1, padding=0, bias=True,
                 dtype=DType.float32):
        super().__init__()

        def pair(v):
            return (v, v) if isinstance(v, int) else tuple(v)

        self.in_channels = in_channels
        self.out_channels = out_channels
        self.kernel_size = pair(kernel_size)
        self.stride = pair(stride)
        self.padding = pair(padding)
        self.weight = Parameter(Tensor.randn([out_channels, in_channels, *self.kernel_size],
                                             dtype))
        if bias:
            self.bias = Parameter(Tensor.zeros([out_channels], dtype))

    def forward(self, x):
        return conv2d(x, self._parameters["weight"], self._parameters.get("bias"),
                      self.stride, self.padding)


class ReLU(Module):
    def forward(self, x):
        return x.relu()


class GELU(Module):
    def forward(self, x):
        return x.gelu()


class Sequential(Module):
    """Runs modules in order; a Linear followed by ReLU (or by GELU when no
    graph is recorded) becomes one GEMM with the activation in its epilogue."""

    def __init__(self, *modules):
        super().__init__()
        for i, m in enumerate(modules):
            self.register_module(str(i), m)

    def _stages(self):
        """(module, fused activation) pairs in execution order."""
        mods = list(self._modules.values())
        i = 0
        while i < len(mods):
            m, nxt = mods[i], mods[i + 1] if i + 1 < len(mods) else None
            act = None
            if isinstance(m, Linear):
                if isinstance(nxt, ReLU):
                    act = "relu"
                elif isinstance(nxt, GELU) and not is_grad_enabled():
                    act = "gelu"
            yield m, act
            i += 2 if act else 1

    def forward(self, x):
        for m, act in self._stages():
            x = m(x, activation=act) if act else m(x)
        return x

    def __getitem__(self, idx):
        return list(self._modules.values())[idx]

    def __len__(self):
        return len(self._modules)
