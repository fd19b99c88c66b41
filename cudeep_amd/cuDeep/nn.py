"""Neural-network modules (reference python/cuDeep/nn.py:17-189) for the
dense-contraction path: Parameter, Module, Linear, Conv2d, ReLU, GELU,
Sequential.

``Linear.forward`` is one fused GEMM (x W^T + b, reference nn.py:110-115
launches a transpose copy, the GEMM and a bias kernel), and ``Sequential``
folds a Linear directly followed by ReLU (always) or GELU (when no graph
is recorded) into that GEMM's epilogue.  Default initialisation follows
the reference: weight ~ N(0, 1), bias = 0 (nn.py:104-108).
"""
from __future__ import annotations

from ._core import DType
from .autograd import is_grad_enabled
from .tensor import Tensor, broadcast_add, conv2d, linear


class Parameter(Tensor):
    """A tensor that requires gradients."""

    def __init__(self, data):
        if isinstance(data, Tensor):
            super().__init__(data._data, requires_grad=True)
        else:
            super().__init__(data, requires_grad=True)

    def __repr__(self):
        return f"Parameter(shape={self.shape()}, dtype={self.dtype()})"


class Module:
    def __init__(self):
        self._parameters: dict = {}
        self._modules: dict = {}
        self._training = True

    def forward(self, *args, **kwargs):
        raise NotImplementedError

    def __call__(self, *args, **kwargs):
        return self.forward(*args, **kwargs)

    def register_parameter(self, name: str, tensor):
        if not isinstance(tensor, Parameter):
            tensor = Parameter(tensor)
        self._parameters[name] = tensor

    def register_module(self, name: str, module: "Module"):
        self._modules[name] = module

    def parameters(self) -> list:
        params = list(self._parameters.values())
        for mod in self._modules.values():
            params.extend(mod.parameters())
        return params

    def named_parameters(self):
        for name, p in self._parameters.items():
            yield name, p
        for mod_name, mod in self._modules.items():
            for pname, p in mod.named_parameters():
                yield f"{mod_name}.{pname}", p

    def train(self, mode=True):
        self._training = mode
        for m in self._modules.values():
            m.train(mode)
        return self

    def eval(self):
        return self.train(False)

    @property
    def training(self):
        return self._training

    def state_dict(self) -> dict:
        return {name: p.numpy() for name, p in self.named_parameters()}

    def load_state_dict(self, sd: dict):
        import numpy as np
        from ._core import Tensor as _RT
        params = dict(self.named_parameters())
        for name, arr in sd.items():
            if name in params:
                params[name]._data = _RT.from_numpy(np.ascontiguousarray(arr))

    def zero_grad(self):
        for p in self.parameters():
            p.grad = None


class Linear(Module):
    """y = x W^T + b."""

    def __init__(self, in_features, out_features, bias=True, dtype=DType.float32):
        super().__init__()
        self.in_features = in_features
        self.out_features = out_features
        self.register_parameter("weight", Tensor.randn([out_features, in_features], dtype))
        if bias:
            self.register_parameter("bias", Tensor.zeros([out_features], dtype))

    def forward(self, x, activation="none"):
        w = self._parameters["weight"]
        b = self._parameters.get("bias")
        if w.dtype() == DType.float64:
            # fp64: the fp64 GEMM with the transposed view, then the bias
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
    """2-D convolution, NCHW / OIHW."""

    def __init__(self, in_channels, out_channels, kernel_size, stride=1, padding=0, bias=True,
                 dtype=DType.float32):
        super().__init__()
        if isinstance(kernel_size, int):
            kernel_size = (kernel_size, kernel_size)
        if isinstance(stride, int):
            stride = (stride, stride)
        if isinstance(padding, int):
            padding = (padding, padding)
        self.in_channels = in_channels
        self.out_channels = out_channels
        self.kernel_size = tuple(kernel_size)
        self.stride = tuple(stride)
        self.padding = tuple(padding)
        self.register_parameter(
            "weight", Tensor.randn([out_channels, in_channels, kernel_size[0], kernel_size[1]], dtype))
        if bias:
            self.register_parameter("bias", Tensor.zeros([out_channels], dtype))

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

    def forward(self, x):
        mods = list(self._modules.values())
        i = 0
        while i < len(mods):
            m = mods[i]
            nxt = mods[i + 1] if i + 1 < len(mods) else None
            if isinstance(m, Linear) and isinstance(nxt, ReLU):
                x = m(x, activation="relu")
                i += 2
            elif isinstance(m, Linear) and isinstance(nxt, GELU) and not is_grad_enabled():
                x = m(x, activation="gelu")
                i += 2
            else:
                x = m(x)
                i += 1
        return x

    def __getitem__(self, idx):
        return list(self._modules.values())[idx]

    def __len__(self):
        return len(self._modules)
