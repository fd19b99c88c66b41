"""Reverse-mode automatic differentiation for cuDeep tensors.

Same contract as the reference engine (python/cuDeep/autograd.py:54-143):
``Function.apply`` records (function, context, parents) on the result when
any input requires grad; ``backward`` walks the graph in reverse
topological order and accumulates parent gradients with the native add.
"""
from __future__ import annotations

_grad_enabled = True


class no_grad:
    """Context manager that disables graph recording."""

    def __enter__(self):
        global _grad_enabled
        self._prev = _grad_enabled
        _grad_enabled = False
        return self

    def __exit__(self, *args):
        global _grad_enabled
        _grad_enabled = self._prev


def is_grad_enabled() -> bool:
    return _grad_enabled


class Context:
    """Holds what a Function's backward needs."""

    __slots__ = ("saved_data", "extra")

    def __init__(self):
        self.saved_data: list = []
        self.extra: dict = {}

    def save_for_backward(self, *args):
        self.saved_data = list(args)

    @property
    def saved_tensors(self) -> list:
        return self.saved_data


class Function:
    """Base class of differentiable operations (static forward / backward)."""

    @staticmethod
    def forward(ctx: Context, *args, **kwargs):
        raise NotImplementedError

    @staticmethod
    def backward(ctx: Context, grad_output):
        raise NotImplementedError

    @classmethod
    def apply(cls, *args, **kwargs):
        from .tensor import Tensor

        ctx = Context()
        parents = tuple(a for a in args if isinstance(a, Tensor))
        needs_grad = _grad_enabled and any(t.requires_grad for t in parents)
        result = cls.forward(ctx, *args, **kwargs)
        outs = result if isinstance(result, tuple) else (result,)
        if needs_grad:
            for r in outs:
                if isinstance(r, Tensor):
                    r.requires_grad = True
                    r._grad_fn = cls
                    r._ctx = ctx
                    r._prev = parents
        return result


def _toposort(root) -> list:
    order, seen = [], set()
    stack = [(root, False)]
    while stack:                       # iterative: deep graphs do not recurse
        t, done = stack.pop()
        if done:
            order.append(t)
            continue
        if id(t) in seen:
            continue
        seen.add(id(t))
        stack.append((t, True))
        for p in t._prev:
            if id(p) not in seen:
                stack.append((p, False))
    return order


def backward(root, grad_output=None):
    """Reverse-mode AD from ``root`` (scalar, or with ``grad_output``)."""
    from .tensor import Tensor, ones_like

    if grad_output is None:
        if root._data.numel() != 1:
            raise RuntimeError("backward() requires grad_output for non-scalar tensors")
        grad_output = ones_like(root)
    root.grad = grad_output
    for t in reversed(_toposort(root)):
        if t._grad_fn is None or t.grad is None:
            continue
        grads = t._grad_fn.backward(t._ctx, t.grad)
        if not isinstance(grads, tuple):
            grads = (grads,)
        for parent, g in zip(t._prev, grads):
            if g is None or not parent.requires_grad:
                continue
            if parent.grad is None:
                parent.grad = g
            else:
                parent.grad = Tensor._wrap(parent.grad._data + g._data)
