"""Reverse-mode automatic differentiation for cuDeep tensors.

Public contract of the reference engine (python/cuDeep/autograd.py:54-143):
``Function`` subclasses define static ``forward(ctx, *args)`` and
``backward(ctx, grad_output)``; ``Function.apply`` runs the forward and, when
gradients are being recorded and some Tensor argument requires them, links
the result into the graph; ``backward(root, grad_output=None)`` propagates
gradients to every tensor that requires them.  ``backward`` returns one
gradient (or None) per Tensor argument of ``forward``, in argument order.

Design.  Each recorded result carries a ``Node`` in ``_grad_fn``: the
Function class, its Context and the input tensors (the graph's edges).  A
backward pass first counts, for every node reachable from the root, how
many recorded consumers feed gradient into it, then runs nodes in
dependency order (Kahn's algorithm): a node runs once all of its
consumers have contributed, from a gradient buffer private to this pass.
Leaf tensors (no node) that require gradients accumulate into ``.grad``
across passes; a recorded result's ``.grad`` is set to the total gradient
it received in the latest pass.

Activation-backward fusion.  During a pass, ``sole_consumer(node)`` tells a
backward whether it is the only recorded consumer feeding gradient into
``node``.  A Linear whose input came out of a ReLU / GELU with no other
consumer then forms its input gradient with that activation's derivative
already applied (in its GEMM epilogue) and the activation's backward passes
it through: one elementwise launch less per activation, the same bits for
every parameter and leaf gradient.  The activation's output then records,
as its ``.grad``, that gradient with the derivative applied (the gradient of
the activation's input).  ``set_fuse_activation_backward(False)`` turns the
fusion off, for callers that read activations' ``.grad``.
"""
from __future__ import annotations

from collections import deque


class _GradMode:
    """Whether Function.apply records graph nodes (process-wide)."""

    enabled = True


class no_grad:
    """Context manager: no graph is recorded inside the block."""

    def __enter__(self):
        self._saved = _GradMode.enabled
        _GradMode.enabled = False
        return self

    def __exit__(self, *exc):
        _GradMode.enabled = self._saved
        return False


def is_grad_enabled() -> bool:
    return _GradMode.enabled


_fuse_activation_backward = True
_pass_counts = []     # consumer counts of the backward passes running (innermost last)


def set_fuse_activation_backward(enabled: bool) -> None:
    """Whether a Linear applies its input's activation derivative in its
    input-gradient GEMM (process-wide, default on)."""
    global _fuse_activation_backward
    _fuse_activation_backward = bool(enabled)


def fuse_activation_backward_enabled() -> bool:
    return _fuse_activation_backward


def sole_consumer(node) -> bool:
    """True inside a backward pass when exactly one recorded consumer feeds
    gradient into ``node`` in that pass."""
    return bool(_pass_counts) and _pass_counts[-1].get(node) == 1


class Context:
    """Per-call scratch of a Function: ``save_for_backward`` / ``saved_tensors``
    for what its backward needs, ``needs_input_grad`` (one flag per Tensor
    argument, set before forward runs), and free attributes for anything
    else the backward wants (e.g. ``ctx.pre = z``)."""

    def __init__(self, needs_input_grad=()):
        self.needs_input_grad = tuple(needs_input_grad)
        self._saved = ()

    def save_for_backward(self, *values):
        self._saved = values

    @property
    def saved_tensors(self):
        return list(self._saved)


class Node:
    """One recorded Function call: how to turn the gradient of its result into
    gradients of its Tensor inputs."""

    __slots__ = ("fn", "ctx", "inputs")

    def __init__(self, fn, ctx, inputs):
        self.fn = fn            # the Function subclass
        self.ctx = ctx          # its Context from the forward
        self.inputs = inputs    # Tensor arguments, in argument order

    @property
    def __name__(self):         # repr of a tensor names its producer
        return self.fn.__name__

    def __repr__(self):
        return f"<Node {self.fn.__name__}>"


class Function:
    """Base class of differentiable operations."""

    @staticmethod
    def forward(ctx: Context, *args, **kwargs):
        raise NotImplementedError

    @staticmethod
    def backward(ctx: Context, grad_output):
        raise NotImplementedError

    @classmethod
    def apply(cls, *args, **kwargs):
        from .tensor import Tensor

        inputs = tuple(a for a in args if isinstance(a, Tensor))
        flags = tuple(bool(t.requires_grad) for t in inputs)
        ctx = Context(flags)
        result = cls.forward(ctx, *args, **kwargs)
        if _GradMode.enabled and any(flags):
            node = Node(cls, ctx, inputs)
            for out in (result if isinstance(result, tuple) else (result,)):
                if isinstance(out, Tensor):
                    out.requires_grad = True
                    out._grad_fn = node
        return result


def _consumer_counts(root_node) -> dict:
    """For every node reachable from root_node: how many edges from other
    reachable nodes point at it (its number of gradient contributions)."""
    counts = {root_node: 0}
    todo = [root_node]
    while todo:
        node = todo.pop()
        for t in node.inputs:
            child = t._grad_fn
            if child is None or not t.requires_grad:
                continue
            if child in counts:
                counts[child] += 1
            else:
                counts[child] = 1
                todo.append(child)
    return counts


def _accumulate(buffers: dict, key, grad):
    prev = buffers.get(key)
    buffers[key] = grad if prev is None else prev._plus(grad)


def backward(root, grad_output=None):
    """Propagate d(root) back through the recorded graph.  ``grad_output``
    defaults to ones for a single-element root and is required otherwise."""
    from .tensor import ones_like

    if grad_output is None:
        if root.numel() != 1:
            raise RuntimeError("backward(): grad_output is required for a tensor with "
                               f"{root.numel()} elements")
        grad_output = ones_like(root)
    root.grad = grad_output
    start = root._grad_fn
    if start is None:
        return
    pending = _consumer_counts(start)
    _pass_counts.append(dict(pending))
    try:
        _run_pass(root, start, grad_output, pending)
    finally:
        _pass_counts.pop()


def _run_pass(root, start, grad_output, pending):
    grads = {start: grad_output}       # gradient buffer per node, this pass only
    outputs = {start: root}            # node -> a tensor it produced (for .grad)
    ready = deque([start])
    while ready:
        node = ready.popleft()
        g = grads.pop(node, None)
        out = outputs.pop(node, None)
        if g is None:
            # every consumer passed None: nothing flows on, but the inputs'
            # pending counts are still released
            in_grads = ()
        else:
            if out is not None and out is not root:
                out.grad = g
            in_grads = node.fn.backward(node.ctx, g)
            if not isinstance(in_grads, tuple):
                in_grads = (in_grads,)
        for i, t in enumerate(node.inputs):
            if not t.requires_grad:
                continue
            gi = in_grads[i] if i < len(in_grads) else None
            child = t._grad_fn
            if child is None:          # leaf: accumulates across passes
                if gi is not None:
                    t.grad = gi if t.grad is None else t.grad._plus(gi)
                continue
            if gi is not None:
                _accumulate(grads, child, gi)
                outputs.setdefault(child, t)
            pending[child] -= 1
            if pending[child] == 0:
                ready.append(child)
