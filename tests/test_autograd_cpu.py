"""The autograd engine on the CPU: tensors whose ``_data`` is a NumPy array
(no GPU), driven by small test-only Functions, so the graph bookkeeping --
ordering, accumulation, None gradients, no_grad -- is checked against hand
derivatives without any device work."""
import numpy as np
import pytest

cuDeep = pytest.importorskip("cudeep_amd.cuDeep")
from cudeep_amd.cuDeep.autograd import Function, backward, no_grad  # noqa: E402
from cudeep_amd.cuDeep.tensor import Tensor  # noqa: E402


def T(values, requires_grad=False):
    return Tensor._wrap(np.asarray(values, np.float64), requires_grad)


class Scale(Function):
    @staticmethod
    def forward(ctx, x, c):
        ctx.c = c
        return Tensor._wrap(x._data * c)

    @staticmethod
    def backward(ctx, g):
        return Tensor._wrap(g._data * ctx.c)


class Mul(Function):
    @staticmethod
    def forward(ctx, a, b):
        ctx.save_for_backward(a, b)
        return Tensor._wrap(a._data * b._data)

    @staticmethod
    def backward(ctx, g):
        a, b = ctx.saved_tensors
        return Tensor._wrap(g._data * b._data), Tensor._wrap(g._data * a._data)


class Add(Function):
    @staticmethod
    def forward(ctx, a, b):
        return Tensor._wrap(a._data + b._data)

    @staticmethod
    def backward(ctx, g):
        return g, g


class FirstOnly(Function):
    """y = a + b, but the backward hands b no gradient (None)."""

    @staticmethod
    def forward(ctx, a, b):
        return Tensor._wrap(a._data + b._data)

    @staticmethod
    def backward(ctx, g):
        return g, None


def ones_like(t):
    return T(np.ones_like(t._data))


def test_diamond_sums_both_paths():
    x = T([1.0, -2.0, 3.0], requires_grad=True)
    a, b = Scale.apply(x, 2.0), Scale.apply(x, 3.0)
    y = Mul.apply(a, b)                 # 6 x^2
    backward(y, ones_like(y))
    np.testing.assert_allclose(x.grad._data, 12 * x._data)
    np.testing.assert_allclose(a.grad._data, b._data)     # intermediate .grad = dy/da
    np.testing.assert_allclose(b.grad._data, a._data)


def test_shared_subexpression_runs_its_backward_once():
    calls = []

    class Probe(Scale):
        @staticmethod
        def backward(ctx, g):
            calls.append(1)
            return Tensor._wrap(g._data * ctx.c)

    x = T([2.0], requires_grad=True)
    h = Probe.apply(x, 5.0)
    y = Add.apply(Mul.apply(h, h), Scale.apply(h, 4.0))   # 25 x^2 + 20 x
    backward(y, ones_like(y))
    assert calls == [1]                 # h's node waits for all three consumers
    np.testing.assert_allclose(x.grad._data, [50 * 2.0 + 20])


def test_leaf_accumulates_across_passes_and_intermediates_do_not():
    x = T([1.5], requires_grad=True)
    for _ in range(3):
        h = Scale.apply(x, 2.0)
        y = Scale.apply(h, 3.0)
        backward(y, ones_like(y))
    np.testing.assert_allclose(x.grad._data, [18.0])
    np.testing.assert_allclose(h.grad._data, [3.0])


def test_same_graph_backward_twice_accumulates_exactly_twice():
    x = T([1.0, 2.0], requires_grad=True)
    y = Mul.apply(Scale.apply(x, 3.0), x)     # 3 x^2
    backward(y, ones_like(y))
    backward(y, ones_like(y))
    np.testing.assert_allclose(x.grad._data, 2 * 6 * x._data)


def test_none_gradient_still_releases_the_input():
    x = T([1.0], requires_grad=True)
    w = T([2.0], requires_grad=True)
    h = Scale.apply(w, 7.0)             # reached by two consumers
    y = Add.apply(FirstOnly.apply(x, h), Scale.apply(h, 1.0))
    backward(y, ones_like(y))
    np.testing.assert_allclose(x.grad._data, [1.0])
    np.testing.assert_allclose(w.grad._data, [7.0])        # only the second path


def test_inputs_without_requires_grad_get_nothing():
    x = T([1.0], requires_grad=True)
    c = T([4.0])
    y = Mul.apply(x, c)
    backward(y, ones_like(y))
    np.testing.assert_allclose(x.grad._data, [4.0])
    assert c.grad is None
    assert y._grad_fn is not None and c._grad_fn is None


def test_no_grad_records_nothing():
    x = T([1.0], requires_grad=True)
    with no_grad():
        y = Scale.apply(x, 2.0)
        assert not cuDeep.autograd.is_grad_enabled()
    assert cuDeep.autograd.is_grad_enabled()
    assert y._grad_fn is None and not y.requires_grad


def test_needs_input_grad_flags():
    seen = {}

    class Spy(Function):
        @staticmethod
        def forward(ctx, a, k, b):
            seen["flags"] = ctx.needs_input_grad
            return Tensor._wrap(a._data + b._data)

        @staticmethod
        def backward(ctx, g):
            return g, g

    Spy.apply(T([1.0]), "not a tensor", T([2.0], requires_grad=True))
    assert seen["flags"] == (False, True)


def test_deep_chain_has_no_recursion_limit():
    x = T([1.0], requires_grad=True)
    y = x
    for _ in range(5000):
        y = Scale.apply(y, 1.0)
    backward(y, ones_like(y))
    np.testing.assert_allclose(x.grad._data, [1.0])


class _Sized(np.ndarray):
    """A NumPy array with the native tensor's numel()."""

    def numel(self):
        return self.size


def test_non_scalar_root_needs_grad_output():
    x = T([1.0, 2.0], requires_grad=True)
    y = Scale.apply(x, 2.0)
    y._data = np.asarray(y._data).view(_Sized)
    with pytest.raises(RuntimeError, match="grad_output"):
        backward(y)
    assert x.grad is None
