"""GPU checks of the tensor-runtime kernels behind the host Tensor:
strided copy (bit-exact vs numpy's view semantics), fill, elementwise
add/sub/mul (bit-exact: one IEEE operation per element), randn (moments,
reproducibility) and the deterministic full sum."""
import numpy as np
import pytest

from tests.gpu_util import dev, host, require_gpu, say

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    require_gpu()


def ops():
    import cudeep_amd.ops as o
    return o


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_strided_copy_views(dtype):
    rng = np.random.default_rng(1)
    x = rng.standard_normal((5, 6, 7, 3)).astype(dtype)
    dx = dev(x)
    for perm in [(1, 0, 2, 3), (3, 2, 1, 0), (0, 2, 1, 3)]:
        say("strided copy", perm, dtype.__name__)
        got = host(ops().strided_copy(dx.permute(*perm)))
        assert np.array_equal(got, np.ascontiguousarray(x.transpose(perm)))
    got = host(ops().strided_copy(dx[1:4, ::2, 3:, :]))
    assert np.array_equal(got, np.ascontiguousarray(x[1:4, ::2, 3:, :]))


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_fill_binary(dtype):
    import torch
    import cudeep_amd as cd
    rng = np.random.default_rng(2)
    a = rng.standard_normal(1001).astype(dtype)
    b = rng.standard_normal(1001).astype(dtype)
    da, db = dev(a), dev(b)
    say("binary", dtype.__name__)
    assert np.array_equal(host(ops().binary(cd._lib.BINARY_ADD, da, db)), a + b)
    assert np.array_equal(host(ops().binary(cd._lib.BINARY_SUB, da, db)), a - b)
    assert np.array_equal(host(ops().binary(cd._lib.BINARY_MUL, da, db)), a * b)
    t = torch.empty(777, device="cuda", dtype=torch.float32 if dtype == np.float32 else torch.float64)
    assert np.array_equal(host(ops().fill(t, 3.25)), np.full(777, 3.25, dtype))


def test_randn_moments_and_reproducibility():
    import torch
    say("randn")
    a = host(ops().randn((1 << 20,), seed=7))
    b = host(ops().randn((1 << 20,), seed=7))
    c = host(ops().randn((1 << 20,), seed=8))
    assert np.array_equal(a, b) and not np.array_equal(a, c)
    assert abs(a.mean()) < 5e-3 and abs(a.std() - 1) < 5e-3
    assert abs(((a - a.mean()) ** 3).mean()) < 2e-2           # skew ~ 0
    assert abs(((a ** 4).mean()) - 3.0) < 5e-2                 # kurtosis ~ 3
    d = host(ops().randn((1001,), dtype=torch.float64, seed=3, offset=10))
    assert np.isfinite(d).all() and d.dtype == np.float64
    # offset shifts the stream by whole pairs
    e = host(ops().randn((40,), seed=5, offset=0))
    f = host(ops().randn((20,), seed=5, offset=10))
    assert np.array_equal(e[20:], f)


@pytest.mark.parametrize("n", [0, 1, 255, 100003, 3000000])
def test_total_sum(n):
    rng = np.random.default_rng(n)
    x = rng.integers(-1000, 1000, n).astype(np.float32)
    say("sum", n)
    got = host(ops().total_sum(dev(x)))[0]
    assert got == np.float32(x.astype(np.float64).sum())
    y = rng.standard_normal(n)
    got = host(ops().total_sum(dev(y)))[0]
    assert abs(got - y.sum()) <= 1e-12 * max(1.0, np.abs(y).sum())
