"""The drop-in Python surface on the GPU: cuDeep.Tensor / nn / init over
the native _cudeep_core module, written like the reference's own tests
(tests/unit/test_tensor_ops.py:210-262, test_autograd.py:85-231,
test_nn.py:29-118, test_layers.py:58-75) plus oracle gates on the fused
Linear / Conv2d paths."""
import numpy as np
import pytest

import oracle
from tests.gpu_util import require_gpu, say

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def cd():
    require_gpu()
    from cudeep_amd import cuDeep
    return cuDeep


@pytest.fixture(autouse=True)
def _precision(cd):
    prev = cd.get_matmul_precision()
    yield
    cd.set_matmul_precision(prev)


# ---- Tensor basics ---------------------------------------------------------

def test_tensor_factories_and_views(cd):
    T = cd.Tensor
    say("tensor basics")
    assert np.array_equal(T.zeros([2, 3]).numpy(), np.zeros((2, 3), np.float32))
    assert np.array_equal(T.ones([4]).numpy(), np.ones(4, np.float32))
    assert T.full([2, 2], 3.5).numpy().tolist() == [[3.5, 3.5], [3.5, 3.5]]
    x = np.arange(24, dtype=np.float32).reshape(2, 3, 4)
    t = T.from_numpy(x)
    assert t.shape() == [2, 3, 4] and t.dtype() == cd.DType.float32
    assert np.array_equal(t.reshape(6, 4).numpy(), x.reshape(6, 4))
    assert np.array_equal(t.reshape([4, -1]).numpy(), x.reshape(4, 6))
    tt = t.transpose(0, 2)
    assert not tt.is_contiguous()
    assert np.array_equal(tt.numpy(), x.transpose(2, 1, 0))
    assert np.array_equal(tt.contiguous().numpy(), x.transpose(2, 1, 0))
    a = np.random.default_rng(0).standard_normal((5, 7)).astype(np.float32)
    b = np.random.default_rng(1).standard_normal((5, 7)).astype(np.float32)
    A, B = T.from_numpy(a), T.from_numpy(b)
    assert np.array_equal((A + B).numpy(), a + b)
    assert np.array_equal((A - B).numpy(), a - b)
    assert np.array_equal((A * B).numpy(), a * b)
    d = T.from_numpy(np.arange(6, dtype=np.float64))
    assert d.dtype() == cd.DType.float64 and d.numpy().dtype == np.float64
    r = T.randn([1000, 100]).numpy()
    assert abs(r.mean()) < 0.02 and abs(r.std() - 1) < 0.02
    assert T.from_numpy(np.array([[1.0, 2.0]], np.float32)).sum().item() == 3.0


def test_memory_pool_and_events(cd):
    say("pool/events")
    pool = cd.MemoryPool.instance()
    before = pool.allocated_bytes
    t = cd.Tensor.zeros([1024, 1024])
    assert pool.allocated_bytes >= before + 4 * 1024 * 1024
    del t
    assert pool.cached_bytes >= 4 * 1024 * 1024
    s = cd.Stream()
    e0, e1 = cd.Event(), cd.Event()
    e0.record(s)
    e1.record(s)
    e1.synchronize()
    assert e1.elapsed_ms(e0) >= 0.0
    info = cd.device_info()
    assert info["multiprocessors"] > 0 and "gfx950" in info["arch"]


# ---- matmul (reference tests/unit/test_tensor_ops.py:210-262) --------------

@pytest.mark.parametrize("prec", ["tf32", "fp32", "tf32x4"])
def test_matmul_reference_cases(cd, prec):
    cd.set_matmul_precision(prec)
    T = cd.Tensor
    say("matmul cases", prec)
    a = T.from_numpy(np.array([[1, 2], [3, 4]], np.float32))
    b = T.from_numpy(np.array([[5, 6], [7, 8]], np.float32))
    assert np.array_equal(a.matmul(b).numpy(), [[19, 22], [43, 50]])
    rng = np.random.default_rng(80)
    x = rng.standard_normal((64, 64)).astype(np.float32)
    out = T.from_numpy(x).matmul(T.from_numpy(np.eye(64, dtype=np.float32))).numpy()
    np.testing.assert_allclose(out, x, rtol=1e-5)
    # The reference's tolerances (test_tensor_ops.py:229-247) hold for FP32.  In
    # the split modes each product may be off by 2^-15 |ab| (bf16x3) or 2^-16
    # |ab| (bf16x4), so near-cancelling outputs are checked against that bound.
    per_product = {"fp32": 0.0, "tf32": 2.0 ** -15, "tf32x4": 2.0 ** -16}[prec]
    for (m, k, n), rtol, atol in (((3, 5, 7), 1e-4, 1e-5), ((64, 128, 32), 1e-3, 1e-3)):
        a = rng.standard_normal((m, k)).astype(np.float32)
        b = rng.standard_normal((k, n)).astype(np.float32)
        got = (T.from_numpy(a) @ T.from_numpy(b)).numpy()
        ref = a.astype(np.float64) @ b
        bound = per_product * (np.abs(a).astype(np.float64) @ np.abs(b)) + 2.0 ** -22 * np.abs(ref)
        assert np.all(np.abs(got - ref) <= np.maximum(atol + rtol * np.abs(ref), bound))


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_core_activations_vs_oracle(cd, dtype):
    """_cudeep_core relu / gelu / sigmoid / silu / tanh_act / leaky_relu and
    activation_backward (reference module.cpp:185-207, :837-872) against the
    fp64 oracle."""
    from cudeep_amd.cuDeep import _core
    x = np.linspace(-12, 12, 4099).astype(dtype)
    go = np.random.default_rng(3).standard_normal(x.shape).astype(dtype)
    # fp64: the oracle's GELU is the reference's 0.5 x (1 + tanh(u)), whose
    # 1 + tanh(u) cancels for x << 0 (absolute error ~ |x| 2^-53), so the
    # gate is a few 1e-12 against the 1e-3 floor
    tol = 2e-6 if dtype == np.float32 else 5e-12
    for name in ("relu", "gelu", "sigmoid", "silu", "tanh", "leaky_relu"):
        say("core activation", name, dtype.__name__)
        fwd = _core.tanh_act if name == "tanh" else getattr(_core, name)
        y = fwd(_core.Tensor.from_numpy(x)).numpy()
        want = oracle.activation(x, name)
        assert y.dtype == dtype
        assert np.max(np.abs(y - want) / np.maximum(np.abs(want), 1e-3)) < tol, name
        g = _core.activation_backward(_core.Tensor.from_numpy(go), _core.Tensor.from_numpy(x),
                                      name).numpy()
        wg = go * oracle.activation_grad(x, name)
        assert np.max(np.abs(g - wg)) < 5 * tol * max(1.0, np.abs(wg).max()), name


def test_matmul_float64_and_transposed_views(cd):
    T = cd.Tensor
    say("matmul f64 / views")
    a = np.random.randn(33, 17)
    b = np.random.randn(17, 9)
    np.testing.assert_allclose((T.from_numpy(a) @ T.from_numpy(b)).numpy(), a @ b, rtol=1e-12)
    # transposed operands are consumed as views (no copy), results identical
    cd.set_matmul_precision("fp32")
    w = np.random.randn(40, 30).astype(np.float32)
    x = np.random.randn(20, 30).astype(np.float32)
    got = T.from_numpy(x).matmul(T.from_numpy(w).t()).numpy()
    C64 = x.astype(np.float64) @ w.T.astype(np.float64)
    e_ref = oracle.rel_fro(oracle.sgemm_seqfma(x, w, transB=True), C64)
    assert oracle.rel_fro(got, C64) <= 2 * e_ref + 2.0 ** -24
    got2 = T.from_numpy(w).matmul(T.from_numpy(x).t()).numpy()          # W x^T
    assert oracle.rel_fro(got2, C64.T) <= 2 * e_ref + 2.0 ** -24
    xt = T.from_numpy(np.ascontiguousarray(x.T))                          # A as a view
    got3 = xt.t().matmul(T.from_numpy(w).t()).numpy()
    assert oracle.rel_fro(got3, C64) <= 2 * e_ref + 2.0 ** -24


def test_native_entry_points_reject_unsupported_dtypes(cd):
    """matmul_ex takes float32 or float64 operands and linear_forward a
    float32 bias; anything else is refused on the host before a launch."""
    from cudeep_amd.cuDeep import _core
    say("dtype checks")
    h = _core.Tensor([4, 4], _core.DType.float16)
    f = _core.Tensor.zeros([4, 4], _core.DType.float32)
    with pytest.raises(RuntimeError, match="float32 or float64"):
        _core.matmul_ex(h, h, False, False)
    with pytest.raises(RuntimeError, match="float32 or float64"):
        _core.matmul_ex(f, h, False, False)
    b64 = _core.Tensor.zeros([4], _core.DType.float64)
    with pytest.raises(RuntimeError, match="linear_forward"):
        _core.linear_forward(f, f, b64, "none")
    out = _core.linear_forward(f, f, _core.Tensor.zeros([4], _core.DType.float32), "relu")
    assert out.numpy().shape == (4, 4)


# ---- autograd (reference tests/unit/test_autograd.py) ----------------------

def test_matmul_grad_kat(cd, kats):
    k = kats["autograd_sum_matmul"]
    T = cd.Tensor
    say("autograd kat")
    a = T.from_numpy(np.array(k["A"], np.float32), requires_grad=True)
    b = T.from_numpy(np.array(k["B"], np.float32), requires_grad=True)
    a.matmul(b).sum().backward()
    assert np.array_equal(a.grad.numpy(), np.array(k["dA"], np.float32))
    assert np.array_equal(b.grad.numpy(), np.array(k["dB"], np.float32))


def test_chain_rule_and_accumulation(cd):
    T = cd.Tensor
    say("chain rule")
    a = T.from_numpy(np.array([2.0], np.float32), requires_grad=True)
    (((a * 3.0) + 1.0) * 2.0).sum().backward()
    np.testing.assert_allclose(a.grad.numpy(), [6.0])
    w = T.from_numpy(np.array([[1.0, 2.0]], np.float32), requires_grad=True)
    x1 = T.from_numpy(np.array([[1.0, 0.0]], np.float32))
    w.matmul(x1.t()).sum().backward()
    assert np.array_equal(w.grad.numpy(), [[1.0, 0.0]])
    w.matmul(x1.t()).sum().backward()           # accumulates
    assert np.array_equal(w.grad.numpy(), [[2.0, 0.0]])
    with cd.no_grad():
        y = w.matmul(x1.t())
    assert y._grad_fn is None


def test_broadcast_add_grad(cd):
    T = cd.Tensor
    say("broadcast add grad")
    mat = T.from_numpy(np.zeros((3, 4), np.float32), requires_grad=True)
    row = T.from_numpy(np.zeros(4, np.float32), requires_grad=True)
    cd.broadcast_add(mat, row).sum().backward()
    np.testing.assert_allclose(mat.grad.numpy(), np.ones((3, 4)))
    np.testing.assert_allclose(row.grad.numpy(), [3, 3, 3, 3])


# ---- nn.Linear / Sequential (reference tests/unit/test_nn.py) --------------

def test_linear_reference_cases(cd, kats):
    nn, T = cd.nn, cd.Tensor
    say("linear cases")
    layer = nn.Linear(10, 5)
    assert len(layer.parameters()) == 2
    assert layer._parameters["weight"].shape() == [5, 10]
    assert len(nn.Linear(10, 5, bias=False).parameters()) == 1
    assert nn.Linear(8, 4)(T.randn([2, 8])).shape() == [2, 4]
    for name in ("linear_fixed_weight", "linear_identity_bias"):
        k = kats[name]
        layer = nn.Linear(len(k["W"][0]), len(k["W"]))
        layer._parameters["weight"] = T.from_numpy(np.array(k["W"], np.float32))
        layer._parameters["bias"] = T.from_numpy(np.array(k["b"], np.float32))
        assert np.array_equal(layer(T.from_numpy(np.array(k["x"], np.float32))).numpy(),
                              np.array(k["y"], np.float32))
    l64 = nn.Linear(4, 3, dtype=cd.DType.float64)
    out = l64(T.randn([1, 4], cd.DType.float64))
    assert out.shape() == [1, 3] and out.dtype() == cd.DType.float64
    model = nn.Sequential(nn.Linear(784, 256), nn.Linear(256, 128), nn.Linear(128, 10))
    assert model(T.randn([8, 784])).shape() == [8, 10] and len(model.parameters()) == 6


@pytest.mark.parametrize("prec", ["fp32", "tf32"])
def test_mlp_c4_forward_backward_vs_oracle(cd, prec):
    """C4 through the drop-in API: Sequential(Linear(784,256), ReLU,
    Linear(256,10)), batch 8192, Xavier-uniform weights, loss = sum(y * g)
    so dY = g.  Every gradient is gated against fp64 closed forms."""
    nn, T, init = cd.nn, cd.Tensor, cd.init
    cd.set_matmul_precision(prec)
    np.random.seed(7)
    model = nn.Sequential(nn.Linear(784, 256), nn.ReLU(), nn.Linear(256, 10))
    init.xavier_uniform_(model[0]._parameters["weight"])
    init.xavier_uniform_(model[2]._parameters["weight"])
    b1 = (np.random.randn(256) * 0.1).astype(np.float32)
    b2 = (np.random.randn(10) * 0.1).astype(np.float32)
    model[0]._parameters["bias"] = nn.Parameter(T.from_numpy(b1))
    model[2]._parameters["bias"] = nn.Parameter(T.from_numpy(b2))
    W1 = model[0]._parameters["weight"].numpy()
    W2 = model[2]._parameters["weight"].numpy()
    bound1 = np.sqrt(6.0 / (784 + 256))
    assert np.abs(W1).max() <= bound1 and np.abs(W1).max() > 0.95 * bound1
    x = np.random.randn(8192, 784).astype(np.float32)
    g = np.random.randn(8192, 10).astype(np.float32)
    say("C4 via cuDeep.nn", prec)
    X = T.from_numpy(x, requires_grad=True)
    y = model(X)
    (y * T.from_numpy(g)).sum().backward()
    # fp64 closed forms
    z1 = x.astype(np.float64) @ W1.T.astype(np.float64) + b1
    h = np.maximum(z1, 0)
    y64 = h @ W2.T.astype(np.float64) + b2
    dh = g.astype(np.float64) @ W2.astype(np.float64)
    dz1 = dh * (z1 > 0)
    want = {"y": y64, "dW2": g.T.astype(np.float64) @ h, "db2": g.sum(0),
            "dW1": dz1.T @ x.astype(np.float64), "db1": dz1.sum(0),
            "dX": dz1 @ W1.astype(np.float64)}
    got = {"y": y.numpy(), "dW2": model[2]._parameters["weight"].grad.numpy(),
           "db2": model[2]._parameters["bias"].grad.numpy(),
           "dW1": model[0]._parameters["weight"].grad.numpy(),
           "db1": model[0]._parameters["bias"].grad.numpy(), "dX": X.grad.numpy()}
    # tolerance: 2x the fp32 seq-FMA error of the same product class (K up
    # to 8192) -- a few 1e-6; TF32 mode (bf16x3) stays well inside 1e-4.
    tol = 2e-5 if prec == "fp32" else 1e-4
    for kname in want:
        e = oracle.rel_fro(got[kname], want[kname])
        print(f"C4 api {prec} {kname}: relFro {e:.2e}")
        assert e < tol, kname


@pytest.mark.parametrize("act", ["relu", "gelu"])
@pytest.mark.parametrize("prec", ["fp32", "tf32"])
def test_activation_backward_fused_into_consumer_gemm(cd, act, prec, monkeypatch):
    """A Linear whose input came out of a ReLU / GELU forms its input
    gradient with the activation derivative in its GEMM epilogue, and the
    activation's own backward launch is skipped (the reference runs it as a
    kernel of its own: tensor.py:430-443, activation_kernel.cu:256-319).
    Every parameter and input gradient is bit for bit the unfused one, with
    ragged sizes and three layers; an activation output feeding two layers
    keeps its own backward (applied to the summed gradient)."""
    from cudeep_amd.cuDeep import autograd
    from cudeep_amd.cuDeep import tensor as tmod
    nn, T = cd.nn, cd.Tensor
    cd.set_matmul_precision(prec)
    rng = np.random.default_rng(11 if act == "relu" else 12)
    dims = [300, 200, 96, 10]
    params = []
    for fi, fo in zip(dims[:-1], dims[1:]):
        params.append(((rng.standard_normal((fo, fi)) / np.sqrt(fi)).astype(np.float32),
                       (rng.standard_normal(fo) * 0.1).astype(np.float32)))
    x = rng.standard_normal((517, 300)).astype(np.float32)
    g = rng.standard_normal((517, 10)).astype(np.float32)
    calls = []
    real = tmod._activation_backward

    def counting(*args):
        calls.append(args[2])
        return real(*args)

    monkeypatch.setattr(tmod, "_activation_backward", counting)
    Act = nn.ReLU if act == "relu" else nn.GELU

    def linear(i):
        layer = nn.Linear(dims[i], dims[i + 1])
        layer._parameters["weight"] = nn.Parameter(T.from_numpy(params[i][0]))
        layer._parameters["bias"] = nn.Parameter(T.from_numpy(params[i][1]))
        return layer

    def run(fuse):
        autograd.set_fuse_activation_backward(fuse)
        try:
            calls.clear()
            model = nn.Sequential(linear(0), Act(), linear(1), Act(), linear(2))
            X = T.from_numpy(x, requires_grad=True)
            model(X).backward(T.from_numpy(g))
            grads = [X.grad.numpy()]
            for p in model.parameters():
                grads.append(p.grad.numpy())
            return grads, len(calls)
        finally:
            autograd.set_fuse_activation_backward(True)

    say("fused activation backward", act, prec)
    fused, n_fused = run(True)
    plain, n_plain = run(False)
    assert (n_fused, n_plain) == (0, 2)
    assert len(fused) == 7
    for a, b in zip(fused, plain):
        assert a.dtype == np.float32 and np.isfinite(a).all()
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))

    # two consumers of one activation output: no fusion, one backward launch
    calls.clear()
    l0, l1, l2 = linear(0), linear(1), nn.Linear(200, 96)
    l2._parameters["weight"] = nn.Parameter(T.from_numpy(params[1][0][::-1].copy()))
    X = T.from_numpy(x, requires_grad=True)
    h = Act()(l0(X)) if act == "gelu" else l0(X, activation="relu")
    out = l1(h) + l2(h)
    out.backward(T.from_numpy(g[:, :1].repeat(96, 1)))
    assert len(calls) == 1
    W0, b0 = params[0]
    z = x.astype(np.float64) @ W0.T.astype(np.float64) + b0
    dh = g[:, :1].repeat(96, 1).astype(np.float64) @ (params[1][0] + params[1][0][::-1]).astype(np.float64)
    if act == "relu":
        dz = dh * (z > 0)
    else:
        dz = dh * oracle.gelu_grad(z)
    assert oracle.rel_fro(l0._parameters["bias"].grad.numpy(), dz.sum(0)) < 1e-4


# ---- nn.Conv2d (reference tests/unit/test_layers.py:58-75) -----------------

def test_conv2d_layer_shapes(cd):
    nn, T = cd.nn, cd.Tensor
    say("conv shapes")
    assert nn.Conv2d(3, 16, kernel_size=3, padding=1)(T.randn([2, 3, 8, 8])).shape() == [2, 16, 8, 8]
    assert nn.Conv2d(1, 4, kernel_size=3)(T.randn([1, 1, 6, 6])).shape() == [1, 4, 4, 4]
    assert nn.Conv2d(1, 1, kernel_size=3, stride=2, padding=1)(T.randn([1, 1, 8, 8])).shape() == [1, 1, 4, 4]


@pytest.mark.parametrize("prec", ["fp32", "tf32"])
def test_conv2d_layer_forward_backward_vs_oracle(cd, prec):
    nn, T = cd.nn, cd.Tensor
    cd.set_matmul_precision(prec)
    rng = np.random.default_rng(3)
    layer = nn.Conv2d(8, 12, kernel_size=3, stride=1, padding=1)
    w = (rng.standard_normal((12, 8, 3, 3)) * np.sqrt(2 / 72)).astype(np.float32)
    b = (rng.standard_normal(12) * 0.1).astype(np.float32)
    layer._parameters["weight"] = nn.Parameter(T.from_numpy(w))
    layer._parameters["bias"] = nn.Parameter(T.from_numpy(b))
    x = rng.standard_normal((4, 8, 14, 14)).astype(np.float32)
    g = rng.standard_normal((4, 12, 14, 14)).astype(np.float32)
    say("conv layer", prec)
    X = T.from_numpy(x, requires_grad=True)
    y = layer(X)
    (y * T.from_numpy(g)).sum().backward()
    tol = 1e-5 if prec == "fp32" else 1e-4
    assert oracle.rel_fro(y.numpy(), oracle.conv2d_direct64(x, w, b, (1, 1), (1, 1))) < tol
    assert oracle.rel_fro(X.grad.numpy(),
                          oracle.conv2d_backward_data64(g, w, x.shape, (1, 1), (1, 1))) < tol
    assert oracle.rel_fro(layer._parameters["weight"].grad.numpy(),
                          oracle.conv2d_backward_weight64(g, x, w.shape, (1, 1), (1, 1))) < tol
    assert oracle.rel_fro(layer._parameters["bias"].grad.numpy(),
                          g.astype(np.float64).sum(axis=(0, 2, 3))) < 1e-5


def test_conv2d_layer_float64(cd):
    """nn.Conv2d on float64 tensors (the reference instantiates its conv
    launchers for double): forward and backward against the fp64 oracles on
    fp32-valued operands."""
    nn, T = cd.nn, cd.Tensor
    rng = np.random.default_rng(64)
    layer = nn.Conv2d(6, 10, kernel_size=3, stride=2, padding=1, dtype=cd.DType.float64)
    w = (rng.standard_normal((10, 6, 3, 3)) * np.sqrt(2 / 54)).astype(np.float32).astype(np.float64)
    b = (rng.standard_normal(10) * 0.1).astype(np.float32).astype(np.float64)
    layer._parameters["weight"] = nn.Parameter(T.from_numpy(w))
    layer._parameters["bias"] = nn.Parameter(T.from_numpy(b))
    x = rng.standard_normal((3, 6, 13, 12)).astype(np.float32).astype(np.float64)
    say("conv layer f64")
    X = T.from_numpy(x, requires_grad=True)
    y = layer(X)
    assert y.dtype() == cd.DType.float64
    g = rng.standard_normal(tuple(y.shape())).astype(np.float32).astype(np.float64)
    (y * T.from_numpy(g)).sum().backward()
    assert oracle.rel_fro(y.numpy(), oracle.conv2d_direct64(x, w, b, (2, 2), (1, 1))) < 1e-14
    assert oracle.rel_fro(X.grad.numpy(),
                          oracle.conv2d_backward_data64(g, w, x.shape, (2, 2), (1, 1))) < 1e-14
    assert oracle.rel_fro(layer._parameters["weight"].grad.numpy(),
                          oracle.conv2d_backward_weight64(g, x, w.shape, (2, 2), (1, 1))) < 1e-14
    assert oracle.rel_fro(layer._parameters["bias"].grad.numpy(), g.sum(axis=(0, 2, 3))) < 1e-14


def test_conv_algorithm_routing(cd):
    """launch_conv2d_forward_kernel routes like the reference
    (conv_kernel.cu:242-275): 3x3 stride-1 layers with >= 16 output pixels
    go to Winograd F(4x4, 3x3), the rest to im2col + GEMM (or the implicit
    GEMM beyond a 4 MiB column buffer); each can be forced.  Backward data
    follows the Winograd rule on its transposed conv."""
    from cudeep_amd.cuDeep import _core
    prev = cd.get_conv_algorithm()
    rng = np.random.default_rng(12)
    x = rng.standard_normal((2, 8, 14, 14)).astype(np.float32)
    w = (rng.standard_normal((12, 8, 3, 3)) * 0.15).astype(np.float32)
    b = (rng.standard_normal(12) * 0.1).astype(np.float32)
    X, W, Bv = (_core.Tensor.from_numpy(a) for a in (x, w, b))

    def run(algo, stride=(1, 1), pad=(1, 1), xt=X):
        cd.set_conv_algorithm(algo)
        return _core.conv2d_forward(xt, W, Bv, list(stride), list(pad)).numpy()
    try:
        cd.set_matmul_precision("fp32")
        say("conv routing")
        y_auto, y_wino, y_i2c = run("auto"), run("winograd"), run("im2col")
        assert np.array_equal(y_auto, y_wino)
        y64 = oracle.conv2d_direct64(x, w, b, (1, 1), (1, 1))
        e_w = oracle.rel_fro(oracle.conv2d_winograd(x, w, b, padding=(1, 1)), y64)
        e_i = oracle.rel_fro(oracle.conv2d_ref_im2col(x, w, b, (1, 1), (1, 1)), y64)
        assert oracle.rel_fro(y_wino, y64) <= 2 * e_w
        assert oracle.rel_fro(y_i2c, y64) <= 2 * e_i
        # stride 2: auto takes im2col, forcing Winograd is an error
        assert np.array_equal(run("auto", (2, 2)), run("im2col", (2, 2)))
        with pytest.raises(RuntimeError):
            run("winograd", (2, 2))
        # fewer than 16 output pixels per image: im2col
        small = _core.Tensor.from_numpy(x[:, :, :5, :5].copy())
        assert np.array_equal(run("auto", pad=(0, 0), xt=small), run("im2col", pad=(0, 0), xt=small))
        # forced implicit GEMM (the reference's route for large non-3x3 layers)
        y_imp = run("implicit")
        assert cd.get_conv_algorithm() == "implicit"
        e_imp = oracle.rel_fro(oracle.conv2d_ref_implicit(x, w, b, (1, 1), (1, 1)), y64)
        assert oracle.rel_fro(y_imp, y64) <= 2 * e_imp

        # backward data: the same rule on the transposed convolution in the
        # TF32 modes; FP32 keeps the GEMM route under auto
        g = rng.standard_normal((2, 12, 14, 14)).astype(np.float32)
        G = _core.Tensor.from_numpy(g)

        def run_bwd(algo, stride=(1, 1), pad=(1, 1), gt=G, shape=(2, 8, 14, 14)):
            cd.set_conv_algorithm(algo)
            return _core.conv2d_backward_data(gt, W, list(shape), list(stride), list(pad)).numpy()
        d_auto, d_wino, d_i2c = run_bwd("auto"), run_bwd("winograd"), run_bwd("im2col")
        assert np.array_equal(d_auto, d_i2c)
        d64 = oracle.conv2d_backward_data64(g, w, x.shape, (1, 1), (1, 1))
        e_w = oracle.rel_fro(oracle.conv2d_backward_data_winograd(g, w, x.shape, (1, 1)), d64)
        e_i = oracle.rel_fro(oracle.conv2d_backward_data_ref(g, w, x.shape, (1, 1), (1, 1)), d64)
        assert oracle.rel_fro(d_wino, d64) <= 2 * e_w
        assert oracle.rel_fro(d_i2c, d64) <= 2 * e_i
        cd.set_matmul_precision("tf32")
        assert np.array_equal(run_bwd("auto"), run_bwd("winograd"))
        assert not np.array_equal(run_bwd("auto"), run_bwd("im2col"))
        cd.set_matmul_precision("fp32")
        g2 = _core.Tensor.from_numpy(rng.standard_normal((2, 12, 7, 7)).astype(np.float32))
        assert np.array_equal(run_bwd("auto", (2, 2), gt=g2), run_bwd("im2col", (2, 2), gt=g2))
        with pytest.raises(RuntimeError):
            run_bwd("winograd", (2, 2), gt=g2)
    finally:
        cd.set_conv_algorithm(prev)


def test_init_distributions(cd):
    T, init = cd.Tensor, cd.init
    say("init")
    np.random.seed(0)
    w = init.kaiming_normal_(T.zeros([64, 64, 3, 3]))
    std = w.numpy().std()
    assert abs(std - np.sqrt(2.0 / 576)) < 0.002     # He-normal, C5 weights
    w = init.xavier_uniform_(T.zeros([256, 784])).numpy()
    bound = np.sqrt(6.0 / (784 + 256))
    assert np.abs(w).max() <= bound and abs(w.std() - bound / np.sqrt(3)) < 0.002
    assert np.array_equal(init.constant_(T.zeros([3]), 2.5).numpy(), [2.5, 2.5, 2.5])


def test_core_leaky_relu_slope(cd):
    """leaky_relu(x, alpha) and its backward with a non-default slope."""
    from cudeep_amd.cuDeep import _core
    x = np.linspace(-3, 3, 257).astype(np.float32)
    go = np.random.default_rng(5).standard_normal(x.shape).astype(np.float32)
    say("leaky relu slope")
    y = _core.leaky_relu(_core.Tensor.from_numpy(x), 0.2).numpy()
    assert np.array_equal(y, oracle.leaky_relu(x, 0.2).astype(np.float32))
    g = _core.activation_backward(_core.Tensor.from_numpy(go), _core.Tensor.from_numpy(x),
                                  "leaky_relu", 0.2).numpy()
    assert np.array_equal(g, (go * oracle.leaky_relu_grad(x, 0.2)).astype(np.float32))
