"""GPU parity of the Linear path (C4: MLP 784 -> 256 -> 10, batch 8192).

The reference's nn.Linear forward is matmul(x, W^T) + broadcast bias, then
the activation module (python/cuDeep/nn.py:110-115); backward is
dX = dY W, dW = dY^T X, db = column sums of dY (tensor.py:430-443,
:617-631).  Here the forward is one fused GEMM (bias + ReLU epilogue) and
the backward uses transposed-operand GEMMs.  Gate: relFro vs fp64 <= 2 x
the error of the reference route restated on the CPU (seq-FMA SGEMM, then
one fp32 bias add, then the activation).
"""
import numpy as np
import pytest

import oracle
from tests.gpu_util import dev, host, normal, require_gpu, say

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    require_gpu()


def ops():
    import cudeep_amd.ops as o
    return o


def xavier(rng, fan_out, fan_in):
    bound = np.sqrt(6.0 / (fan_in + fan_out))    # init.py:28-40, gain 1
    return rng.uniform(-bound, bound, (fan_out, fan_in)).astype(np.float32)


@pytest.fixture(scope="module")
def mlp():
    rng = np.random.default_rng(4040)
    X = normal(rng, (8192, 784))
    W1 = xavier(rng, 256, 784)
    W2 = xavier(rng, 10, 256)
    b1 = normal(rng, (256,), 0.1)
    b2 = normal(rng, (10,), 0.1)
    dY2 = normal(rng, (8192, 10))
    return X, W1, b1, W2, b2, dY2


def _ref_route_linear(x, W, b, act, prec=0):
    """The reference's Linear route on the CPU: GEMM (seq-FMA for FP32, the
    emulated TF32 kernel for TF32 mode), one fp32 bias add, activation."""
    if prec == 0:
        z = oracle.sgemm_seqfma(x, W, transB=True)
    else:
        z = oracle.gemm_tf32emu(x, np.ascontiguousarray(W.T), "rne")
    z = (z + b[None, :]).astype(np.float32)
    if act == "relu":
        z = np.maximum(z, np.float32(0))
    return z


@pytest.mark.parametrize("prec", [0, 1])
def test_mlp_forward_fused(mlp, prec):
    import cudeep_amd as cd
    X, W1, b1, W2, b2, _ = mlp
    say("C4 forward prec", prec)
    dX, dW1, db1, dW2, db2 = map(dev, (X, W1, b1, W2, b2))
    H = ops().gemm(dX, dW1, transB=True, bias=db1, bias_mode=cd.BIAS_COL,
                   epilogue=cd.EPI_RELU, precision=prec)
    Y = ops().gemm(H, dW2, transB=True, bias=db2, bias_mode=cd.BIAS_COL, precision=prec)
    H, Y = host(H), host(Y)
    H64 = oracle.relu(oracle.dgemm(X, W1, transB=True) + b1[None, :])
    e1 = oracle.rel_fro(H, H64)
    e1_ref = oracle.rel_fro(_ref_route_linear(X, W1, b1, "relu", prec), H64)
    # layer 2 judged on the GPU's own H (errors do not compound in the gate)
    Y64 = oracle.dgemm(H, W2, transB=True) + b2[None, :]
    e2 = oracle.rel_fro(Y, Y64)
    e2_ref = oracle.rel_fro(_ref_route_linear(H, W2, b2, None, prec), Y64)
    print(f"C4 fwd prec={prec}: L1 {e1:.3e} (ref {e1_ref:.3e})  L2 {e2:.3e} (ref {e2_ref:.3e})")
    if prec == 0:
        assert e1 <= 2 * e1_ref and e2 <= 2 * e2_ref
    else:
        assert e1 <= e1_ref and e2 <= e2_ref


@pytest.mark.parametrize("prec", [0, 1])
def test_mlp_backward(mlp, prec):
    import cudeep_amd as cd
    X, W1, b1, W2, b2, dY2 = mlp
    rng = np.random.default_rng(4041)
    dY1 = normal(rng, (8192, 256))
    say("C4 backward prec", prec)
    gX, gW1, gY1 = dev(X), dev(W1), dev(dY1)
    dX1 = host(ops().gemm(gY1, gW1, precision=prec))                    # dY W
    dW1 = host(ops().gemm(gY1, gX, transA=True, precision=prec))        # dY^T X
    db1 = host(ops().sum_reduce_rows(gY1))
    dX2 = host(ops().gemm(dev(dY2), dev(W2), precision=prec))           # K = 10
    dW2 = host(ops().gemm(dev(dY2), gY1, transA=True, precision=prec))  # M = 10
    cases = [
        ("dX1", dX1, dY1, W1, False), ("dW1", dW1, dY1, X, True),
        ("dX2", dX2, dY2, W2, False), ("dW2", dW2, dY2, dY1, True)]
    for name, got, a, bm, tA in cases:
        ref64 = oracle.dgemm(a, bm, transA=tA)
        e = oracle.rel_fro(got, ref64)
        e_ref = oracle.rel_fro(oracle.sgemm_seqfma(a, bm, transA=tA), ref64)
        print(f"C4 bwd prec={prec} {name}: {e:.3e} (ref {e_ref:.3e})")
        if prec == 0:
            assert e <= 2 * e_ref, name
        else:
            e_tf = oracle.rel_fro(oracle.gemm_tf32emu(
                np.ascontiguousarray(a.T if tA else a), bm, "rne"), ref64)
            assert e <= e_tf, name
    db64 = dY1.astype(np.float64).sum(0)
    e = oracle.rel_fro(db1, db64)
    e_ref = oracle.rel_fro(oracle.colsum(dY1), db64)
    assert e <= 2 * e_ref + 2.0 ** -24


def test_linear_kats(kats):
    import cudeep_amd as cd
    for name in ("linear_fixed_weight", "linear_identity_bias"):
        k = kats[name]
        say("linear kat", name)
        y = host(ops().gemm(dev(np.array(k["x"], np.float32)), dev(np.array(k["W"], np.float32)),
                            transB=True, bias=dev(np.array(k["b"], np.float32)),
                            bias_mode=cd.BIAS_COL))
        assert np.array_equal(y, np.array(k["y"], np.float32))


def test_autograd_kat_via_gemms(kats):
    """grads of sum(A @ B): dA = 1 B^T, dB = A^T 1 (test_autograd.py:85-94)."""
    k = kats["autograd_sum_matmul"]
    A = np.array(k["A"], np.float32)
    B = np.array(k["B"], np.float32)
    ones = np.ones((2, 2), np.float32)
    say("autograd kat")
    dA = host(ops().gemm(dev(ones), dev(B), transB=True))
    dB = host(ops().gemm(dev(A), dev(ones), transA=True))
    assert np.array_equal(dA, np.array(k["dA"], np.float32))
    assert np.array_equal(dB, np.array(k["dB"], np.float32))


@pytest.mark.parametrize("rows,cols", [(1, 1), (7, 3), (33, 65), (8192, 256), (8192, 10),
                                       (1000, 1000), (100003, 7), (0, 5)])
def test_sum_reduce_rows(rows, cols):
    rng = np.random.default_rng(rows + cols)
    x = rng.integers(-100, 100, (rows, cols)).astype(np.float32)
    say("colsum", rows, cols)
    got = host(ops().sum_reduce_rows(dev(x)))
    assert np.array_equal(got, x.astype(np.float64).sum(0).astype(np.float32))
    y = normal(rng, (rows, cols))
    got = host(ops().sum_reduce_rows(dev(y)))
    want = y.astype(np.float64).sum(0)
    if rows:
        e_ref = oracle.rel_fro(oracle.colsum(y), want)
        assert oracle.rel_fro(got, want) <= 2 * e_ref + 2.0 ** -24


@pytest.mark.parametrize("act", ["relu", "gelu", "silu", "sigmoid"])
def test_activations(act):
    import cudeep_amd as cd
    a = {"relu": cd.EPI_RELU, "gelu": cd.EPI_GELU, "silu": cd.EPI_SILU,
         "sigmoid": cd.EPI_SIGMOID}[act]
    x = np.linspace(-8, 8, 100003).astype(np.float32)
    go = np.random.default_rng(9).standard_normal(x.shape).astype(np.float32)
    say("activation", act)
    y = host(ops().activation(dev(x), a))
    g = host(ops().activation_backward(dev(go), dev(x), a))
    if act == "relu":
        assert np.array_equal(y, np.maximum(x, 0))
        assert np.array_equal(g, np.where(x > 0, go, 0).astype(np.float32))
    else:
        want = oracle.activation(x, act)
        assert np.max(np.abs(y - want) / np.maximum(np.abs(want), 1e-3)) < 2e-6
        wg = go * oracle.activation_grad(x, act)
        assert np.max(np.abs(g - wg)) < 1e-5 * max(1.0, np.abs(wg).max())


def test_broadcast_add_row():
    rng = np.random.default_rng(11)
    m = normal(rng, (300, 77))
    r = normal(rng, (77,))
    say("broadcast add")
    got = host(ops().broadcast_add_row(dev(m), dev(r)))
    assert np.array_equal(got, (m + r[None, :]).astype(np.float32))


# ---------------------------------------------------------------------------
# fused backward: activation-backward epilogue and bias-gradient column
# ---------------------------------------------------------------------------

BWD_ACTS = ["relu", "gelu", "silu", "sigmoid"]


@pytest.mark.parametrize("act", BWD_ACTS)
@pytest.mark.parametrize("shape", [(8192, 256, 10), (300, 200, 96), (64, 64, 4096)])
@pytest.mark.parametrize("prec", [0, 1])
def test_bwd_epilogue_equals_gemm_then_activation_backward(act, shape, prec):
    """dZ = (dY W) * act'(Z) in the GEMM's epilogue is bit for bit the GEMM
    followed by the reference's activation_backward kernel (the same float
    formula on the same product), unsplit, ragged and split-K; and against
    fp64 the fused result is inside the reference route's bar (relu_grad x
    dgemm: seq-FMA GEMM then the mask)."""
    import cudeep_amd as cd
    M, N, K = shape
    rng = np.random.default_rng(M + N + K + prec)
    dY = normal(rng, (M, K))
    W = normal(rng, (K, N), 1.0 / np.sqrt(K))
    Z = normal(rng, (M, N))
    code = {"relu": cd.EPI_BWD_RELU, "gelu": cd.EPI_BWD_GELU, "silu": cd.EPI_BWD_SILU,
            "sigmoid": cd.EPI_BWD_SIGMOID}[act]
    fwd_code = {"relu": cd.EPI_RELU, "gelu": cd.EPI_GELU, "silu": cd.EPI_SILU,
                "sigmoid": cd.EPI_SIGMOID}[act]
    say("bwd epilogue", act, shape, prec)
    gY, gW, gZ = dev(dY), dev(W), dev(Z)
    fused = host(ops().gemm(gY, gW, precision=prec, epilogue=code, aux=gZ))
    P = ops().gemm(gY, gW, precision=prec)
    sep = host(ops().activation_backward(P, gZ, fwd_code))
    assert np.array_equal(fused.view(np.uint32), sep.view(np.uint32))
    if act == "relu":
        want = oracle.dgemm(dY, W) * oracle.relu_grad(Z)
        e = oracle.rel_fro(fused, want)
        if prec == 0:
            e_ref = oracle.rel_fro(oracle.sgemm_seqfma(dY, W) * (Z > 0), want)
            assert e <= 2 * e_ref, (e, e_ref)
        else:
            e_ref = min(oracle.rel_fro(oracle.gemm_tf32emu(dY, W, m) * (Z > 0), want)
                        for m in ("rz", "rne"))
            assert e <= e_ref, (e, e_ref)


@pytest.mark.parametrize("M,N,K", [(256, 784, 8192), (10, 256, 8192), (33, 17, 3001),
                                   (300, 200, 96), (64, 63, 128)])
@pytest.mark.parametrize("prec", [0, 1])
def test_weight_grad_with_fused_bias_grad(M, N, K, prec):
    """dW = dZ^T X with db = column sums of dZ from the same launch (a virtual
    column of ones appended to X): dW inside the FP32 bar against fp64 (the
    fused call runs exact FP32 products in every mode), db inside 2x the
    serial fp32 column sum's error, and the workspace query covers it."""
    import torch
    rng = np.random.default_rng(7 * M + N + K)
    dZ = normal(rng, (K, M))
    X = normal(rng, (K, N))
    say("fused bias grad", M, N, K, prec)
    cs = torch.full((M,), float("nan"), device="cuda")
    nbytes = ops().gemm_workspace_bytes(M, N, K, precision=prec, transA=True, colsum=True)
    ws = torch.empty(nbytes // 4 + 1, dtype=torch.float32, device="cuda")
    dW = host(ops().gemm(dev(dZ), dev(X), transA=True, precision=prec, colsum=cs,
                         workspace=ws))
    db = host(cs)
    want = oracle.dgemm(dZ, X, transA=True)
    e_ref = oracle.rel_fro(oracle.sgemm_seqfma(dZ, X, transA=True), want)
    assert oracle.rel_fro(dW, want) <= 2 * e_ref + 2.0 ** -24
    db64 = dZ.astype(np.float64).sum(0)
    eb = oracle.rel_fro(db, db64)
    eb_ref = oracle.rel_fro(oracle.colsum(dZ), db64)
    assert eb <= 2 * eb_ref + 2.0 ** -24, (eb, eb_ref)
    # the same FP32 product without the column has the same tiles and k-slices
    # when the extra column needs no extra 64-wide tile: then dW is identical
    if prec == 0 and N > 16 and (N + 63) // 64 == (N + 64) // 64:
        plain = host(ops().gemm(dev(dZ), dev(X), transA=True))
        assert np.array_equal(plain.view(np.uint32), dW.view(np.uint32))


@pytest.mark.parametrize("M,N,K,transA", [(1, 100, 5000, True), (16, 4096, 1024, False),
                                          (7, 33, 2049, True), (12, 520, 70000, True),
                                          (16, 64, 1024, False), (10, 257, 8191, True),
                                          (5, 37, 3001, False), (4, 100, 2048, True),
                                          (8, 64, 1500, False), (13, 129, 1024, True)])
@pytest.mark.parametrize("prec", [0, 1])
def test_skinny_m_long_k(M, N, K, transA, prec):
    """M <= 16 with K >= 1024 (the 10-wide layer's weight-gradient shape): the
    split-K FMA kernel (its row count M rounded up to 4, 8, 12 or 16, each
    with M at and off the boundary) and its slice reduction -- ragged and
    unaligned widths, op(A) either way, the slice cap (K = 70000), with the ones
    column (bias gradient) on a caller workspace, and with a bias + ReLU
    epilogue applied by the reduction."""
    import torch
    import cudeep_amd as cd
    rng = np.random.default_rng(131 * M + N + K)
    A = normal(rng, (K, M) if transA else (M, K))
    B = normal(rng, (K, N))
    bias = normal(rng, (N,))
    say("skinny M", M, N, K, transA, prec)
    want = oracle.dgemm(A, B, transA=transA)
    e_ref = oracle.rel_fro(oracle.sgemm_seqfma(A, B, transA=transA), want)
    nbytes = ops().gemm_workspace_bytes(M, N, K, precision=prec, transA=transA, colsum=True)
    assert nbytes > 0
    ws = torch.empty(nbytes // 4, dtype=torch.float32, device="cuda")
    cs = torch.full((M,), float("nan"), device="cuda")
    C = host(ops().gemm(dev(A), dev(B), transA=transA, precision=prec, colsum=cs, workspace=ws))
    assert oracle.rel_fro(C, want) <= 2 * e_ref + 2.0 ** -24
    opA = A.T if transA else A                       # [M, K]
    db64 = opA.astype(np.float64).sum(1)
    eb_ref = oracle.rel_fro(oracle.colsum(np.ascontiguousarray(opA.T)), db64)
    assert oracle.rel_fro(host(cs), db64) <= 2 * eb_ref + 2.0 ** -24
    Y = host(ops().gemm(dev(A), dev(B), transA=transA, precision=prec, bias=dev(bias),
                        bias_mode=cd.BIAS_COL, epilogue=cd.EPI_RELU))
    ref = np.maximum(want + bias, 0.0)
    # ReLU is 1-Lipschitz: the error stays within the product's (+ the bias add's rounding)
    assert np.linalg.norm(Y - ref) <= (2 * e_ref + 2.0 ** -23) * np.linalg.norm(want + bias)


@pytest.mark.parametrize("act", BWD_ACTS)
@pytest.mark.parametrize("M,N,K", [(10, 256, 8192), (5, 37, 3001), (16, 1030, 1024)])
@pytest.mark.parametrize("prec", [0, 1])
def test_skinny_m_bwd_epilogue(act, M, N, K, prec):
    """The skinny-M route (M <= 16, K >= 1024: a Linear input gradient
    dH = (dZ W) * act'(H) at a batch of <= 16) with an activation-backward
    epilogue, which its slice reduction applies: bit for bit the same
    product followed by the elementwise activation-backward kernel, with
    ragged widths and aux a view whose leading dimension exceeds N."""
    import cudeep_amd as cd
    rng = np.random.default_rng(17 * M + N + K + prec)
    A = normal(rng, (M, K))
    B = normal(rng, (K, N), 1.0 / np.sqrt(K))
    Zwide = normal(rng, (M, N + 7))
    code = {"relu": cd.EPI_BWD_RELU, "gelu": cd.EPI_BWD_GELU, "silu": cd.EPI_BWD_SILU,
            "sigmoid": cd.EPI_BWD_SIGMOID}[act]
    fwd_code = {"relu": cd.EPI_RELU, "gelu": cd.EPI_GELU, "silu": cd.EPI_SILU,
                "sigmoid": cd.EPI_SIGMOID}[act]
    say("skinny M bwd epilogue", act, M, N, K, prec)
    gA, gB = dev(A), dev(B)
    aux = dev(Zwide)[:, :N]
    assert aux.stride(0) == N + 7
    fused = host(ops().gemm(gA, gB, precision=prec, epilogue=code, aux=aux))
    P = ops().gemm(gA, gB, precision=prec)
    sep = host(ops().activation_backward(P, dev(np.ascontiguousarray(Zwide[:, :N])), fwd_code))
    assert np.array_equal(fused.view(np.uint32), sep.view(np.uint32))
    if act == "relu":
        want = oracle.dgemm(A, B) * oracle.relu_grad(Zwide[:, :N])
        e_ref = oracle.rel_fro(oracle.sgemm_seqfma(A, B) * (Zwide[:, :N] > 0), want)
        assert oracle.rel_fro(fused, want) <= 2 * e_ref + 2.0 ** -24


def test_fused_bias_grad_k_zero_and_empty_columns():
    """K = 0: dW = 0 and db = 0; N = 0: only db."""
    import torch
    say("fused bias grad edge cases")
    cs = torch.full((5,), float("nan"), device="cuda")
    out = host(ops().gemm(torch.empty((0, 5), device="cuda"), torch.empty((0, 3), device="cuda"),
                          transA=True, colsum=cs))
    assert not out.any() and not host(cs).any()
    dZ = np.random.default_rng(3).standard_normal((40, 5)).astype(np.float32)
    cs2 = torch.full((5,), float("nan"), device="cuda")
    ops().gemm(dev(dZ), torch.empty((40, 0), device="cuda"), transA=True, colsum=cs2)
    np.testing.assert_allclose(host(cs2), dZ.astype(np.float64).sum(0), rtol=1e-5, atol=1e-5)
