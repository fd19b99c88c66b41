"""Pins the CPU oracle before anything is checked against it.

Every oracle routine is checked against (i) the reference's own known-answer
tests (tests/golden/kats.json, from the reference's test files), and (ii)
facts the mathematics fixes independently of the oracle's code: exact
rational arithmetic on tiny inputs, closed forms, special cases that reduce
to a library routine (numpy / torch fp64), and hand-built inputs whose result
changes if a term is dropped, the order of accumulation changes, or the FMA
is split into a multiply and an add.
"""
from fractions import Fraction

import numpy as np
import pytest

import oracle


# ---------------------------------------------------------------------------
# exact rational helpers (independent of the C code)
# ---------------------------------------------------------------------------

def round_f32(q: Fraction) -> np.float32:
    """Correctly rounded (RNE) conversion of an exact rational to fp32."""
    if q == 0:
        return np.float32(0.0)
    sign = -1 if q < 0 else 1
    q = abs(q)
    e = q.numerator.bit_length() - q.denominator.bit_length()
    # normalise so that 2^e <= q < 2^(e+1)
    while Fraction(2) ** e > q:
        e -= 1
    while Fraction(2) ** (e + 1) <= q:
        e += 1
    e = max(e, -126)                      # subnormal range keeps exponent -126
    ulp = Fraction(2) ** (e - 23)
    n = q / ulp
    fl = n.numerator // n.denominator
    rem = n - fl
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2 == 1):
        fl += 1
    return np.float32(sign * float(fl * ulp))


def fma_f32(a, b, c) -> np.float32:
    return round_f32(Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c)))


# ---------------------------------------------------------------------------
# sequential-FMA SGEMM (matmul_kernel.cu:499-520)
# ---------------------------------------------------------------------------

def test_sgemm_kats(kats):
    k = kats["matmul_2x2"]
    C = oracle.sgemm_seqfma(np.array(k["A"], np.float32), np.array(k["B"], np.float32))
    assert np.array_equal(C, np.array(k["C"], np.float32))
    k = kats["matmul_diag_identity"]
    C = oracle.sgemm_seqfma(np.array(k["A"], np.float32), np.array(k["B"], np.float32))
    assert np.array_equal(C, np.array(k["C"], np.float32))
    k = kats["matmul_partial_identity"]
    C = oracle.sgemm_seqfma(np.array(k["A"], np.float32), np.array(k["B"], np.float32))
    assert np.array_equal(C[0], np.array(k["C_row0"], np.float32))
    k = kats["matmul_scaled_identity_8"]
    A = np.array(k["A"], np.float32)
    C = oracle.sgemm_seqfma(A, np.eye(8, dtype=np.float32))
    assert np.allclose(C, A, atol=k["atol"])
    for name in ("mma_identity", "mma_integer_pattern"):
        k = kats[name]
        C = oracle.sgemm_seqfma(np.array(k["A"], np.float32), np.array(k["B"], np.float32))
        assert np.array_equal(C, np.array(k["C"], np.float32)), name


def test_sgemm_is_fused_not_mul_add():
    # (1+2^-12)^2 - 1 = 2^-11 + 2^-24 exactly with one rounding (FMA);
    # a separate multiply rounds the product to 1+2^-11 first.
    a = np.float32(1 + 2.0 ** -12)
    A = np.array([[-1.0, a]], np.float32)
    B = np.array([[1.0], [a]], np.float32)
    C = oracle.sgemm_seqfma(A, B)
    assert C[0, 0] == np.float32(2.0 ** -11 + 2.0 ** -24)


def test_sgemm_accumulates_in_ascending_k():
    # acc: 1e8 -> 1e8 (+1 lost, ulp=8) -> 0 -> 1.  Any other order gives 0 or 2.
    A = np.array([[1e8, 1.0, -1e8, 1.0]], np.float32)
    B = np.ones((4, 1), np.float32)
    assert oracle.sgemm_seqfma(A, B)[0, 0] == np.float32(1.0)
    # reversed k order starting from the other end gives a different value
    assert oracle.sgemm_seqfma(A[:, ::-1].copy(), B)[0, 0] == np.float32(0.0)


@pytest.mark.parametrize("tA,tB", [(False, False), (False, True), (True, False), (True, True)])
def test_sgemm_matches_exact_fma_chain(tA, tB):
    rng = np.random.default_rng(7)
    M, N, K = 3, 5, 17
    A = rng.standard_normal((K, M) if tA else (M, K)).astype(np.float32)
    B = rng.standard_normal((N, K) if tB else (K, N)).astype(np.float32)
    opA = A.T if tA else A
    opB = B.T if tB else B
    C = oracle.sgemm_seqfma(A, B, transA=tA, transB=tB)
    for i in range(M):
        for j in range(N):
            acc = np.float32(0.0)
            for k in range(K):
                acc = fma_f32(opA[i, k], opB[k, j], acc)
            assert C[i, j] == acc, (i, j)


def test_sgemm_blocked_equals_rowsample_and_fp64_error():
    rng = np.random.default_rng(3)
    M, N, K = 300, 520, 257           # crosses the 16-row / 256-col blocks
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = rng.standard_normal((K, N)).astype(np.float32)
    C = oracle.sgemm_seqfma(A, B)
    part = oracle.sgemm_seqfma(A, B, rows=(37, 101))
    assert np.array_equal(C[37:101], part)
    C64 = A.astype(np.float64) @ B.astype(np.float64)
    err = oracle.rel_fro(C, C64)
    assert 1e-8 < err < 1e-6           # fp32 chain error at K=257
    D = oracle.dgemm(A, B)
    assert oracle.rel_fro(D, C64) < 1e-14
    Dt = oracle.dgemm(A.T.copy(), B.T.copy(), transA=True, transB=True)
    assert oracle.rel_fro(Dt, C64) < 1e-14


# ---------------------------------------------------------------------------
# TF32 emulation (matmul_kernel.cu:179-214)
# ---------------------------------------------------------------------------

def test_tf32_round_known_values():
    one_half_ulp = np.float32(1 + 2.0 ** -11)     # exactly half a tf32 ulp
    assert oracle.tf32_round(one_half_ulp, "rz") == 1.0
    assert oracle.tf32_round(one_half_ulp, "rne") == 1.0            # tie -> even
    x = np.float32(1 + 2.0 ** -10 + 2.0 ** -11)                    # tie, odd lsb
    assert oracle.tf32_round(x, "rne") == np.float32(1 + 2.0 ** -9)
    assert oracle.tf32_round(x, "rz") == np.float32(1 + 2.0 ** -10)
    y = np.float32(-(1 + 2.0 ** -11 + 2.0 ** -20))                  # above half
    assert oracle.tf32_round(y, "rne") == np.float32(-(1 + 2.0 ** -10))
    assert oracle.tf32_round(y, "rz") == np.float32(-1.0)
    assert np.isinf(oracle.tf32_round(np.float32(np.inf), "rne"))
    # C routine agrees with the numpy one
    L = oracle.lib()
    for v in (one_half_ulp, x, y, np.float32(3.14159)):
        assert L.orc_tf32_round(float(v), 1) == oracle.tf32_round(v, "rne")
        assert L.orc_tf32_round(float(v), 0) == oracle.tf32_round(v, "rz")


def test_tf32emu_integer_exact_and_chunked():
    rng = np.random.default_rng(5)
    A = rng.integers(-8, 9, (20, 24)).astype(np.float32)
    B = rng.integers(-8, 9, (24, 12)).astype(np.float32)
    for mode in ("rz", "rne"):
        assert np.array_equal(oracle.gemm_tf32emu(A, B, mode), A @ B)
    # exact rational restatement on tiny random input: chunks of 8, one
    # rounding per chunk into the fp32 accumulator
    A = rng.standard_normal((2, 19)).astype(np.float32)
    B = rng.standard_normal((19, 3)).astype(np.float32)
    for mode in ("rz", "rne"):
        C = oracle.gemm_tf32emu(A, B, mode)
        Ar, Br = oracle.tf32_round(A, mode), oracle.tf32_round(B, mode)
        for i in range(2):
            for j in range(3):
                acc = np.float32(0)
                for k0 in range(0, 19, 8):
                    s = sum(Fraction(float(Ar[i, k])) * Fraction(float(Br[k, j]))
                            for k in range(k0, min(k0 + 8, 19)))
                    acc = round_f32(Fraction(float(acc)) + s)
                assert C[i, j] == acc


def test_tf32emu_error_scale():
    rng = np.random.default_rng(11)
    A = rng.standard_normal((128, 512)).astype(np.float32)
    B = rng.standard_normal((512, 96)).astype(np.float32)
    C64 = A.astype(np.float64) @ B.astype(np.float64)
    e_rz = oracle.rel_fro(oracle.gemm_tf32emu(A, B, "rz"), C64)
    e_rne = oracle.rel_fro(oracle.gemm_tf32emu(A, B, "rne"), C64)
    assert 2e-4 < e_rne < e_rz < 5e-3


# ---------------------------------------------------------------------------
# im2col / transpose_bias / direct conv (conv_kernel.cu:32-159)
# ---------------------------------------------------------------------------

def _conv_kat(k):
    x = np.array(k["x"], np.float32).reshape(k["x_shape"])
    w = np.array(k["w"], np.float32).reshape(k["w_shape"])
    b = None if k["bias"] is None else np.array(k["bias"], np.float32)
    return x, w, b


@pytest.mark.parametrize("name", ["conv_identity_1x1", "conv_3x3_ones",
                                  "conv_3x3_bias", "conv_3x3_pad1"])
def test_conv_kats(kats, name):
    k = kats[name]
    x, w, b = _conv_kat(k)
    y = np.array(k["y"], np.float64)
    d = oracle.conv2d_direct64(x, w, b, k["stride"], k["padding"])
    assert np.array_equal(d.ravel(), y)
    r = oracle.conv2d_ref_im2col(x, w, b, k["stride"], k["padding"])
    assert np.array_equal(r.ravel(), y.astype(np.float32))


@pytest.mark.parametrize("name", ["conv_identity_1x1", "conv_3x3_ones",
                                  "conv_3x3_bias", "conv_3x3_pad1"])
def test_conv_implicit_kats(kats, name):
    k = kats[name]
    x, w, b = _conv_kat(k)
    r = oracle.conv2d_ref_implicit(x, w, b, k["stride"], k["padding"])
    assert np.array_equal(r.ravel(), np.array(k["y"], np.float32))


@pytest.mark.parametrize("geom", [(2, 3, 6, 7, 2, 3, 3, 1, 1, 1, 1),
                                  (1, 2, 7, 5, 3, 5, 3, 2, 1, 2, 0),
                                  (2, 2, 5, 6, 2, 1, 1, 1, 1, 0, 0)])
def test_conv_implicit_is_bias_first_fma_chain(geom):
    """conv2d_ref_implicit against an exact-rational restatement of the
    reference's implicit kernel (conv_kernel.cu:172-215): acc = bias, then one
    correctly rounded fma per in-range tap, ic -> kh -> kw.  Fails if the bias
    is added last, a tap order changes, or padding taps are not skipped."""
    Bn, IC, H, W, OC, KH, KW, SH, SW, PH, PW = geom
    rng = np.random.default_rng(31 + sum(geom))
    x = rng.standard_normal((Bn, IC, H, W)).astype(np.float32)
    w = rng.standard_normal((OC, IC, KH, KW)).astype(np.float32)
    b = (rng.standard_normal(OC) * 100).astype(np.float32)   # large: bias order matters
    got = oracle.conv2d_ref_implicit(x, w, b, (SH, SW), (PH, PW))
    OH, OW = oracle.conv_out_size(H, KH, SH, PH), oracle.conv_out_size(W, KW, SW, PW)
    want = np.empty((Bn, OC, OH, OW), np.float32)
    for bi in range(Bn):
        for oc in range(OC):
            for oh in range(OH):
                for ow in range(OW):
                    acc = b[oc]
                    for ic in range(IC):
                        for kh in range(KH):
                            ih = oh * SH - PH + kh
                            if not 0 <= ih < H:
                                continue
                            for kw in range(KW):
                                iw = ow * SW - PW + kw
                                if 0 <= iw < W:
                                    acc = fma_f32(x[bi, ic, ih, iw], w[oc, ic, kh, kw], acc)
                    want[bi, oc, oh, ow] = acc
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # integer-valued operands: every partial sum exact, so = fp64 closed form
    xi = rng.integers(-4, 5, x.shape).astype(np.float32)
    wi = rng.integers(-4, 5, w.shape).astype(np.float32)
    bi_ = rng.integers(-9, 10, OC).astype(np.float32)
    assert np.array_equal(oracle.conv2d_ref_implicit(xi, wi, bi_, (SH, SW), (PH, PW)),
                          oracle.conv2d_direct64(xi, wi, bi_, (SH, SW), (PH, PW)).astype(np.float32))


def test_im2col_1x1_is_relayout():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((3, 5, 4, 6)).astype(np.float32)
    col = oracle.im2col(x, 1, 1)
    assert np.array_equal(col, x.transpose(1, 0, 2, 3).reshape(5, -1))


def test_im2col_zero_count_and_values():
    # every col entry is either an input value or an inserted zero; the number
    # of zeros is fixed by the geometry
    rng = np.random.default_rng(4)
    Bn, C, H, W, KH, KW, S, P = 2, 3, 7, 5, 3, 2, 2, 1
    x = (rng.standard_normal((Bn, C, H, W)) + 10).astype(np.float32)  # no zeros
    col = oracle.im2col(x, KH, KW, S, S, P, P)
    OH, OW = oracle.conv_out_size(H, KH, S, P), oracle.conv_out_size(W, KW, S, P)
    assert col.shape == (C * KH * KW, Bn * OH * OW)
    valid_h = sum(1 for oh in range(OH) for kh in range(KH) if 0 <= oh * S - P + kh < H)
    valid_w = sum(1 for ow in range(OW) for kw in range(KW) if 0 <= ow * S - P + kw < W)
    assert np.count_nonzero(col) == Bn * C * valid_h * valid_w
    assert set(np.unique(col[col != 0])) <= set(np.unique(x))


@pytest.mark.parametrize("geom", [(2, 3, 8, 9, 4, 3, 3, 1, 1, 1, 1),
                                  (1, 2, 7, 7, 3, 5, 3, 2, 1, 2, 0),
                                  (3, 4, 6, 5, 2, 1, 1, 1, 1, 0, 0)])
def test_im2col_gemm_equals_direct_conv_and_torch(geom):
    torch = pytest.importorskip("torch")
    Bn, IC, H, W, OC, KH, KW, SH, SW, PH, PW = geom
    rng = np.random.default_rng(9)
    x = rng.standard_normal((Bn, IC, H, W)).astype(np.float32)
    w = rng.standard_normal((OC, IC, KH, KW)).astype(np.float32)
    b = rng.standard_normal(OC).astype(np.float32)
    col = oracle.im2col(x, KH, KW, SH, SW, PH, PW)
    flat = w.reshape(OC, -1).astype(np.float64) @ col.astype(np.float64)
    OH = oracle.conv_out_size(H, KH, SH, PH)
    OW = oracle.conv_out_size(W, KW, SW, PW)
    via_col = flat.reshape(OC, Bn, OH, OW).transpose(1, 0, 2, 3) + b[None, :, None, None]
    direct = oracle.conv2d_direct64(x, w, b, (SH, SW), (PH, PW))
    lib_ref = torch.nn.functional.conv2d(
        torch.from_numpy(x).double(), torch.from_numpy(w).double(),
        torch.from_numpy(b).double(), stride=(SH, SW), padding=(PH, PW)).numpy()
    assert np.allclose(direct, lib_ref, rtol=1e-12, atol=1e-12)
    assert np.allclose(via_col, lib_ref, rtol=1e-12, atol=1e-12)


def test_transpose_bias_vs_numpy():
    rng = np.random.default_rng(6)
    OC, Bn, S = 5, 3, 11
    src = rng.standard_normal((OC, Bn * S)).astype(np.float32)
    bias = rng.standard_normal(OC).astype(np.float32)
    got = oracle.transpose_bias(src, OC, Bn, S, bias)
    want = src.reshape(OC, Bn, S).transpose(1, 0, 2) + bias[None, :, None]
    assert np.array_equal(got, want.astype(np.float32))
    assert np.array_equal(oracle.transpose_bias(src, OC, Bn, S),
                          src.reshape(OC, Bn, S).transpose(1, 0, 2))


# ---------------------------------------------------------------------------
# column sum and activations
# ---------------------------------------------------------------------------

def test_colsum():
    rng = np.random.default_rng(8)
    x = rng.integers(-50, 50, (333, 17)).astype(np.float32)
    assert np.array_equal(oracle.colsum(x), x.astype(np.float64).sum(0).astype(np.float32))
    y = rng.standard_normal((1000, 9)).astype(np.float32)
    assert np.allclose(oracle.colsum(y), y.astype(np.float64).sum(0), rtol=1e-4, atol=1e-4)


def test_gelu_against_torch_and_derivative():
    torch = pytest.importorskip("torch")
    x = np.linspace(-6, 6, 1001)
    ref = torch.nn.functional.gelu(torch.from_numpy(x), approximate="tanh").numpy()
    # the reference's constant 0.7978845608 is sqrt(2/pi) to 10 digits
    assert np.allclose(oracle.gelu(x), ref, rtol=1e-9, atol=1e-10)
    h = 1e-6
    num = (oracle.gelu(x + h) - oracle.gelu(x - h)) / (2 * h)
    assert np.allclose(oracle.gelu_grad(x), num, atol=1e-7)
    assert oracle.gelu(np.array([0.0]))[0] == 0.0
    assert np.array_equal(oracle.relu(np.array([-1.0, 0.0, 2.0])), [0.0, 0.0, 2.0])
    assert np.array_equal(oracle.relu_grad(np.array([-1.0, 0.0, 2.0])), [0.0, 0.0, 1.0])


def test_tanh_and_leaky_relu_closed_forms():
    """tanh against its exponential form and its derivative against central
    differences; leaky ReLU at known points (slope 0.01 as fp32)."""
    x = np.linspace(-8, 8, 801)
    e = np.exp(-2 * np.abs(x))
    assert np.allclose(oracle.tanh(x), np.sign(x) * (1 - e) / (1 + e), rtol=1e-13, atol=1e-15)
    h = 1e-6
    num = (oracle.tanh(x + h) - oracle.tanh(x - h)) / (2 * h)
    assert np.allclose(oracle.tanh_grad(x), num, atol=1e-8)
    a = float(np.float32(0.01))
    assert np.array_equal(oracle.leaky_relu(np.array([-2.0, 0.0, 3.0])), [-2.0 * a, 0.0, 3.0])
    assert np.array_equal(oracle.leaky_relu_grad(np.array([-2.0, 0.0, 3.0])), [a, a, 1.0])
    assert np.array_equal(oracle.leaky_relu(np.array([-1.0]), 0.2), [-float(np.float32(0.2))])


def test_tf32_round_is_identity_on_16bit_values():
    """fp16 and bf16 values have at most 11 significant bits, so TF32 rounding
    (either mode) leaves them unchanged: gemm_tf32emu on fp32-converted 16-bit
    operands is the exact-product, 8-term-chunk ideal MMA used as the FP16 /
    BF16 GEMM yardstick."""
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(16)
    x = rng.standard_normal(20000).astype(np.float32) * 10.0 ** rng.uniform(-4, 4, 20000)
    for td in (torch.float16, torch.bfloat16):
        v = torch.from_numpy(x.astype(np.float32)).to(td).float().numpy()
        v = v[np.isfinite(v)]
        for mode in ("rz", "rne"):
            assert np.array_equal(oracle.tf32_round(v, mode), v)
    # and a value with 12 significant bits is changed (the check has teeth)
    y = np.float32(1 + 2.0 ** -11)
    assert oracle.tf32_round(np.array([y]), "rz")[0] != y


def test_sigmoid_silu_against_tanh_torch_and_derivative():
    """sigmoid against scipy's expit and, away from the cancelling tail, the
    closed form (1 + tanh(x/2)) / 2; SiLU against torch's silu; both
    derivatives against central differences; the tails stay finite."""
    torch = pytest.importorskip("torch")
    special = pytest.importorskip("scipy.special")
    x = np.linspace(-30, 30, 2001)
    assert np.allclose(oracle.sigmoid(x), special.expit(x), rtol=1e-14, atol=0)
    xm = x[x > -8]
    assert np.allclose(oracle.sigmoid(xm), 0.5 * (1.0 + np.tanh(0.5 * xm)), rtol=1e-11, atol=0)
    assert oracle.sigmoid(np.array([0.0]))[0] == 0.5
    assert np.allclose(oracle.silu(x), torch.nn.functional.silu(torch.from_numpy(x)).numpy(),
                       rtol=1e-13, atol=1e-300)
    h = 1e-6
    for f, g in ((oracle.sigmoid, oracle.sigmoid_grad), (oracle.silu, oracle.silu_grad)):
        num = (f(x + h) - f(x - h)) / (2 * h)
        assert np.allclose(g(x), num, atol=1e-8)
    big = np.array([-1000.0, 1000.0])
    assert np.all(np.isfinite(oracle.sigmoid(big))) and np.all(np.isfinite(oracle.silu_grad(big)))
    assert np.array_equal(oracle.sigmoid(big), [0.0, 1.0])


# ---------------------------------------------------------------------------
# col2im and the backward-conv routes (conv_kernel.cu:344-545)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("geom", [(2, 3, 8, 9, 3, 3, 1, 1, 1, 1), (1, 2, 7, 7, 3, 5, 2, 1, 2, 0),
                                  (2, 4, 9, 6, 2, 2, 2, 2, 0, 1)])
def test_col2im_is_adjoint_of_im2col(geom):
    """<im2col(x), C> == <x, col2im(C)> for every x, C (fp64 gather)."""
    Bn, IC, H, W, KH, KW, SH, SW, PH, PW = geom
    rng = np.random.default_rng(31)
    x = rng.standard_normal((Bn, IC, H, W)).astype(np.float32)
    col = oracle.im2col(x, KH, KW, SH, SW, PH, PW)
    C = rng.standard_normal(col.shape)
    back = oracle.col2im(C, x.shape, KH, KW, SH, SW, PH, PW)
    lhs = float((col.astype(np.float64) * C).sum())
    rhs = float((x.astype(np.float64) * back).sum())
    assert abs(lhs - rhs) <= 1e-9 * max(1.0, abs(lhs))
    # fp32 gather on exactly representable (integer) data equals the fp64 one
    Ci = rng.integers(-20, 20, col.shape).astype(np.float32)
    assert np.array_equal(oracle.col2im(Ci, x.shape, KH, KW, SH, SW, PH, PW),
                          oracle.col2im(Ci.astype(np.float64), x.shape, KH, KW, SH, SW, PH, PW))


def test_conv_backward_kats(kats):
    k = kats["conv_bwd_data_1x1_w2"]
    dy = np.array(k["dy"], np.float32).reshape(k["dy_shape"])
    w = np.array(k["w"], np.float32).reshape(k["w_shape"])
    dx = oracle.conv2d_backward_data_ref(dy, w, tuple(k["x_shape"]), k["stride"], k["padding"])
    assert np.array_equal(dx.ravel(), np.array(k["dx"], np.float32))
    k = kats["conv_bwd_weight_ones"]
    dy = np.array(k["dy"], np.float32).reshape(k["dy_shape"])
    x = np.array(k["x"], np.float32).reshape(k["x_shape"])
    dw = oracle.conv2d_backward_weight_ref(dy, x, tuple(k["w_shape"]), k["stride"], k["padding"])
    assert np.array_equal(dw.ravel(), np.array(k["dw"], np.float32))


@pytest.mark.parametrize("geom", [(2, 3, 8, 9, 4, 3, 3, 1, 1, 1, 1), (1, 2, 7, 7, 3, 3, 5, 2, 1, 2, 0),
                                  (3, 4, 6, 5, 2, 2, 1, 1, 1, 0, 0)])
def test_conv_backward_vs_torch_fp64(geom):
    torch = pytest.importorskip("torch")
    Bn, IC, H, W, OC, KH, KW, SH, SW, PH, PW = geom
    rng = np.random.default_rng(41)
    x = rng.standard_normal((Bn, IC, H, W)).astype(np.float32)
    w = rng.standard_normal((OC, IC, KH, KW)).astype(np.float32)
    OH = oracle.conv_out_size(H, KH, SH, PH)
    OW = oracle.conv_out_size(W, KW, SW, PW)
    dy = rng.standard_normal((Bn, OC, OH, OW)).astype(np.float32)
    tx, tw, tdy = (torch.from_numpy(a).double() for a in (x, w, dy))
    dx_t = torch.nn.grad.conv2d_input(x.shape, tw, tdy, stride=(SH, SW), padding=(PH, PW)).numpy()
    dw_t = torch.nn.grad.conv2d_weight(tx, w.shape, tdy, stride=(SH, SW), padding=(PH, PW)).numpy()
    dx64 = oracle.conv2d_backward_data64(dy, w, x.shape, (SH, SW), (PH, PW))
    dw64 = oracle.conv2d_backward_weight64(dy, x, w.shape, (SH, SW), (PH, PW))
    assert np.allclose(dx64, dx_t, rtol=1e-10, atol=1e-10)
    assert np.allclose(dw64, dw_t, rtol=1e-10, atol=1e-10)
    # the fp32 reference routes sit at fp32 error from them
    dx32 = oracle.conv2d_backward_data_ref(dy, w, x.shape, (SH, SW), (PH, PW))
    dw32 = oracle.conv2d_backward_weight_ref(dy, x, w.shape, (SH, SW), (PH, PW))
    assert oracle.rel_fro(dx32, dx64) < 1e-6 and oracle.rel_fro(dw32, dw64) < 1e-6


@pytest.mark.parametrize("geom", [(2, 3, 8, 9, 4, 3, 3, 1, 1), (1, 2, 7, 7, 3, 3, 5, 2, 0),
                                  (3, 4, 6, 5, 2, 2, 2, 1, 0), (2, 3, 5, 6, 2, 1, 1, 0, 0),
                                  (1, 2, 9, 4, 3, 5, 3, 4, 1)])
def test_backward_data_is_flipped_forward(geom):
    """Stride-1 backward data equals the forward convolution of dY with the
    channel-swapped, spatially reversed filter padded K-1-P (the identity
    the stride-1 backward-data route runs on).  A filter read unflipped,
    unswapped or with the wrong padding fails at O(1)."""
    Bn, IC, H, W, OC, KH, KW, PH, PW = geom
    rng = np.random.default_rng(43 + sum(geom))
    w = rng.standard_normal((OC, IC, KH, KW)).astype(np.float32)
    OH, OW = oracle.conv_out_size(H, KH, 1, PH), oracle.conv_out_size(W, KW, 1, PW)
    dy = rng.standard_normal((Bn, OC, OH, OW)).astype(np.float32)
    want = oracle.conv2d_backward_data64(dy, w, (Bn, IC, H, W), (1, 1), (PH, PW))
    got = oracle.conv2d_direct64(dy, oracle.flip_filter(w), None, (1, 1), (KH - 1 - PH, KW - 1 - PW))
    assert got.shape == want.shape
    assert np.allclose(got, want, rtol=1e-12, atol=1e-12)
    if KH == 3 and KW == 3 and PH <= 2 and PW <= 2:
        wino = oracle.conv2d_backward_data_winograd(dy, w, (Bn, IC, H, W), (PH, PW), double=True)
        assert oracle.rel_fro(wino, want) < 1e-13


# ---------------------------------------------------------------------------
# Winograd F(4x4, 3x3) route (conv_kernel.cu:557-789)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("B,IC,OC,H,W,P", [(2, 3, 4, 9, 11, 1), (1, 5, 2, 6, 6, 0),
                                           (2, 8, 8, 16, 16, 1), (1, 1, 1, 7, 5, 2),
                                           (1, 4, 3, 3, 3, 0), (1, 2, 2, 13, 4, 1)])
def test_winograd_double_equals_direct_conv(B, IC, OC, H, W, P):
    """In exact arithmetic F(4x4, 3x3) is the 3x3 cross-correlation, so the
    fp64 form must match the fp64 direct convolution to rounding: a wrong
    transform coefficient, sign or tile offset breaks this at O(1)."""
    rng = np.random.default_rng(B * 100 + IC * 10 + H + P)
    x = rng.standard_normal((B, IC, H, W)).astype(np.float32)
    w = rng.standard_normal((OC, IC, 3, 3)).astype(np.float32)
    b = rng.standard_normal(OC).astype(np.float32)
    d = oracle.conv2d_direct64(x, w, b, padding=(P, P))
    w64 = oracle.conv2d_winograd(x, w, b, padding=(P, P), double=True)
    assert w64.shape == d.shape
    assert np.abs(w64 - d).max() <= 1e-12 * np.abs(d).max()
    # fp32: transform rounding, bounded well below the data scale
    w32 = oracle.conv2d_winograd(x, w, b, padding=(P, P))
    assert oracle.rel_fro(w32, d) < 1e-5
    # TF32 operand rounding costs about 2^-11 relative, more than fp32
    wt = oracle.conv2d_winograd(x, w, b, padding=(P, P), tf32="rne")
    assert oracle.rel_fro(w32, d) < oracle.rel_fro(wt, d) < 1e-2


def test_winograd_reference_conv_kats(kats):
    """The reference's 3x3 conv known answers (test_kernels.cu:352-425) through
    the Winograd route: all-ones -> 9, bias 10 -> 19, pad 1 -> 4 / 6 / 9."""
    for name in ("conv_3x3_ones", "conv_3x3_bias", "conv_3x3_pad1"):
        k = kats[name]
        x = np.array(k["x"], np.float32).reshape(k["x_shape"])
        w = np.array(k["w"], np.float32).reshape(k["w_shape"])
        b = np.array(k["bias"], np.float32) if k.get("bias") is not None else None
        assert tuple(k["stride"]) == (1, 1)
        y = oracle.conv2d_winograd(x, w, b, padding=tuple(k["padding"]))
        want = np.array(k["y"], np.float32).reshape(y.shape)
        assert np.allclose(y, want, rtol=0, atol=1e-5), name
