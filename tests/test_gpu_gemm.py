"""GPU parity of the GEMM entry points against the CPU oracle.

Gates (the north_star bars):
  * FP32: relFro(gpu vs fp64) <= 2 x relFro(seq-FMA restatement of the
    reference SGEMM vs fp64), on the same seeded inputs.
  * TF32 mode (bf16x3): relFro(gpu vs fp64) <= min over {RZ, RNE} of the
    emulated reference TF32 kernel's relFro.
  * integer-valued inputs (reference MMA KATs): exact.
At 4096^3 the CPU oracle runs on a sample of rows; the full output is
checked by a size-independent identity: column sums of C equal
(column sums of A) @ B, computed in fp64.
"""
import numpy as np
import pytest

import oracle
from tests.gpu_util import F32_FLOOR, dev, host, normal, require_gpu, say, uniform

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    require_gpu()
    import cudeep_amd.ops  # noqa: F401  (loads libcudeep_amd.so)


def ops():
    import cudeep_amd.ops as o
    return o


def _ref_errors(A, B, tA=False, tB=False, rows=None):
    C64 = oracle.dgemm(A, B, tA, tB, rows=rows)
    Cs = oracle.sgemm_seqfma(A, B, tA, tB, rows=rows)
    return C64, oracle.rel_fro(Cs, C64)


# ---------------------------------------------------------------------------
# reference known answers (tests/golden/kats.json)
# ---------------------------------------------------------------------------

def _gemm_fn(mode):
    """NN GEMM entry for a precision mode name."""
    import cudeep_amd as cd
    if mode == "fp32":
        return ops().sgemm
    if mode == "tf32":
        return ops().gemm_tf32mode
    return lambda A, B: ops().gemm(A, B, precision=cd.PREC_TF32MODE4)


@pytest.mark.parametrize("name", ["matmul_2x2", "matmul_diag_identity", "mma_identity",
                                  "mma_integer_pattern"])
@pytest.mark.parametrize("mode", ["fp32", "tf32", "tf32x4"])
def test_gemm_kats_exact(kats, name, mode):
    k = kats[name]
    A = np.array(k["A"], np.float32)
    B = np.array(k["B"], np.float32)
    say("kat", name, mode)
    C = host(_gemm_fn(mode)(dev(A), dev(B)))
    assert np.array_equal(C, np.array(k["C"], np.float32))


def test_gemm_kat_partial_identity_and_scaled(kats):
    k = kats["matmul_partial_identity"]
    say("kat partial identity")
    C = host(ops().sgemm(dev(np.array(k["A"], np.float32)), dev(np.array(k["B"], np.float32))))
    assert np.array_equal(C[0], np.array(k["C_row0"], np.float32))
    k = kats["matmul_scaled_identity_8"]
    A = np.array(k["A"], np.float32)
    for f in (ops().sgemm, ops().gemm_tf32mode):
        C = host(f(dev(A), dev(np.eye(8, dtype=np.float32))))
        assert np.allclose(C, A, atol=k["atol"])


def test_randn_times_identity_rtol_1e5():
    # tests/unit/test_tensor_ops.py:220-227: randn(N,N) @ I within rtol 1e-5
    rng = np.random.default_rng(21)
    A = normal(rng, (96, 96))
    say("randn @ I")
    for f in (ops().sgemm, ops().gemm_tf32mode):
        C = host(f(dev(A), dev(np.eye(96, dtype=np.float32))))
        assert np.allclose(C, A, rtol=1e-5, atol=0)


@pytest.mark.parametrize("mode", ["fp32", "tf32", "tf32x4"])
def test_integer_inputs_exact_any_shape(mode):
    rng = np.random.default_rng(22)
    for (M, N, K) in [(16, 8, 8), (130, 70, 200), (256, 256, 64)]:
        A = rng.integers(-8, 9, (M, K)).astype(np.float32)
        B = rng.integers(-8, 9, (K, N)).astype(np.float32)
        say("integer", mode, M, N, K)
        assert np.array_equal(host(_gemm_fn(mode)(dev(A), dev(B))), A.astype(np.float64) @ B)


# ---------------------------------------------------------------------------
# FP32 parity vs the sequential-FMA restatement
# ---------------------------------------------------------------------------

SHAPES = [(1, 1, 1), (2, 3, 5), (17, 33, 65), (64, 64, 16), (128, 128, 128),
          (127, 255, 33), (300, 200, 784), (8192, 10, 256), (10, 8192, 256),
          (64, 4096, 576), (256, 512, 1000), (513, 129, 4099)]


@pytest.mark.parametrize("M,N,K", SHAPES)
@pytest.mark.parametrize("tA,tB", [(False, False), (False, True), (True, False), (True, True)])
def test_fp32_gemm_parity_shapes(M, N, K, tA, tB):
    rng = np.random.default_rng(M * 7919 + N * 31 + K + 2 * tA + tB)
    A = normal(rng, (K, M) if tA else (M, K))
    B = normal(rng, (N, K) if tB else (K, N))
    say("fp32", M, N, K, "tA", tA, "tB", tB)
    C = host(ops().gemm(dev(A), dev(B), transA=tA, transB=tB))
    C64, e_ref = _ref_errors(A, B, tA, tB)
    e = oracle.rel_fro(C, C64)
    floor = F32_FLOOR if K < 64 else 0.0
    assert e <= 2 * e_ref + floor, (e, e_ref)


@pytest.mark.parametrize("M,N,K", [(8192, 256, 10), (37, 129, 1), (300, 17, 16), (5, 3, 7)])
@pytest.mark.parametrize("tA,tB", [(False, False), (False, True), (True, False), (True, True)])
@pytest.mark.parametrize("mode", ["fp32", "tf32"])
def test_tiny_k_bit_exact_with_reference_chain(M, N, K, tA, tB, mode):
    """K <= 16 runs an fp32 FMA chain per output over k ascending -- the
    reference SGEMM's arithmetic (matmul_kernel.cu:632-647) -- in every
    precision mode: bit-exact with the oracle's seq-FMA restatement."""
    import cudeep_amd as cd
    rng = np.random.default_rng(M + 7 * N + 31 * K)
    A = normal(rng, (K, M) if tA else (M, K))
    B = normal(rng, (N, K) if tB else (K, N))
    prec = cd.PREC_FP32 if mode == "fp32" else cd.PREC_TF32MODE
    say("tiny-K bit-exact", M, N, K, tA, tB, mode)
    C = host(ops().gemm(dev(A), dev(B), transA=tA, transB=tB, precision=prec))
    want = oracle.sgemm_seqfma(A, B, tA, tB)
    assert np.array_equal(C.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("M,K", [(8192, 256), (100, 64), (4097, 1000)])
@pytest.mark.parametrize("N", [1, 10, 16])
@pytest.mark.parametrize("tA,tB", [(False, True), (True, False)])
def test_narrow_n_parity(M, N, K, tA, tB):
    """N <= 16 (the MLP's 10-class layer): MFMA on operands read straight
    from global memory, K in four quarters summed in a fixed order."""
    rng = np.random.default_rng(M + N + K)
    A = normal(rng, (K, M) if tA else (M, K))
    B = normal(rng, (N, K) if tB else (K, N))
    say("narrow-N", M, N, K, tA, tB)
    C = host(ops().gemm(dev(A), dev(B), transA=tA, transB=tB))
    C64, e_ref = _ref_errors(A, B, tA, tB)
    e = oracle.rel_fro(C, C64)
    assert e <= 2 * e_ref + F32_FLOOR, (e, e_ref)


def test_fp32_c1_512_uniform():
    """C1: 512^3, A, B ~ U[-1, 1]."""
    rng = np.random.default_rng(101)
    A = uniform(rng, (512, 512))
    B = uniform(rng, (512, 512))
    say("C1 512^3")
    C = host(ops().sgemm(dev(A), dev(B)))
    C64, e_ref = _ref_errors(A, B)
    e = oracle.rel_fro(C, C64)
    print(f"C1 relFro gpu={e:.3e} seqfma={e_ref:.3e}")
    assert e <= 2 * e_ref


def _checksum_identity(A, B, C):
    """e^T C == (e^T A) B in fp64; returns the relative error."""
    lhs = C.astype(np.float64).sum(0)
    rhs = A.astype(np.float64).sum(0) @ B.astype(np.float64)
    return np.linalg.norm(lhs - rhs) / np.linalg.norm(rhs)


def test_fp32_c2_4096_sampled_rows_and_checksum():
    """C2: 4096^3, A, B ~ N(0, 1)."""
    rng = np.random.default_rng(202)
    n = 4096
    A = normal(rng, (n, n))
    B = normal(rng, (n, n))
    say("C2 4096^3 fp32")
    C = host(ops().sgemm(dev(A), dev(B)))
    assert np.isfinite(C).all()
    errs = []
    for r0 in (0, 1792, n - 128):
        rows = (r0, r0 + 128)
        C64, e_ref = _ref_errors(A, B, rows=rows)
        e = oracle.rel_fro(C[r0:r0 + 128], C64)
        errs.append((e, e_ref))
        assert e <= 2 * e_ref, (rows, e, e_ref)
    print("C2 sampled relFro (gpu, seqfma):", errs)
    assert _checksum_identity(A, B, C) < 1e-5


@pytest.mark.parametrize("M,N,K", [(2048, 2048, 2048), (3072, 3072, 512), (4096, 1024, 1024)])
@pytest.mark.parametrize("tA,tB", [(False, False), (True, True)])
def test_fp32_mid_size_tile_choice(M, N, K, tA, tB):
    """Mid-size problems on both sides of the 128x128 / 64x64 choice (128-tiles
    that spread evenly over the CUs -- 256 of them at 2048^2 and 4096 x 1024 --
    against 576 at 3072^2): sampled rows against the seq-FMA restatement and
    the column-checksum identity over the whole product."""
    rng = np.random.default_rng(M + 3 * N + 7 * K + 2 * tA + tB)
    A = normal(rng, (K, M) if tA else (M, K))
    B = normal(rng, (N, K) if tB else (K, N))
    say("fp32 mid-size", M, N, K, tA, tB)
    C = host(ops().gemm(dev(A), dev(B), transA=tA, transB=tB))
    for r0 in (0, M // 2 + 5, M - 64):
        rows = (r0, r0 + 64)
        C64, e_ref = _ref_errors(A, B, tA, tB, rows=rows)
        e = oracle.rel_fro(C[r0:r0 + 64], C64)
        assert e <= 2 * e_ref, (rows, e, e_ref)
    assert _checksum_identity(A.T if tA else A, B.T if tB else B, C) < 1e-5


@pytest.mark.parametrize("tiles", [20, 100, 256 + 40, 256 + 100, 512 + 150, 512 + 174])
@pytest.mark.parametrize("K", [48, 576])
def test_fp32_skinny_last_round_split(tiles, K):
    """64-row NN products whose 64-column tiles leave a short last round over
    the 256 CUs run that round as 64 x 32 or 64 x 16 tiles (the conv GEMM's
    shape).  The same columns inside a wider product of whole rounds only
    (every tile 64 x 64) must come out bit for bit the same; sampled columns
    across the full / split boundary and the last ones against the seq-FMA
    restatement; the column-checksum identity over the whole product."""
    N = 64 * tiles
    Nw = 64 * 256 * ((tiles + 255) // 256)          # whole rounds: no split tiles
    rng = np.random.default_rng(tiles * 7 + K)
    A = normal(rng, (64, K))
    Bw = normal(rng, (K, Nw))
    B = np.ascontiguousarray(Bw[:, :N])
    say("fp32 skinny split", tiles, K)
    C = host(ops().gemm(dev(A), dev(B)))
    Cw = host(ops().gemm(dev(A), dev(Bw)))
    assert np.array_equal(C.view(np.uint32), Cw[:, :N].view(np.uint32))
    full = 64 * (tiles - tiles % 256)
    for c0 in sorted({max(0, full - 96), N - 192}):
        Bs = np.ascontiguousarray(B[:, c0:c0 + 192])
        C64, e_ref = _ref_errors(A, Bs)
        e = oracle.rel_fro(np.ascontiguousarray(C[:, c0:c0 + 192]), C64)
        assert e <= 2 * e_ref, (c0, e, e_ref)
    assert _checksum_identity(A, B, C) < 1e-5


@pytest.mark.parametrize("M,N,K", [(8192, 784, 256), (5000, 784, 100), (4100, 1008, 77)])
@pytest.mark.parametrize("tA,tB", [(False, False), (False, True), (True, False), (True, True)])
def test_fp32_w112_tiles(M, N, K, tA, tB):
    """Widths that are multiples of 112 but not of 64 take 128 x 112 tiles
    (C4's 784-wide backward-data product, ragged M and K too): sampled rows
    against the seq-FMA restatement, the column-checksum identity, and a
    fused bias + ReLU epilogue against the unfused product."""
    import cudeep_amd as cd
    rng = np.random.default_rng(M + 5 * N + 11 * K + 2 * tA + tB)
    A = normal(rng, (K, M) if tA else (M, K))
    B = normal(rng, (N, K) if tB else (K, N))
    say("fp32 w112", M, N, K, tA, tB)
    C = host(ops().gemm(dev(A), dev(B), transA=tA, transB=tB))
    for r0 in (0, M // 2 + 3, M - 64):
        rows = (r0, r0 + 64)
        C64, e_ref = _ref_errors(A, B, tA, tB, rows=rows)
        e = oracle.rel_fro(C[r0:r0 + 64], C64)
        assert e <= 2 * e_ref, (rows, e, e_ref)
    assert _checksum_identity(A.T if tA else A, B.T if tB else B, C) < 1e-5
    bias = normal(rng, (N,))
    Cf = host(ops().gemm(dev(A), dev(B), transA=tA, transB=tB, bias=dev(bias),
                         bias_mode=cd.BIAS_COL, epilogue=cd.EPI_RELU))
    assert np.array_equal(Cf, np.maximum(C + bias[None, :], 0))
    # the TF32 modes run these shapes on the same FP32 kernel (exact products,
    # inside their error bar): the same bits
    for prec in (cd.PREC_TF32MODE, cd.PREC_TF32MODE4):
        Ct = host(ops().gemm(dev(A), dev(B), transA=tA, transB=tB, precision=prec))
        assert np.array_equal(Ct.view(np.uint32), C.view(np.uint32))


@pytest.mark.parametrize("n", [2048, 4096])
@pytest.mark.parametrize("terms", [3, 4])
def test_tf32mode_c3(n, terms):
    """C3: TF32 mode (bf16x3 / bf16x4) at 2048^3 / 4096^3, inputs N(0,1),
    read as raw fp32 (the bits the reference feeds its MMA): the error must
    not exceed the emulated reference TF32 error under either operand
    rounding (RZ / RNE)."""
    import cudeep_amd as cd
    rng = np.random.default_rng(303 + n)
    A = normal(rng, (n, n))
    B = normal(rng, (n, n))
    say("C3 tf32mode raw", n, terms)
    prec = cd.PREC_TF32MODE if terms == 3 else cd.PREC_TF32MODE4
    C = host(ops().gemm(dev(A), dev(B), precision=prec))
    rows = (n // 2, n // 2 + 96)
    C64 = oracle.dgemm(A, B, rows=rows)
    e = oracle.rel_fro(C[rows[0]:rows[1]], C64)
    e_rz = oracle.rel_fro(oracle.gemm_tf32emu(A, B, "rz", rows=rows), C64)
    e_rne = oracle.rel_fro(oracle.gemm_tf32emu(A, B, "rne", rows=rows), C64)
    print(f"C3 n={n} raw: bf16x{terms}={e:.3e} tf32(rz)={e_rz:.3e} tf32(rne)={e_rne:.3e}")
    assert e <= min(e_rz, e_rne)
    assert _checksum_identity(A, B, C) < 1e-4


@pytest.mark.parametrize("n", [2048, 4096])
def test_tf32mode_c3_prerounded(n):
    """C3 under the second reading: operands pre-rounded to TF32 (RNE), so
    the reference's TF32 products are exact and its error is fp32
    accumulation only.  bf16x4 splits such operands exactly (hi + lo has 16
    significant bits) and sums each 32-k step from zero before one add into
    C, so its error must not exceed the emulated reference's (an ideal MMA:
    exact 8-term chunks, one fp32 rounding each).  bf16x3 drops lo*lo, which is at most
    2^-18 |a b| here (|lo| <= 2^-9 |x|), so per element its error is bounded
    by 2^-18 sum_k |a_ik b_kj| on top of accumulation."""
    import cudeep_amd as cd
    rng = np.random.default_rng(313 + n)
    A = oracle.tf32_round(normal(rng, (n, n)), "rne")
    B = oracle.tf32_round(normal(rng, (n, n)), "rne")
    rows = (n // 3, n // 3 + 96)
    C64 = oracle.dgemm(A, B, rows=rows)
    e_ref = oracle.rel_fro(oracle.gemm_tf32emu(A, B, "rne", rows=rows), C64)
    absAB = np.abs(A[rows[0]:rows[1]]).astype(np.float64) @ np.abs(B).astype(np.float64)
    bound3 = 2.0 ** -18 * np.linalg.norm(absAB) / np.linalg.norm(C64) + 2 * e_ref
    res = {}
    for terms, prec in ((3, cd.PREC_TF32MODE), (4, cd.PREC_TF32MODE4)):
        say("C3 tf32mode pre-rounded", n, terms)
        C = host(ops().gemm(dev(A), dev(B), precision=prec))
        res[terms] = oracle.rel_fro(C[rows[0]:rows[1]], C64)
    print(f"C3 n={n} pre-rounded: bf16x3={res[3]:.3e} bf16x4={res[4]:.3e} "
          f"tf32 ideal={e_ref:.3e} bf16x3 bound={bound3:.3e}")
    assert res[4] <= e_ref
    assert res[3] <= bound3


@pytest.mark.parametrize("mode", ["tf32", "tf32x4"])
def test_tf32mode_parity_shapes(mode):
    rng = np.random.default_rng(304)
    for (M, N, K) in [(17, 33, 65), (300, 200, 784), (8192, 10, 256), (64, 1000, 576),
                      (8192, 256, 784), (10, 256, 8192)]:
        A = normal(rng, (M, K))
        B = normal(rng, (K, N))
        say("tf32 shape", mode, M, N, K)
        C = host(_gemm_fn(mode)(dev(A), dev(B)))
        C64 = oracle.dgemm(A, B)
        e = oracle.rel_fro(C, C64)
        e_rne = oracle.rel_fro(oracle.gemm_tf32emu(A, B, "rne"), C64)
        assert e <= e_rne, (M, N, K, e, e_rne)


@pytest.mark.parametrize("tA,tB", [(False, False), (False, True), (True, False), (True, True)])
@pytest.mark.parametrize("K", [32, 64, 96, 544])
def test_tf32mode_256_tile_path(tA, tB, K):
    """The 256 x 256 two-group (ping-pong) TF32-mode kernel, which M = N =
    4096 selects (256 tiles, aligned).  K = 32 / 64 / 96 give one, two and
    three k-tiles (the prologue and the loop-tail branches), K = 544 a
    longer loop.  Gate: relFro on sampled rows <= the emulated reference
    TF32 error (either operand rounding), plus the column-checksum identity
    on the whole output."""
    import cudeep_amd as cd
    rng = np.random.default_rng(1000 + K + 2 * tA + tB)
    n = 4096
    A = normal(rng, (K, n) if tA else (n, K))
    B = normal(rng, (n, K) if tB else (K, n))
    say("tf32 256-tile path", tA, tB, K)
    C = host(ops().gemm(dev(A), dev(B), transA=tA, transB=tB, precision=cd.PREC_TF32MODE))
    opA = np.ascontiguousarray(A.T if tA else A)
    opB = np.ascontiguousarray(B.T if tB else B)
    for rows in ((0, 48), (n // 2 - 16, n // 2 + 16), (n - 48, n)):
        C64 = oracle.dgemm(opA, opB, rows=rows)
        e = oracle.rel_fro(C[rows[0]:rows[1]], C64)
        e_rz = oracle.rel_fro(oracle.gemm_tf32emu(opA, opB, "rz", rows=rows), C64)
        e_rne = oracle.rel_fro(oracle.gemm_tf32emu(opA, opB, "rne", rows=rows), C64)
        assert e <= min(e_rz, e_rne), (rows, e, e_rz, e_rne)
    assert _checksum_identity(opA, opB, C) < 1e-4


@pytest.mark.parametrize("tA,tB", [(False, False), (False, True), (True, False), (True, True)])
@pytest.mark.parametrize("K", [32, 64, 96, 544, 2080])
@pytest.mark.parametrize("prec_name", ["PREC_TF32MODE", "PREC_TF32MODE4"])
def test_tf32mode_kalt_path(tA, tB, K, prec_name):
    """The k-alternating 128 x 128 TF32-mode kernel, which 2048 x 2048
    outputs select (256 tiles of 128 x 128, too few of 256 x 256): its two
    wave groups take alternate k-tiles and add their sums at the end.  K = 32
    leaves the second group without a k-tile; K = 96 and 2080 give odd k-tile
    counts (the groups end on padded barrier counts); both variants (three
    terms with two staging sets, four with one).  Gate: relFro on sampled
    rows <= the emulated reference TF32 error, and the checksum identity."""
    import cudeep_amd as cd
    rng = np.random.default_rng(2000 + K + 2 * tA + tB)
    n = 2048
    A = normal(rng, (K, n) if tA else (n, K))
    B = normal(rng, (n, K) if tB else (K, n))
    say("tf32 k-alternating path", tA, tB, K, prec_name)
    C = host(ops().gemm(dev(A), dev(B), transA=tA, transB=tB,
                        precision=getattr(cd, prec_name)))
    opA = np.ascontiguousarray(A.T if tA else A)
    opB = np.ascontiguousarray(B.T if tB else B)
    for rows in ((0, 40), (n // 2 - 24, n // 2 + 24), (n - 40, n)):
        C64 = oracle.dgemm(opA, opB, rows=rows)
        e = oracle.rel_fro(C[rows[0]:rows[1]], C64)
        e_rz = oracle.rel_fro(oracle.gemm_tf32emu(opA, opB, "rz", rows=rows), C64)
        e_rne = oracle.rel_fro(oracle.gemm_tf32emu(opA, opB, "rne", rows=rows), C64)
        assert e <= min(e_rz, e_rne), (rows, e, e_rz, e_rne)
    assert _checksum_identity(opA, opB, C) < 1e-4


@pytest.mark.parametrize("epi,bias_mode", [("gelu", "col"), ("relu", "row")])
@pytest.mark.parametrize("prec_name", ["PREC_TF32MODE", "PREC_TF32MODE4"])
def test_tf32mode_kalt_epilogue(epi, bias_mode, prec_name):
    """Bias + activation epilogue of the k-alternating kernel (each wave
    group writes half of every wave's sub-tile after the hand-over)."""
    import cudeep_amd as cd
    rng = np.random.default_rng(1200)
    M, N, K = 2048, 2048, 160
    A = normal(rng, (M, K))
    W = normal(rng, (N, K))
    bias = normal(rng, (M if bias_mode == "row" else N,))
    bm = {"row": cd.BIAS_ROW, "col": cd.BIAS_COL}[bias_mode]
    ep = {"relu": cd.EPI_RELU, "gelu": cd.EPI_GELU}[epi]
    say("tf32 k-alternating epilogue", epi, bias_mode, prec_name)
    C = host(ops().gemm(dev(A), dev(W), transB=True, precision=getattr(cd, prec_name),
                        bias=dev(bias), bias_mode=bm, epilogue=ep))
    for rows in ((0, 64), (1000, 1064), (M - 64, M)):
        Z = oracle.dgemm(A, np.ascontiguousarray(W.T), rows=rows)
        Z = Z + (bias[rows[0]:rows[1], None] if bias_mode == "row" else bias[None, :])
        want = oracle.activation(Z, epi)
        assert np.max(np.abs(C[rows[0]:rows[1]] - want)) <= 2e-5 * np.abs(Z).max() + 1e-6


@pytest.mark.parametrize("epi,bias_mode", [("gelu", "col"), ("relu", "row"), ("silu", "none")])
def test_tf32mode_256_tile_epilogue(epi, bias_mode):
    """Bias + activation epilogue of the 256 x 256 TF32-mode kernel (the
    fused Linear forward at a large batch: x @ W^T)."""
    import cudeep_amd as cd
    rng = np.random.default_rng(1100)
    M, N, K = 4096, 4096, 128
    A = normal(rng, (M, K))
    W = normal(rng, (N, K))
    bias = normal(rng, (M if bias_mode == "row" else N,))
    bm = {"none": cd.BIAS_NONE, "row": cd.BIAS_ROW, "col": cd.BIAS_COL}[bias_mode]
    ep = {"relu": cd.EPI_RELU, "gelu": cd.EPI_GELU, "silu": cd.EPI_SILU}[epi]
    say("tf32 256-tile epilogue", epi, bias_mode)
    C = host(ops().gemm(dev(A), dev(W), transB=True, precision=cd.PREC_TF32MODE,
                        bias=dev(bias) if bm else None, bias_mode=bm, epilogue=ep))
    rows = (1000, 1064)
    Z = oracle.dgemm(A, np.ascontiguousarray(W.T), rows=rows)
    if bias_mode == "row":
        Z = Z + bias[rows[0]:rows[1], None]
    elif bias_mode == "col":
        Z = Z + bias[None, :]
    want = oracle.activation(Z, epi)
    assert np.max(np.abs(C[rows[0]:rows[1]] - want)) <= 2e-5 * np.abs(Z).max() + 1e-6


@pytest.mark.parametrize("tA,tB", [(False, True), (True, False), (True, True)])
@pytest.mark.parametrize("prec_name", ["PREC_TF32MODE", "PREC_TF32MODE4"])
def test_tf32mode_transposes(tA, tB, prec_name):
    import cudeep_amd as cd
    rng = np.random.default_rng(305)
    M, N, K = 200, 300, 500
    A = normal(rng, (K, M) if tA else (M, K))
    B = normal(rng, (N, K) if tB else (K, N))
    say("tf32 transposes", tA, tB, prec_name)
    C = host(ops().gemm(dev(A), dev(B), transA=tA, transB=tB, precision=getattr(cd, prec_name)))
    C64 = oracle.dgemm(A, B, tA, tB)
    opA = A.T if tA else A
    opB = B.T if tB else B
    e_rne = oracle.rel_fro(oracle.gemm_tf32emu(np.ascontiguousarray(opA),
                                               np.ascontiguousarray(opB), "rne"), C64)
    assert oracle.rel_fro(C, C64) <= e_rne


# ---------------------------------------------------------------------------
# fused epilogues (bias per row / column, ReLU, GELU)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("mode", ["fp32", "tf32", "tf32x4"])
@pytest.mark.parametrize("epi", ["none", "relu", "gelu", "silu", "sigmoid"])
@pytest.mark.parametrize("bias_mode", ["none", "row", "col"])
def test_fused_epilogue(mode, epi, bias_mode):
    import cudeep_amd as cd
    rng = np.random.default_rng(401)
    M, N, K = 333, 257, 200
    A = normal(rng, (M, K))
    B = normal(rng, (K, N))
    bias = normal(rng, (M if bias_mode == "row" else N,))
    bm = {"none": cd.BIAS_NONE, "row": cd.BIAS_ROW, "col": cd.BIAS_COL}[bias_mode]
    ep = {"none": cd.EPI_NONE, "relu": cd.EPI_RELU, "gelu": cd.EPI_GELU,
          "silu": cd.EPI_SILU, "sigmoid": cd.EPI_SIGMOID}[epi]
    prec = {"fp32": cd.PREC_FP32, "tf32": cd.PREC_TF32MODE, "tf32x4": cd.PREC_TF32MODE4}[mode]
    say("epilogue", mode, epi, bias_mode)
    C = host(ops().gemm(dev(A), dev(B), precision=prec, bias=dev(bias) if bm else None,
                        bias_mode=bm, epilogue=ep))
    Z = oracle.dgemm(A, B)
    if bias_mode == "row":
        Z = Z + bias[:, None]
    elif bias_mode == "col":
        Z = Z + bias[None, :]
    want = Z if epi == "none" else oracle.activation(Z, epi)
    scale = np.abs(Z).max()
    # GEMM error (<= ~1e-6 relative) plus the epilogue's own few-ulp error
    assert np.max(np.abs(C - want)) <= 2e-5 * scale + 1e-6


def test_matmul_fused_act_entry_point():
    import ctypes
    import torch
    from cudeep_amd import _lib as L
    rng = np.random.default_rng(402)
    A = normal(rng, (128, 64))
    B = normal(rng, (64, 96))
    dA, dB = dev(A), dev(B)
    out = torch.empty((128, 96), device="cuda")
    say("matmul_fused_act relu")
    L.call("cdx_matmul_fused_act", dA.data_ptr(), dB.data_ptr(), out.data_ptr(), 128, 96, 64,
           L.EPI_RELU, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    C = host(out)
    Z = oracle.dgemm(A, B)
    want = oracle.relu(Z)
    # TF32 mode (bf16x3): per-product relative error <= ~3 * 2^-16
    assert np.max(np.abs(C - want)) <= 2e-5 * np.abs(Z).max()


# ---------------------------------------------------------------------------
# fp64 GEMM, degenerate shapes
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("tA,tB", [(False, False), (True, True), (False, True)])
def test_dgemm(tA, tB):
    rng = np.random.default_rng(501)
    M, N, K = 129, 77, 300
    A = rng.standard_normal((K, M) if tA else (M, K))
    B = rng.standard_normal((N, K) if tB else (K, N))
    say("dgemm", tA, tB)
    C = host(ops().dgemm(dev(A), dev(B), tA, tB))
    want = (A.T if tA else A) @ (B.T if tB else B)
    assert np.allclose(C, want, rtol=1e-12, atol=1e-12)


def test_k_zero_gives_bias_only():
    import torch
    import cudeep_amd as cd
    say("K=0")
    A = torch.empty((5, 0), device="cuda")
    B = torch.empty((0, 7), device="cuda")
    bias = torch.arange(7, dtype=torch.float32, device="cuda")
    for prec in (cd.PREC_FP32, cd.PREC_TF32MODE):
        C = host(ops().gemm(A, B, precision=prec, bias=bias, bias_mode=cd.BIAS_COL))
        assert np.array_equal(C, np.tile(np.arange(7, dtype=np.float32), (5, 1)))


def test_leading_dimension_views():
    """op(A) with lda > K: a column window of a wider matrix."""
    rng = np.random.default_rng(502)
    big = normal(rng, (200, 300))
    B = normal(rng, (120, 90))
    dbig = dev(big)
    view = dbig[:, 40:160]          # 200 x 120, lda = 300
    say("lda view")
    C = host(ops().gemm(view, dev(B)))
    C64 = oracle.dgemm(big[:, 40:160], B)
    _, e_ref = _ref_errors(np.ascontiguousarray(big[:, 40:160]), B)
    assert oracle.rel_fro(C, C64) <= 2 * e_ref


# ---------------------------------------------------------------------------
# split-K (few output tiles, long K): partial slices + ordered reduction
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("M,N,K,tA", [(64, 64, 8192, False), (100, 50, 5000, False),
                                      (256, 784, 8192, True), (10, 256, 8192, True),
                                      (33, 17, 3001, True), (200, 300, 4096, False)])
@pytest.mark.parametrize("mode", ["fp32", "tf32", "tf32x4"])
def test_split_k_parity(M, N, K, tA, mode):
    import cudeep_amd as cd
    rng = np.random.default_rng(M + N + K)
    A = normal(rng, (K, M) if tA else (M, K))
    B = normal(rng, (K, N))
    bias = normal(rng, (N,))
    prec = {"fp32": cd.PREC_FP32, "tf32": cd.PREC_TF32MODE, "tf32x4": cd.PREC_TF32MODE4}[mode]
    say("split-K", mode, M, N, K, tA)
    C = host(ops().gemm(dev(A), dev(B), transA=tA, precision=prec, bias=dev(bias),
                        bias_mode=cd.BIAS_COL, epilogue=cd.EPI_RELU))
    Z64 = oracle.dgemm(A, B, transA=tA) + bias[None, :]
    want = oracle.relu(Z64)
    if mode == "fp32":
        Zs = oracle.sgemm_seqfma(A, B, transA=tA) + bias[None, :]
        e_ref = oracle.rel_fro(oracle.relu(Zs.astype(np.float32)), want)
        assert oracle.rel_fro(C, want) <= 2 * e_ref
    else:
        opA = np.ascontiguousarray(A.T if tA else A)
        Zt = oracle.gemm_tf32emu(opA, B, "rne") + bias[None, :]
        e_ref = oracle.rel_fro(oracle.relu(Zt.astype(np.float32)), want)
        assert oracle.rel_fro(C, want) <= e_ref


@pytest.mark.parametrize("epi", ["relu", "gelu", "silu", "sigmoid"])
@pytest.mark.parametrize("bias_mode", ["col", "row"])
@pytest.mark.parametrize("mode", ["fp32", "tf32"])
def test_split_k_epilogue_equals_unsplit(epi, bias_mode, mode):
    """The split-K reduction applies bias + activation with the same float
    operations as the GEMM kernels' own epilogue.  P = A B (split, no
    epilogue) is pushed through an unsplit FP32 GEMM P I_N (exact: products
    with 1 and 0, sums with 0), whose epilogue must then equal the split
    GEMM's epilogue bit for bit."""
    import cudeep_amd as cd
    M, N, K = 64, 64, 8192
    rng = np.random.default_rng(17)
    A = normal(rng, (M, K), 0.05)
    B = normal(rng, (K, N))
    bias = normal(rng, (M if bias_mode == "row" else N,))
    prec = cd.PREC_FP32 if mode == "fp32" else cd.PREC_TF32MODE
    bm = cd.BIAS_ROW if bias_mode == "row" else cd.BIAS_COL
    code = {"relu": cd.EPI_RELU, "gelu": cd.EPI_GELU, "silu": cd.EPI_SILU,
            "sigmoid": cd.EPI_SIGMOID}[epi]
    assert ops().gemm_workspace_bytes(M, N, K, precision=prec) > 0     # it does split
    assert ops().gemm_workspace_bytes(M, N, N) == 0                     # this one does not
    say("split-K epilogue", epi, bias_mode, mode)
    dA, dB, db = dev(A), dev(B), dev(bias)
    fused = host(ops().gemm(dA, dB, precision=prec, bias=db, bias_mode=bm, epilogue=code))
    P = ops().gemm(dA, dB, precision=prec)
    eye = dev(np.eye(N, dtype=np.float32))
    unsplit = host(ops().gemm(P, eye, bias=db, bias_mode=bm, epilogue=code))
    assert np.array_equal(fused.view(np.uint32), unsplit.view(np.uint32))


# ---------------------------------------------------------------------------
# special values
# ---------------------------------------------------------------------------

def _special_operands(M, N, K, seed):
    rng = np.random.default_rng(seed)
    A = normal(rng, (M, K))
    B = normal(rng, (K, N))
    A[3, 5] = np.inf
    A[7, 1] = -np.inf
    A[11, 2] = np.nan
    return A, B


@pytest.mark.parametrize("M,N,K", [(64, 64, 64), (300, 200, 784), (4096, 4096, 64)])
def test_fp32_special_values_follow_ieee(M, N, K):
    """FP32 mode: +-Inf and NaN operands propagate as in IEEE fp64 arithmetic on the
    same operands (each output is one sum of products): the same Inf / NaN pattern and
    signs, and the finite outputs within the usual FP32 gate."""
    A, B = _special_operands(M, N, K, 808 + M)
    say("fp32 special values", M, N, K)
    C = host(ops().gemm(dev(A), dev(B)))
    with np.errstate(invalid="ignore", over="ignore"):
        C64 = A.astype(np.float64) @ B.astype(np.float64)
    assert np.array_equal(np.isnan(C), np.isnan(C64))
    assert np.array_equal(np.isinf(C), np.isinf(C64))
    inf = np.isinf(C64)
    assert np.array_equal(np.sign(C[inf]), np.sign(C64[inf]))
    fin = np.isfinite(C64).all(axis=1)
    Af = A[fin]
    Cs = oracle.sgemm_seqfma(Af, B)
    e_ref = oracle.rel_fro(Cs, C64[fin])
    assert oracle.rel_fro(C[fin], C64[fin]) <= 2 * e_ref + (F32_FLOOR if K < 64 else 0.0)


# beyond bf16's rounding limit (the split's hi part rounds to Inf) but well
# inside TF32's finite range under both RZ and RNE
HUGE = np.float32(3.4e38)


def _tf32_special_operands(M, N, K, seed):
    """Operands with +-Inf, NaN and beyond-bf16 finite elements in A (rows) and
    B (columns).  The k-rows / k-columns that multiply the huge values hold
    +-0.25 (products ~8.5e37: finite by a wide margin) and +-2 (products
    ~6.8e38: overflow by a wide margin), so every output's class (finite,
    +-Inf, NaN) is the same under any rounding of the operands or order of
    the sum."""
    rng = np.random.default_rng(seed)
    A = normal(rng, (M, K))
    B = normal(rng, (K, N))
    kh, kb = 9 % K, 16 % K
    pat_n = np.array([0.25, -0.25, 2.0, -2.0], np.float32)[np.arange(N) % 4]
    pat_m = np.array([0.25, 2.0, -0.25, -2.0], np.float32)[np.arange(M) % 4]
    B[kh, :] = pat_n
    A[:, kb] = pat_m
    A[3, 5 % K] = np.inf
    A[7, 1] = -np.inf
    A[11, 2] = np.nan
    A[13, kh] = HUGE
    A[17, kh] = -HUGE
    B[4 % K, 6] = np.inf
    B[8 % K, 10] = -np.inf
    B[12 % K, 14] = np.nan
    B[kb, 18] = HUGE
    B[kb, 22] = -HUGE
    return A, B


def _classes(C):
    return np.isnan(C), np.isinf(C), np.sign(np.where(np.isinf(C), C, 0))


@pytest.mark.parametrize("M,N,K,tA,tB", [
    (64, 64, 64, False, False),
    (300, 200, 784, False, False),       # ragged tiles (bounds-checked kernel)
    (300, 200, 784, True, True),         # both operands transposed
    (128, 128, 4096, False, False),      # split-K slices repair their own k-range
    (4096, 4096, 64, False, False),      # two-group 256 x 256 kernel (four terms: k-alternating)
    (4096, 4096, 64, True, False),
    (2048, 2048, 96, False, False),      # k-alternating 128 x 128 kernel, odd k-tile count
    (2048, 2048, 96, True, True),
])
def test_tf32mode_special_values_follow_reference(M, N, K, tA, tB):
    """TF32 modes: +-Inf, NaN and finite operands beyond bf16's range give the
    reference TF32 kernel's results (matmul_kernel.cu:186-201 feeds raw fp32
    bits to the MMA): the NaN / Inf pattern and the Inf signs equal those of
    oracle.gemm_tf32emu (which agrees under RZ and RNE on these operands), and
    outputs untouched by a special operand stay inside the TF32-mode gate."""
    import cudeep_amd as cd
    A, B = _tf32_special_operands(M, N, K, 909 + M + K)
    rows = [(0, 64)] if M <= 64 else [(0, 64), (M - 64, M)]
    want = {}
    for r in rows:
        with np.errstate(invalid="ignore", over="ignore"):
            rz = oracle.gemm_tf32emu(A, B, "rz", rows=r)
            rne = oracle.gemm_tf32emu(A, B, "rne", rows=r)
        for x, y in zip(_classes(rz), _classes(rne)):
            assert np.array_equal(x, y)          # the expectation is unambiguous
        want[r] = rz
    touched_rows = ~np.isfinite(A).all(axis=1) | (np.abs(A) >= HUGE).any(axis=1)
    touched_cols = ~np.isfinite(B).all(axis=0) | (np.abs(B) >= HUGE).any(axis=0)
    clean_cols = ~touched_cols
    Ad = dev(np.ascontiguousarray(A.T) if tA else A)
    Bd = dev(np.ascontiguousarray(B.T) if tB else B)
    for prec in (cd.PREC_TF32MODE, cd.PREC_TF32MODE4):
        say("tf32 special values", M, N, K, tA, tB, prec)
        C = host(ops().gemm(Ad, Bd, precision=prec, transA=tA, transB=tB))
        for r, ref in want.items():
            got = C[r[0]:r[1]]
            for kind, x, y in zip(("nan", "inf", "sign"), _classes(got), _classes(ref)):
                assert np.array_equal(x, y), (prec, r, kind, np.argwhere(x != y)[:5])
        # outputs without a special operand: finite, and inside the gate
        clean_rows = ~touched_rows
        assert np.isfinite(C[np.ix_(clean_rows, clean_cols)]).all()
        r0, r1 = rows[0]
        sel = clean_rows[r0:r1]
        Ag = A[r0:r1][sel]
        C64 = oracle.dgemm(Ag, B)[:, clean_cols]
        e = oracle.rel_fro(C[r0:r1][sel][:, clean_cols], C64)
        e_ref = min(oracle.rel_fro(oracle.gemm_tf32emu(Ag, B, m)[:, clean_cols], C64)
                    for m in ("rz", "rne"))
        assert e <= e_ref, (prec, e, e_ref)
