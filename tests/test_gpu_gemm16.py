"""FP16 / BF16 GEMM (cdx_hgemm_f16, cdx_gemm16_ex) on the GPU vs the oracle.

The reference's fp16 path is hgemm_tc_kernel (src/kernels/matmul_kernel.cu:745-930,
launched by launch_matmul_kernel_fp16 :1926-1943): fp16 A, B, exact products, fp32
accumulation in 16-term MMA k-steps, fp32 C.  Its "ideal MMA" error is reproduced on
the CPU by oracle.gemm_tf32emu on the fp32-converted operands: TF32 rounding leaves
fp16 / bf16 values unchanged (at most 11 significant bits), so the emulation forms the
exact products and rounds once per 8-term chunk.  Gate: relFro vs fp64 <= 2x that
error (the same factor as the FP32 SGEMM gate)."""
import numpy as np
import pytest

import oracle
from tests.gpu_util import dev, host, require_gpu, say

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    require_gpu()


def ops():
    import cudeep_amd.ops as o
    return o


def _operands(rng, shape, dtype):
    """Random N(0,1) operand as (device tensor, exact float32 host copy)."""
    import torch
    x = torch.from_numpy(rng.standard_normal(shape).astype(np.float32))
    x = x.to(torch.float16 if dtype == "f16" else torch.bfloat16)
    return x.cuda(), x.float().numpy()


def _ideal_err(A32, B32, C64):
    return oracle.rel_fro(oracle.gemm_tf32emu(np.ascontiguousarray(A32),
                                              np.ascontiguousarray(B32), "rne"), C64)


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_gemm16_kats_exact(kats, dtype):
    import torch
    td = torch.float16 if dtype == "f16" else torch.bfloat16
    for name in ("matmul_2x2", "matmul_diag_identity", "mma_identity", "mma_integer_pattern"):
        k = kats[name]
        A = torch.tensor(k["A"], dtype=torch.float32)
        B = torch.tensor(k["B"], dtype=torch.float32)
        if dtype == "bf16" and max(A.abs().max(), B.abs().max()) > 256:
            continue          # bf16 holds integers exactly only up to 256
        say("gemm16 kat", dtype, name)
        C = host(ops().gemm16(A.to(td).cuda(), B.to(td).cuda()))
        assert np.array_equal(C, np.array(k["C"], np.float32)), name


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_gemm16_integer_exact(dtype):
    import torch
    rng = np.random.default_rng(61)
    td = torch.float16 if dtype == "f16" else torch.bfloat16
    for (M, N, K) in [(16, 8, 8), (130, 70, 200), (256, 256, 64), (513, 129, 1000)]:
        A = rng.integers(-8, 9, (M, K)).astype(np.float32)
        B = rng.integers(-8, 9, (K, N)).astype(np.float32)
        say("gemm16 integer", dtype, M, N, K)
        C = host(ops().gemm16(torch.from_numpy(A).to(td).cuda(), torch.from_numpy(B).to(td).cuda()))
        assert np.array_equal(C, A.astype(np.float64) @ B)


SHAPES16 = [(1, 1, 1), (17, 33, 65), (64, 64, 64), (127, 255, 33), (300, 200, 784),
            (8192, 10, 256), (64, 4096, 576), (256, 512, 1000), (1024, 1024, 1024)]


@pytest.mark.parametrize("M,N,K", SHAPES16)
@pytest.mark.parametrize("tA,tB", [(False, False), (False, True), (True, False), (True, True)])
@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_gemm16_parity_shapes(M, N, K, tA, tB, dtype):
    rng = np.random.default_rng(M * 7 + N * 3 + K + int(tA) * 2 + int(tB))
    A, A32 = _operands(rng, (K, M) if tA else (M, K), dtype)
    B, B32 = _operands(rng, (N, K) if tB else (K, N), dtype)
    say("gemm16", dtype, M, N, K, tA, tB)
    C = host(ops().gemm16(A, B, transA=tA, transB=tB))
    C64 = oracle.dgemm(A32, B32, tA, tB)
    e = oracle.rel_fro(C, C64)
    e_ideal = _ideal_err(A32.T if tA else A32, B32.T if tB else B32, C64)
    assert e <= 2 * e_ideal + 2.0 ** -24, (e, e_ideal)


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_gemm16_4096_sampled_rows(dtype):
    rng = np.random.default_rng(64)
    n = 4096
    A, A32 = _operands(rng, (n, n), dtype)
    B, B32 = _operands(rng, (n, n), dtype)
    say("gemm16 4096", dtype)
    C = host(ops().gemm16(A, B))
    for r0 in (0, 2048, n - 64):
        rows = (r0, r0 + 64)
        C64 = oracle.dgemm(A32, B32, rows=rows)
        e = oracle.rel_fro(C[r0:r0 + 64], C64)
        e_ideal = oracle.rel_fro(oracle.gemm_tf32emu(A32, B32, "rne", rows=rows), C64)
        print(f"gemm16 {dtype} 4096 rows {rows}: {e:.3e} ideal MMA {e_ideal:.3e}")
        assert e <= 2 * e_ideal
    # checksum identity e^T C = (e^T A) B over the whole matrix
    lhs = C.astype(np.float64).sum(0)
    rhs = A32.astype(np.float64).sum(0) @ B32.astype(np.float64)
    assert np.linalg.norm(lhs - rhs) / np.linalg.norm(rhs) < 1e-5


@pytest.mark.parametrize("tA,tB", [(False, False), (False, True), (True, False), (True, True)])
@pytest.mark.parametrize("K", [64, 128, 192, 1088])
@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_gemm16_256_tile_path(tA, tB, K, dtype):
    """The 256 x 256 two-group (ping-pong) kernel for 16-bit operands, which
    M = N = 4096 selects: K = 64 / 128 / 192 give one, two and three k-tiles,
    K = 1088 a longer loop; all four transposes.  Same gate as the other
    16-bit tests on sampled rows, plus the column-checksum identity."""
    rng = np.random.default_rng(2000 + K + 2 * tA + tB)
    n = 4096
    A, A32 = _operands(rng, (K, n) if tA else (n, K), dtype)
    B, B32 = _operands(rng, (n, K) if tB else (K, n), dtype)
    say("gemm16 256-tile path", dtype, tA, tB, K)
    C = host(ops().gemm16(A, B, transA=tA, transB=tB))
    opA = np.ascontiguousarray(A32.T if tA else A32)
    opB = np.ascontiguousarray(B32.T if tB else B32)
    for r0 in (0, 1500, n - 48):
        rows = (r0, r0 + 48)
        C64 = oracle.dgemm(opA, opB, rows=rows)
        e = oracle.rel_fro(C[r0:r0 + 48], C64)
        e_ideal = oracle.rel_fro(oracle.gemm_tf32emu(opA, opB, "rne", rows=rows), C64)
        assert e <= 2 * e_ideal, (rows, e, e_ideal)
    lhs = C.astype(np.float64).sum(0)
    rhs = opA.astype(np.float64).sum(0) @ opB.astype(np.float64)
    assert np.linalg.norm(lhs - rhs) / np.linalg.norm(rhs) < 1e-5


@pytest.mark.parametrize("pad", [4, 8])
@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_gemm16_256_tile_padded_rows(pad, dtype):
    """M = N = 4096 with leading dimensions K + pad: rows at 8-element
    multiples (pad 8) take the two-group kernel, whose 16-bit loads move 8
    elements per lane; rows at 4-element multiples only (pad 4) fall back to
    the 256 x 256 in-step kernel.  Both against the oracle on sampled rows."""
    import torch
    from cudeep_amd import _lib as L
    rng = np.random.default_rng(3100 + pad)
    n, K = 4096, 192
    Ap, _ = _operands(rng, (n, K + pad), dtype)
    Bp, _ = _operands(rng, (K, n + pad), dtype)
    A32 = Ap.float().cpu().numpy()[:, :K]
    B32 = Bp.float().cpu().numpy()[:, :n]
    C = torch.empty((n, n), device="cuda")
    dt = L.DTYPE_F16 if dtype == "f16" else L.DTYPE_BF16
    say("gemm16 padded rows", dtype, pad)
    L.call("cdx_gemm16_ex", dt, 0, 0, n, n, K, Ap.data_ptr(), K + pad, Bp.data_ptr(), n + pad,
           C.data_ptr(), n, None, 0, 0, torch.cuda.current_stream().cuda_stream)
    Ch = host(C)
    opA, opB = np.ascontiguousarray(A32), np.ascontiguousarray(B32)
    for r0 in (0, 2000, n - 48):
        rows = (r0, r0 + 48)
        C64 = oracle.dgemm(opA, opB, rows=rows)
        e = oracle.rel_fro(Ch[r0:r0 + 48], C64)
        e_ideal = oracle.rel_fro(oracle.gemm_tf32emu(opA, opB, "rne", rows=rows), C64)
        assert e <= 2 * e_ideal, (rows, e, e_ideal)


def test_hgemm_entry_point_and_epilogue():
    import cudeep_amd as cd
    rng = np.random.default_rng(65)
    A, A32 = _operands(rng, (333, 200), "f16")
    B, B32 = _operands(rng, (200, 257), "f16")
    say("hgemm entry")
    C = host(ops().hgemm(A, B))
    C64 = oracle.dgemm(A32, B32)
    assert oracle.rel_fro(C, C64) <= 2 * _ideal_err(A32, B32, C64) + 2.0 ** -24
    bias = rng.standard_normal(257).astype(np.float32)
    for ep, name in ((cd.EPI_RELU, "relu"), (cd.EPI_GELU, "gelu"), (cd.EPI_SILU, "silu")):
        say("gemm16 epilogue", name)
        Cf = host(ops().gemm16(A, B, bias=dev(bias), bias_mode=cd.BIAS_COL, epilogue=ep))
        want = oracle.activation(C64 + bias[None, :], name)
        assert np.max(np.abs(Cf - want)) <= 2e-5 * np.abs(C64).max() + 1e-6


def test_gemm16_rejects_bad_dtype():
    import torch
    from cudeep_amd import _lib as L
    x = torch.zeros((4, 4), device="cuda", dtype=torch.float16)
    with pytest.raises(TypeError):
        ops().gemm16(x, x.float())
    with pytest.raises(L.CdxError):
        L.call("cdx_gemm16_ex", 7, 0, 0, 4, 4, 4, x.data_ptr(), 4, x.data_ptr(), 4,
               x.data_ptr(), 4, None, 0, 0, None)
