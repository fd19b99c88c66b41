"""Seeded random sweep of the GEMM entry point (cdx_gemm_ex_ws through
cudeep_amd.ops.gemm): shapes 1..300 in each dimension, all four transposes,
operands and output as row-strided views of larger buffers (leading dimension
> row length), every precision mode, bias mode and epilogue.

Gates: FP32 relFro vs fp64 <= 2 x the seq-FMA restatement of the reference
SGEMM (+ a floor for very short K); TF32 modes <= the emulated reference TF32
error (min over RZ / RNE operand rounding) + the same floor; bias and
activation applied to the fp64 product before the comparison.  Every element
of the output buffer outside the view must be left exactly as it was (no
out-of-bounds or padding writes)."""
import numpy as np
import pytest

import oracle
from tests.gpu_util import F32_FLOOR, require_gpu, say

pytestmark = pytest.mark.gpu

_EPIS = ["none", "relu", "gelu", "silu", "sigmoid"]


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    require_gpu()
    import cudeep_amd.ops  # noqa: F401  (loads libcudeep_amd.so)


def _strided(rng, rows, cols, pad):
    """A rows x cols view (unit column stride, row stride cols + pad) of a
    larger N(0, 1) device buffer, and its dense host copy."""
    import torch
    full = rng.standard_normal((rows, cols + pad)).astype(np.float32)
    t = torch.from_numpy(full).cuda()[:, :cols]
    return t, np.ascontiguousarray(full[:, :cols])


@pytest.mark.parametrize("seed", range(12))
def test_gemm_random_sweep(seed):
    import torch
    import cudeep_amd as cd
    import cudeep_amd.ops as o
    rng = np.random.default_rng(9000 + seed)
    precs = [cd.PREC_FP32, cd.PREC_TF32MODE, cd.PREC_TF32MODE4]
    for case in range(6):
        M, N, K = (int(v) for v in rng.integers(1, 301, 3))
        tA, tB = bool(rng.integers(2)), bool(rng.integers(2))
        prec = precs[int(rng.integers(3))]
        epi = _EPIS[int(rng.integers(len(_EPIS)))]
        bias_mode = int(rng.integers(3))   # none / row / col
        pads = [int(v) for v in rng.integers(0, 9, 3)]
        say("sweep", seed, case, M, N, K, tA, tB, prec, epi, bias_mode, pads)
        A, A32 = _strided(rng, K if tA else M, M if tA else K, pads[0])
        B, B32 = _strided(rng, N if tB else K, K if tB else N, pads[1])
        # output view inside a sentinel-filled buffer
        sentinel = np.float32(-7.25)
        cbuf = torch.full((M, N + pads[2]), float(sentinel), device="cuda")
        C = cbuf[:, :N]
        bias = None
        b64 = 0.0
        if bias_mode != cd.BIAS_NONE:
            nb = M if bias_mode == cd.BIAS_ROW else N
            bh = (rng.standard_normal(nb) * 0.5).astype(np.float32)
            bias = torch.from_numpy(bh).cuda()
            b64 = bh[:, None] if bias_mode == cd.BIAS_ROW else bh[None, :]
        code = {"none": cd.EPI_NONE, "relu": cd.EPI_RELU, "gelu": cd.EPI_GELU,
                "silu": cd.EPI_SILU, "sigmoid": cd.EPI_SIGMOID}[epi]
        o.gemm(A, B, precision=prec, transA=tA, transB=tB, bias=bias, bias_mode=bias_mode,
               epilogue=code, out=C)
        got_full = cbuf.cpu().numpy()
        assert np.all(got_full[:, N:] == sentinel), "write outside the output view"
        got = got_full[:, :N]
        C64 = oracle.dgemm(A32, B32, tA, tB)
        opA = A32.T if tA else A32
        opB = B32.T if tB else B32
        if prec == cd.PREC_FP32:
            ref_err_src = oracle.sgemm_seqfma(A32, B32, tA, tB)
        else:
            ref_err_src = min((oracle.gemm_tf32emu(np.ascontiguousarray(opA),
                                                   np.ascontiguousarray(opB), m)
                               for m in ("rz", "rne")),
                              key=lambda c: oracle.rel_fro(c, C64))
        pre64 = C64 + b64
        pre_ref = ref_err_src.astype(np.float64) + b64
        want = pre64 if epi == "none" else oracle.activation(pre64, epi)
        ref = pre_ref if epi == "none" else oracle.activation(pre_ref, epi)
        e_ref = oracle.rel_fro(ref, want)
        e = oracle.rel_fro(got, want)
        floor = F32_FLOOR if K < 64 else 2.0 ** -22
        bound = (2 * e_ref if prec == cd.PREC_FP32 else e_ref) + floor
        assert e <= bound, (seed, case, M, N, K, tA, tB, prec, epi, bias_mode, e, e_ref)
