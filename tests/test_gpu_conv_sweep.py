"""Seeded random sweep of conv backward weight and data (cdx_conv2d_backward_*
through cudeep_amd.ops), the im2col forward and the implicit forward: mostly 3x3 stride-1 layers
with random widths (1 .. 130: one or two row segments of the row-window
weight-gradient kernel), pads 0 .. 2, channel counts off the 16-channel and
64-channel tile sizes, plus other kernel sizes and strides.  FP32 mode gates:
<= 2 x the error of the reference's routes restated on the CPU (im2col +
seq-FMA GEMM), against fp64."""
import numpy as np
import pytest

import oracle
from tests.gpu_util import dev, host, normal, require_gpu, say

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    require_gpu()
    import cudeep_amd.ops  # noqa: F401  (loads libcudeep_amd.so)


def _geometry(rng):
    if rng.random() < 0.75:
        KH = KW = 3
        SH = SW = 1
        PH, PW = (int(v) for v in rng.integers(0, 3, 2))
    else:
        KH, KW = (int(v) for v in rng.integers(1, 6, 2))
        SH, SW = (int(v) for v in rng.integers(1, 3, 2))
        PH, PW = int(rng.integers(0, KH)), int(rng.integers(0, KW))
    Bn = int(rng.integers(1, 4))
    C = int(rng.integers(1, 41))
    OC = int(rng.integers(1, 81))
    H = int(rng.integers(max(1, KH - 2 * PH), 12))
    W = int(rng.integers(max(1, KW - 2 * PW), 131))
    return Bn, C, H, W, OC, KH, KW, SH, SW, PH, PW


@pytest.mark.parametrize("seed", range(10))
def test_conv_random_sweep(seed):
    import cudeep_amd.ops as o
    rng = np.random.default_rng(7100 + seed)
    for case in range(4):
        Bn, C, H, W, OC, KH, KW, SH, SW, PH, PW = g = _geometry(rng)
        OH = oracle.conv_out_size(H, KH, SH, PH)
        OW = oracle.conv_out_size(W, KW, SW, PW)
        x = normal(rng, (Bn, C, H, W))
        w = normal(rng, (OC, C, KH, KW), std=np.sqrt(2.0 / (C * KH * KW)))
        dy = normal(rng, (Bn, OC, OH, OW))
        st, pd = (SH, SW), (PH, PW)
        say("conv sweep", seed, case, g)
        dw = host(o.conv2d_backward_weight(dev(dy), dev(x), w.shape, st, pd))
        dw64 = oracle.conv2d_backward_weight64(dy, x, w.shape, st, pd)
        ew_ref = oracle.rel_fro(oracle.conv2d_backward_weight_ref(dy, x, w.shape, st, pd), dw64)
        assert oracle.rel_fro(dw, dw64) <= 2 * ew_ref + 2.0 ** -24, (g, "weight")
        dx = host(o.conv2d_backward_data(dev(dy), dev(w), x.shape, st, pd))
        dx64 = oracle.conv2d_backward_data64(dy, w, x.shape, st, pd)
        ex_ref = oracle.rel_fro(oracle.conv2d_backward_data_ref(dy, w, x.shape, st, pd), dx64)
        assert oracle.rel_fro(dx, dx64) <= 2 * ex_ref + 2.0 ** -24, (g, "data")
        y = host(o.conv2d_forward(dev(x), dev(w), None, st, pd))
        y64 = oracle.conv2d_direct64(x, w, None, st, pd)
        ey_ref = oracle.rel_fro(oracle.conv2d_ref_im2col(x, w, None, st, pd), y64)
        assert oracle.rel_fro(y, y64) <= 2 * ey_ref + 2.0 ** -24, (g, "forward")
        # implicit forward (the row-window kernel wherever its window fits)
        b = normal(rng, (OC,), 0.1)
        yi = host(o.conv2d_implicit(dev(x), dev(w), dev(b), st, pd))
        yi64 = oracle.conv2d_direct64(x, w, b, st, pd)
        ei_ref = oracle.rel_fro(oracle.conv2d_ref_implicit(x, w, b, st, pd), yi64)
        assert oracle.rel_fro(yi, yi64) <= 2 * ei_ref + 2.0 ** -24, (g, "implicit forward")
