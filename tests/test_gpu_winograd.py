"""Winograd F(4x4, 3x3) conv forward (cdx_conv2d_forward_winograd_f32) vs the
oracle: the fp64 form of the same algorithm equals direct convolution (pinned in
test_oracle.py) and is the yardstick; the gate is the error of the reference's
route restated on the CPU (fp32 transforms + seq-FMA GEMMs; in TF32 mode, GEMM
operands rounded to TF32 under RZ or RNE, whichever errs less)."""
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


def _gate(x, w, b, pad, prec):
    """(fp64 yardstick, allowed relFro) for one problem."""
    import cudeep_amd as cd
    y64 = oracle.conv2d_winograd(x, w, b, padding=pad, double=True)
    if prec == cd.PREC_FP32:
        e_ref = oracle.rel_fro(oracle.conv2d_winograd(x, w, b, padding=pad), y64)
        return y64, 2 * e_ref
    e_rz = oracle.rel_fro(oracle.conv2d_winograd(x, w, b, padding=pad, tf32="rz"), y64)
    e_rne = oracle.rel_fro(oracle.conv2d_winograd(x, w, b, padding=pad, tf32="rne"), y64)
    return y64, min(e_rz, e_rne)


def test_winograd_reference_kats(kats):
    for name in ("conv_3x3_ones", "conv_3x3_bias", "conv_3x3_pad1"):
        k = kats[name]
        x = np.array(k["x"], np.float32).reshape(k["x_shape"])
        w = np.array(k["w"], np.float32).reshape(k["w_shape"])
        b = np.array(k["bias"], np.float32) if k.get("bias") is not None else None
        say("winograd kat", name)
        y = host(ops().conv2d_winograd(dev(x), dev(w), None if b is None else dev(b),
                                       padding=tuple(k["padding"])))
        assert np.allclose(y, np.array(k["y"], np.float32).reshape(y.shape), rtol=0, atol=1e-5)


SHAPES = [(1, 1, 1, 3, 3, 0), (2, 3, 4, 9, 11, 1), (1, 5, 2, 6, 6, 0), (2, 8, 8, 16, 16, 1),
          (1, 1, 1, 7, 5, 2), (3, 16, 24, 13, 17, 1), (2, 64, 64, 28, 28, 1),
          (1, 33, 65, 10, 30, 0), (4, 128, 32, 14, 14, 1)]


@pytest.mark.parametrize("B,IC,OC,H,W,P", SHAPES)
@pytest.mark.parametrize("mode", ["fp32", "tf32"])
def test_winograd_parity(B, IC, OC, H, W, P, mode):
    import cudeep_amd as cd
    prec = cd.PREC_FP32 if mode == "fp32" else cd.PREC_TF32MODE
    rng = np.random.default_rng(B * 1000 + IC * 10 + H + P)
    x = normal(rng, (B, IC, H, W))
    w = normal(rng, (OC, IC, 3, 3), std=(2.0 / (9 * IC)) ** 0.5)
    b = normal(rng, (OC,), 0.1)
    say("winograd", mode, B, IC, OC, H, W, P)
    y = host(ops().conv2d_winograd(dev(x), dev(w), dev(b), padding=(P, P), precision=prec))
    y64, tol = _gate(x, w, b, (P, P), prec)
    assert y.shape == y64.shape
    assert oracle.rel_fro(y, y64) <= tol, (oracle.rel_fro(y, y64), tol)


@pytest.mark.parametrize("mode", ["fp32", "tf32"])
def test_winograd_c5_full(mode):
    """C5 (N=32, C=64, 56x56 -> 64, pad 1), whole output."""
    import cudeep_amd as cd
    prec = cd.PREC_FP32 if mode == "fp32" else cd.PREC_TF32MODE
    rng = np.random.default_rng(55)
    x = normal(rng, (32, 64, 56, 56))
    w = normal(rng, (64, 64, 3, 3), std=(2.0 / 576) ** 0.5)
    b = normal(rng, (64,), 0.1)
    say("winograd C5", mode)
    y = host(ops().conv2d_winograd(dev(x), dev(w), dev(b), padding=(1, 1), precision=prec))
    y64, tol = _gate(x, w, b, (1, 1), prec)
    e = oracle.rel_fro(y, y64)
    print(f"winograd C5 {mode}: relFro {e:.3e} gate {tol:.3e}")
    assert e <= tol


def test_winograd_workspace_paths():
    from cudeep_amd import _lib as L
    import torch
    rng = np.random.default_rng(7)
    x = normal(rng, (2, 8, 12, 12))
    w = normal(rng, (4, 8, 3, 3), 0.2)
    need = ops().conv2d_winograd_workspace_bytes(x.shape, 4, (1, 1))
    assert need == 36 * (4 * 8 + 8 * 2 * 9 + 4 * 2 * 9) * 4
    say("winograd workspace")
    ws = torch.empty(need // 4, device="cuda")
    y1 = host(ops().conv2d_winograd(dev(x), dev(w), padding=(1, 1), workspace=ws))
    y2 = host(ops().conv2d_winograd(dev(x), dev(w), padding=(1, 1)))
    assert np.array_equal(y1, y2)
    small = torch.empty(need // 4 - 1, device="cuda")
    with pytest.raises(L.CdxError):
        ops().conv2d_winograd(dev(x), dev(w), padding=(1, 1), workspace=small)


# ---------------------------------------------------------------------------
# backward data by Winograd on the transposed convolution
# ---------------------------------------------------------------------------

def _bwd_gate(dy, w, x_shape, pad, prec):
    """(fp64 grad_input, allowed relFro): the fp64 gradient is pinned against
    torch in test_oracle.py; the gate is the CPU Winograd restatement of the
    same transposed convolution (fp32, or TF32 operands under RZ / RNE)."""
    import cudeep_amd as cd
    d64 = oracle.conv2d_backward_data64(dy, w, x_shape, (1, 1), pad)
    if prec == cd.PREC_FP32:
        e = oracle.rel_fro(oracle.conv2d_backward_data_winograd(dy, w, x_shape, pad), d64)
        return d64, 2 * e
    e = min(oracle.rel_fro(oracle.conv2d_backward_data_winograd(dy, w, x_shape, pad, tf32=m), d64)
            for m in ("rz", "rne"))
    return d64, e


BWD_SHAPES = [(1, 1, 1, 3, 3, 0), (2, 3, 4, 9, 11, 1), (1, 5, 2, 6, 6, 2), (2, 8, 8, 16, 16, 1),
              (1, 1, 1, 7, 5, 2), (3, 16, 24, 13, 17, 1), (2, 64, 64, 28, 28, 1),
              (1, 33, 65, 10, 30, 0), (4, 128, 32, 14, 14, 1)]


@pytest.mark.parametrize("B,IC,OC,H,W,P", BWD_SHAPES)
@pytest.mark.parametrize("mode", ["fp32", "tf32"])
def test_winograd_backward_data_parity(B, IC, OC, H, W, P, mode):
    import cudeep_amd as cd
    prec = cd.PREC_FP32 if mode == "fp32" else cd.PREC_TF32MODE
    rng = np.random.default_rng(B * 1000 + IC * 10 + H + P + 7)
    w = normal(rng, (OC, IC, 3, 3), std=(2.0 / (9 * IC)) ** 0.5)
    OH, OW = H + 2 * P - 2, W + 2 * P - 2
    dy = normal(rng, (B, OC, OH, OW))
    say("winograd bwd data", mode, B, IC, OC, H, W, P)
    dx = host(ops().conv2d_backward_data_winograd(dev(dy), dev(w), (B, IC, H, W), (P, P),
                                                  precision=prec))
    d64, tol = _bwd_gate(dy, w, (B, IC, H, W), (P, P), prec)
    assert dx.shape == d64.shape
    assert oracle.rel_fro(dx, d64) <= tol, (oracle.rel_fro(dx, d64), tol)


def test_winograd_backward_data_workspace():
    """Caller workspace of exactly the queried size gives the same bits as
    the library-allocated one, on two calls in a row."""
    import torch
    rng = np.random.default_rng(77)
    w = normal(rng, (6, 5, 3, 3), 0.2)
    dy = normal(rng, (2, 6, 9, 12))
    x_shape = (2, 5, 9, 12)
    nbytes = ops().conv2d_backward_data_winograd_workspace_bytes(x_shape, 6, (1, 1))
    assert nbytes > 0
    ws = torch.empty(nbytes // 4, dtype=torch.float32, device="cuda")
    say("winograd bwd data workspace", nbytes)
    a = host(ops().conv2d_backward_data_winograd(dev(dy), dev(w), x_shape, (1, 1), workspace=ws))
    b = host(ops().conv2d_backward_data_winograd(dev(dy), dev(w), x_shape, (1, 1)))
    assert np.array_equal(a, b)


@pytest.mark.parametrize("mode", ["fp32", "tf32"])
def test_winograd_backward_data_c5(mode):
    """C5 backward data (N=32, C=64, 56x56, OC=64, pad 1), whole batch run;
    batch items 0 and 31 checked against the fp64 gradient."""
    import cudeep_amd as cd
    prec = cd.PREC_FP32 if mode == "fp32" else cd.PREC_TF32MODE
    rng = np.random.default_rng(5152)
    w = normal(rng, (64, 64, 3, 3), std=(2.0 / 576) ** 0.5)
    dy = normal(rng, (32, 64, 56, 56))
    say("winograd bwd data C5", mode)
    dx = host(ops().conv2d_backward_data_winograd(dev(dy), dev(w), (32, 64, 56, 56), (1, 1),
                                                  precision=prec))
    for i in (0, 31):
        d64, tol = _bwd_gate(dy[i:i + 1], w, (1, 64, 56, 56), (1, 1), prec)
        assert oracle.rel_fro(dx[i:i + 1], d64) <= tol
