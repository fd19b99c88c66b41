"""GPU parity of im2col and the im2col-Conv2d forward.

  * im2col: bit-exact (compared as uint32 bit patterns) with the oracle's
    restatement of conv_kernel.cu:32-65, including the full C5 geometry.
  * conv forward: relFro vs the fp64 direct convolution <= 2 x that of the
    reference route restated on the CPU (im2col -> seq-FMA SGEMM ->
    transpose + bias); TF32 mode against the emulated TF32 route.
  * the reference's conv known answers (identity, 3x3 ones, bias, padding).
  * implicit-GEMM forward (the reference's route for large non-3x3 layers):
    relFro <= 2 x that of its bias-first FMA chain restated on the CPU,
    including a C5-size 7x7 layer routed there by cdx_conv2d_forward_f32.
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


GEOMS = [  # (B, C, H, W, KH, KW, SH, SW, PH, PW)
    (1, 1, 4, 4, 1, 1, 1, 1, 0, 0),
    (2, 3, 8, 9, 3, 3, 1, 1, 1, 1),
    (1, 2, 7, 7, 3, 5, 2, 1, 2, 0),
    (3, 4, 6, 5, 2, 1, 1, 1, 0, 0),       # spatial % 4 != 0 -> scalar stores
    (2, 5, 11, 13, 5, 5, 2, 2, 2, 2),
    (4, 16, 28, 28, 3, 3, 1, 1, 1, 1),
    (2, 8, 15, 17, 1, 1, 2, 2, 0, 0),
    (1, 3, 3, 3, 3, 3, 1, 1, 0, 0),       # single output pixel
    (1, 2, 130, 131, 3, 3, 1, 1, 1, 1),   # plane > 64 KiB -> generic gather kernel
    (2, 1, 129, 130, 3, 2, 2, 1, 0, 1),   # generic kernel, odd spatial
]


@pytest.mark.parametrize("g", GEOMS)
def test_im2col_bit_exact(g):
    Bn, C, H, W, KH, KW, SH, SW, PH, PW = g
    rng = np.random.default_rng(sum(g))
    x = normal(rng, (Bn, C, H, W))
    x[0, 0, 0, 0] = -0.0                   # sign of zero must survive
    say("im2col", g)
    col = host(ops().im2col(dev(x), KH, KW, (SH, SW), (PH, PW)))
    want = oracle.im2col(x, KH, KW, SH, SW, PH, PW)
    assert col.shape == want.shape
    assert np.array_equal(col.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("g", [
    # strides / paddings beyond 32 bits: the window origins ow*SW - PW need
    # 64-bit arithmetic (only output column 1 lands inside the image; cut
    # to 32 bits, SW = 2^32 + 1 and PW = 2^32 would read like 1 and 0)
    (1, 2, 4, 4, 1, 1, 1, 2**32 + 1, 0, 2**32),
    (1, 2, 4, 4, 1, 3, 1, 2**32 + 1, 1, 2**32),
    (1, 2, 4, 4, 1, 1, 1, 2**31 + 1, 0, 2**31),
    (2, 1, 4, 5, 3, 1, 2**32 + 1, 1, 2**32, 0),
])
def test_im2col_huge_stride_padding(g):
    Bn, C, H, W, KH, KW, SH, SW, PH, PW = g
    rng = np.random.default_rng(7)
    x = normal(rng, (Bn, C, H, W))
    say("im2col huge stride/padding", g)
    col = host(ops().im2col(dev(x), KH, KW, (SH, SW), (PH, PW)))
    want = oracle.im2col(x, KH, KW, SH, SW, PH, PW)
    assert col.shape == want.shape
    assert np.count_nonzero(want) > 0          # some taps inside the image
    assert np.array_equal(col.view(np.uint32), want.view(np.uint32))


def test_im2col_c5_full_bit_exact():
    """C5 geometry: N=32, C=64, 56x56, 3x3, s1, p1 -> col [576, 100352]."""
    rng = np.random.default_rng(555)
    x = normal(rng, (32, 64, 56, 56))
    say("im2col C5 full")
    col = host(ops().im2col(dev(x), 3, 3, (1, 1), (1, 1)))
    want = oracle.im2col(x, 3, 3, 1, 1, 1, 1)
    assert col.shape == (576, 100352)
    assert np.array_equal(col.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("name", ["conv_identity_1x1", "conv_3x3_ones", "conv_3x3_bias",
                                  "conv_3x3_pad1"])
@pytest.mark.parametrize("prec", [0, 1])
def test_conv_kats(kats, name, prec):
    k = kats[name]
    x = np.array(k["x"], np.float32).reshape(k["x_shape"])
    w = np.array(k["w"], np.float32).reshape(k["w_shape"])
    b = None if k["bias"] is None else dev(np.array(k["bias"], np.float32))
    say("conv kat", name, prec)
    y = host(ops().conv2d_forward(dev(x), dev(w), b, k["stride"], k["padding"], precision=prec))
    assert np.array_equal(y.ravel(), np.array(k["y"], np.float32))


def _conv_gate(x, w, b, stride, padding, y):
    d64 = oracle.conv2d_direct64(x, w, b, stride, padding)
    ref = oracle.conv2d_ref_im2col(x, w, b, stride, padding)
    return oracle.rel_fro(y, d64), oracle.rel_fro(ref, d64)


@pytest.mark.parametrize("g", GEOMS[1:6])
def test_conv_forward_parity(g):
    Bn, C, H, W, KH, KW, SH, SW, PH, PW = g
    OC = 7
    rng = np.random.default_rng(100 + sum(g))
    x = normal(rng, (Bn, C, H, W))
    w = normal(rng, (OC, C, KH, KW), std=np.sqrt(2.0 / (C * KH * KW)))
    b = normal(rng, (OC,), 0.1)
    say("conv fwd", g)
    y = host(ops().conv2d_forward(dev(x), dev(w), dev(b), (SH, SW), (PH, PW)))
    e, e_ref = _conv_gate(x, w, b, (SH, SW), (PH, PW), y)
    assert e <= 2 * e_ref + 2.0 ** -24, (e, e_ref)


@pytest.mark.parametrize("prec", [0, 1])
def test_conv_c5_full_batch_sampled(prec):
    """C5: N=32, C=64, 56x56 -> 64, 3x3, s1, p1, He-normal weights, seeded
    bias.  GPU runs the full batch; the oracle checks batch items 0 and 31
    (conv outputs are independent per batch item)."""
    rng = np.random.default_rng(5050)
    x = normal(rng, (32, 64, 56, 56))
    w = normal(rng, (64, 64, 3, 3), std=np.sqrt(2.0 / 576))
    b = normal(rng, (64,), 0.1)
    say("conv C5 full batch prec", prec)
    y = host(ops().conv2d_forward(dev(x), dev(w), dev(b), (1, 1), (1, 1), precision=prec))
    assert y.shape == (32, 64, 56, 56) and np.isfinite(y).all()
    for i in (0, 31):
        xi = x[i:i + 1]
        d64 = oracle.conv2d_direct64(xi, w, b, (1, 1), (1, 1))
        e = oracle.rel_fro(y[i:i + 1], d64)
        if prec == 0:
            e_ref = oracle.rel_fro(oracle.conv2d_ref_im2col(xi, w, b, (1, 1), (1, 1)), d64)
            print(f"C5 item {i}: fp32 gpu={e:.3e} seqfma-route={e_ref:.3e}")
            assert e <= 2 * e_ref
        else:
            col = oracle.im2col(xi, 3, 3, 1, 1, 1, 1)
            errs = []
            for mode in ("rz", "rne"):
                flat = oracle.gemm_tf32emu(w.reshape(64, -1), col, mode)
                yr = oracle.transpose_bias(flat, 64, 1, 3136, b).reshape(1, 64, 56, 56)
                errs.append(oracle.rel_fro(yr, d64))
            print(f"C5 item {i}: tf32mode gpu={e:.3e} tf32 route rz/rne={errs}")
            assert e <= min(errs)


@pytest.mark.parametrize("prec", [0, 1])
def test_conv_c5_rounds_same_bits_as_single_images(prec):
    """The im2col route runs C5's 32 images in rounds (18 + 14: column
    buffers within 128 MiB): images on either side of the round boundary
    come out bit for bit as when each image is convolved alone (one round,
    one GEMM of 3136 columns), since every output column's k-sum is one
    image's in the same order."""
    rng = np.random.default_rng(5151)
    x = normal(rng, (32, 64, 56, 56))
    w = normal(rng, (64, 64, 3, 3), std=np.sqrt(2.0 / 576))
    b = normal(rng, (64,), 0.1)
    say("conv C5 rounds vs single images prec", prec)
    gx, gw, gb = dev(x), dev(w), dev(b)
    y = host(ops().conv2d_forward(gx, gw, gb, (1, 1), (1, 1), precision=prec))
    for i in (0, 17, 18, 31):
        yi = host(ops().conv2d_forward(gx[i:i + 1].contiguous(), gw, gb, (1, 1), (1, 1),
                                       precision=prec))
        assert np.array_equal(yi[0].view(np.uint32), y[i].view(np.uint32)), i


IMPLICIT_GEOMS = [  # (B, C, H, W, OC, KH, KW, SH, SW, PH, PW)
    (2, 3, 20, 21, 32, 7, 7, 1, 1, 3, 3),      # 7x7 stem-like, Kc = 147 (% 4 != 0)
    (2, 5, 11, 13, 70, 5, 5, 2, 2, 2, 2),      # OC > one 64-channel tile
    (1, 16, 9, 9, 8, 1, 1, 1, 1, 0, 0),        # 1x1
    (3, 4, 10, 7, 9, 3, 5, 2, 1, 2, 0),        # rectangular kernel, mixed strides
    (1, 2, 3, 3, 5, 3, 3, 1, 1, 0, 0),         # single output pixel
    (2, 8, 6, 130, 16, 3, 3, 1, 2, 1, 1),      # pixels not a multiple of the 128 tile
    (1, 37, 12, 12, 65, 2, 2, 2, 2, 0, 0),     # Kc = 148: k-tail, OC = 65
    (2, 16, 14, 14, 64, 3, 3, 1, 1, 1, 1),     # 3x3 stride 1 through the implicit kernel
    # row-window form: 5 chunks of 8 channels, a 7 x 104 window (3 of 4
    # positions per thread used), 200 taps per chunk padded to 208
    (2, 40, 12, 100, 24, 5, 5, 1, 1, 2, 2),
    # enough workgroups that the plan takes 128- and 112-pixel tiles (the
    # small layers above take 80)
    (48, 8, 20, 32, 16, 3, 3, 1, 1, 1, 1),
    (42, 8, 20, 32, 16, 3, 3, 1, 1, 1, 1),
]


def _implicit_gate(x, w, b, stride, padding, y, batches=None):
    xs = x if batches is None else x[list(batches)]
    d64 = oracle.conv2d_direct64(xs, w, b, stride, padding)
    ref = oracle.conv2d_ref_implicit(xs, w, b, stride, padding)
    return oracle.rel_fro(y, d64), oracle.rel_fro(ref, d64)


@pytest.mark.parametrize("g", IMPLICIT_GEOMS)
def test_conv_implicit_parity(g):
    """Implicit-GEMM forward (cdx_conv2d_forward_implicit_f32): relFro vs
    fp64 <= 2 x that of the reference's implicit kernel restated on the CPU
    (bias-first FMA chain, conv_kernel.cu:172-215)."""
    Bn, C, H, W, OC, KH, KW, SH, SW, PH, PW = g
    rng = np.random.default_rng(700 + sum(g))
    x = normal(rng, (Bn, C, H, W))
    w = normal(rng, (OC, C, KH, KW), std=np.sqrt(2.0 / (C * KH * KW)))
    b = normal(rng, (OC,), 0.1)
    say("conv implicit", g)
    y = host(ops().conv2d_implicit(dev(x), dev(w), dev(b), (SH, SW), (PH, PW)))
    e, e_ref = _implicit_gate(x, w, b, (SH, SW), (PH, PW), y)
    assert e <= 2 * e_ref + 2.0 ** -24, (e, e_ref)
    y0 = host(ops().conv2d_implicit(dev(x), dev(w), None, (SH, SW), (PH, PW)))
    e0, e0_ref = _implicit_gate(x, w, None, (SH, SW), (PH, PW), y0)
    assert e0 <= 2 * e0_ref + 2.0 ** -24, (e0, e0_ref)


@pytest.mark.parametrize("g", [
    (1, 17, 9, 40, 10, 3, 3, 1, 1, 1, 1),     # OW 40: 8 and 5 divide it; 17 channels: masked chunk
    (3, 64, 13, 56, 64, 3, 3, 1, 1, 1, 1),    # OW 56 (C5's width): 8 and 7; tiles run past S
    (2, 3, 11, 35, 100, 3, 3, 1, 1, 1, 1),    # OW 35: 7 and 5; 3 channels, 100 output channels
    (2, 24, 7, 70, 33, 5, 5, 1, 1, 2, 2),     # 5x5, OW 70: 7 and 5; 2 + 4 halo rows
    (1, 40, 6, 120, 64, 3, 3, 1, 1, 1, 1),    # OW 120: 8 and 5; wider window, more positions per thread
    (2, 8, 10, 56, 16, 3, 3, 1, 1, 0, 1),     # no vertical padding
])
def test_rowwin_consecutive_pixel_lanes(g):
    """Stride-1 layers whose output width the row-window kernel's pixel-block
    count divides: each lane then takes consecutive pixels of one output row
    and reads them at immediate offsets, with the output tile staged through
    LDS.  The implicit forward (one-level k sum) and the stride-1 backward
    data through the same kernel (two-level sum, the flipped filter) both
    pass the gates of the other geometries: <= 2 x the reference routes'
    errors against fp64."""
    Bn, C, H, W, OC, KH, KW, SH, SW, PH, PW = g
    rng = np.random.default_rng(900 + sum(g))
    x = normal(rng, (Bn, C, H, W))
    w = normal(rng, (OC, C, KH, KW), std=np.sqrt(2.0 / (C * KH * KW)))
    b = normal(rng, (OC,), 0.1)
    st, pd = (SH, SW), (PH, PW)
    say("conv rowwin consecutive lanes", g)
    y = host(ops().conv2d_implicit(dev(x), dev(w), dev(b), st, pd))
    e, e_ref = _implicit_gate(x, w, b, st, pd, y)
    assert e <= 2 * e_ref + 2.0 ** -24, (e, e_ref)
    OH = oracle.conv_out_size(H, KH, SH, PH)
    OW = oracle.conv_out_size(W, KW, SW, PW)
    dy = normal(rng, (Bn, OC, OH, OW))
    dx = host(ops().conv2d_backward_data(dev(dy), dev(w), x.shape, st, pd))
    dx64 = oracle.conv2d_backward_data64(dy, w, x.shape, st, pd)
    ex_ref = oracle.rel_fro(oracle.conv2d_backward_data_ref(dy, w, x.shape, st, pd), dx64)
    assert oracle.rel_fro(dx, dx64) <= 2 * ex_ref + 2.0 ** -24


@pytest.mark.parametrize("name", ["conv_identity_1x1", "conv_3x3_ones", "conv_3x3_bias",
                                  "conv_3x3_pad1"])
def test_conv_implicit_kats(kats, name):
    k = kats[name]
    x = np.array(k["x"], np.float32).reshape(k["x_shape"])
    w = np.array(k["w"], np.float32).reshape(k["w_shape"])
    b = None if k["bias"] is None else dev(np.array(k["bias"], np.float32))
    say("conv implicit kat", name)
    y = host(ops().conv2d_implicit(dev(x), dev(w), b, k["stride"], k["padding"]))
    assert np.array_equal(y.ravel(), np.array(k["y"], np.float32))


@pytest.mark.parametrize("prec", [0, 1])
def test_conv_forward_large_7x7_takes_implicit_route(prec):
    """A 7x7 layer at C5's size (32 x 64 x 56^2 -> 64, pad 3) would need a
    1.26 GB column buffer: cdx_conv2d_forward_f32 routes it to the implicit
    GEMM like the reference (conv_kernel.cu:263-275): workspace query 0, and
    images 0 and 31 pass the implicit route's parity gate."""
    rng = np.random.default_rng(7077)
    x = normal(rng, (32, 64, 56, 56))
    w = normal(rng, (64, 64, 7, 7), std=np.sqrt(2.0 / (64 * 49)))
    b = normal(rng, (64,), 0.1)
    assert ops().conv2d_workspace_bytes(x.shape, w.shape, (1, 1), (3, 3)) == 0
    # a 3x3 stride-1 layer of the same size keeps the im2col route (rounds of
    # at most 18 images)
    assert ops().conv2d_workspace_bytes(x.shape, (64, 64, 3, 3), (1, 1), (1, 1)) == 576 * 56448 * 4
    say("conv 7x7 C5-size prec", prec)
    y = host(ops().conv2d_forward(dev(x), dev(w), dev(b), (1, 1), (3, 3), precision=prec))
    assert y.shape == (32, 64, 56, 56) and np.isfinite(y).all()
    e, e_ref = _implicit_gate(x, w, b, (1, 1), (3, 3), y[[0, 31]], batches=(0, 31))
    print(f"7x7 C5-size items 0, 31: gpu={e:.3e} reference implicit route={e_ref:.3e}")
    assert e <= 2 * e_ref


def test_conv_implicit_c5_3x3_split_last_round():
    """C5's 3x3 layer through the row-window implicit kernel: 896 tiles on
    256 CUs run as 768 whole tiles plus the last 128 as 256 half tiles (32
    output channels each, the four k-steps of every 16-k group split over
    two waves and added in the epilogue).  Image 0 (whole tiles) and images
    28 and 31 (half tiles) pass the implicit route's parity gate."""
    rng = np.random.default_rng(7078)
    x = normal(rng, (32, 64, 56, 56))
    w = normal(rng, (64, 64, 3, 3), std=np.sqrt(2.0 / 576))
    b = normal(rng, (64,), 0.1)
    say("conv implicit C5 3x3")
    y = host(ops().conv2d_implicit(dev(x), dev(w), dev(b), (1, 1), (1, 1)))
    assert y.shape == (32, 64, 56, 56) and np.isfinite(y).all()
    e, e_ref = _implicit_gate(x, w, b, (1, 1), (1, 1), y[[0, 28, 31]], batches=(0, 28, 31))
    print(f"C5 3x3 implicit items 0, 28, 31: gpu={e:.3e} reference implicit route={e_ref:.3e}")
    assert e <= 2 * e_ref


def test_conv_workspace_and_no_bias():
    import torch
    rng = np.random.default_rng(77)
    x = normal(rng, (2, 3, 9, 9))
    w = normal(rng, (5, 3, 3, 3))
    nbytes = ops().conv2d_workspace_bytes(x.shape, w.shape, (1, 1), (1, 1))
    assert nbytes == 27 * 2 * 81 * 4
    ws = torch.empty(nbytes // 4, device="cuda")
    say("conv with workspace")
    y1 = host(ops().conv2d_forward(dev(x), dev(w), None, (1, 1), (1, 1), workspace=ws))
    y2 = host(ops().conv2d_forward(dev(x), dev(w), None, (1, 1), (1, 1)))
    assert np.array_equal(y1, y2)
    e, e_ref = _conv_gate(x, w, None, (1, 1), (1, 1), y1)
    assert e <= 2 * e_ref + 2.0 ** -24


@pytest.mark.parametrize("g", [(32, 64, 56, 56, 64, 3, 3, 1, 1, 1, 1),    # C5: rows kernel
                               (2, 5, 13, 11, 7, 3, 2, 2, 1, 1, 0)])       # gather kernel
def test_backward_weight_workspace_query_is_what_the_launch_takes(g):
    """cdx_conv2d_backward_weight_workspace_size is the scratch of the route
    the launch takes: a workspace of exactly that size is accepted, one
    byte less is refused, and the result equals the self-allocating call's."""
    import torch
    import cudeep_amd._lib as L
    Bn, C, H, W, OC, KH, KW, SH, SW, PH, PW = g
    rng = np.random.default_rng(sum(g))
    x = normal(rng, (Bn, C, H, W))
    OH, OW = oracle.conv_out_size(H, KH, SH, PH), oracle.conv_out_size(W, KW, SW, PW)
    dy = normal(rng, (Bn, OC, OH, OW))
    nbytes = ops().conv2d_backward_weight_workspace_bytes(x.shape, (OC, C, KH, KW), (SH, SW),
                                                          (PH, PW))
    say("wgrad workspace", g, nbytes)
    dx, ddy = dev(x), dev(dy)
    ref = host(ops().conv2d_backward_weight(ddy, dx, (OC, C, KH, KW), (SH, SW), (PH, PW)))
    if nbytes > 0:
        small = torch.empty(nbytes - 1, dtype=torch.uint8, device="cuda")
        with pytest.raises(L.CdxError) as err:
            ops().conv2d_backward_weight(ddy, dx, (OC, C, KH, KW), (SH, SW), (PH, PW),
                                         workspace=small)
        assert err.value.code == L.CDX_ERR_WORKSPACE
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device="cuda")
    got = host(ops().conv2d_backward_weight(ddy, dx, (OC, C, KH, KW), (SH, SW), (PH, PW),
                                            workspace=ws))
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


# ---------------------------------------------------------------------------
# backward: col2im (bit-exact), data / weight / bias gradients
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("g", GEOMS[:8])
def test_col2im_bit_exact(g):
    Bn, C, H, W, KH, KW, SH, SW, PH, PW = g
    rng = np.random.default_rng(7 + sum(g))
    OH = oracle.conv_out_size(H, KH, SH, PH)
    OW = oracle.conv_out_size(W, KW, SW, PW)
    col = normal(rng, (C * KH * KW, Bn * OH * OW))
    say("col2im", g)
    got = host(ops().col2im(dev(col), (Bn, C, H, W), KH, KW, (SH, SW), (PH, PW)))
    want = oracle.col2im(col, (Bn, C, H, W), KH, KW, SH, SW, PH, PW)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_conv_backward_kats(kats):
    k = kats["conv_bwd_data_1x1_w2"]
    say("conv bwd kats")
    dx = host(ops().conv2d_backward_data(
        dev(np.array(k["dy"], np.float32).reshape(k["dy_shape"])),
        dev(np.array(k["w"], np.float32).reshape(k["w_shape"])), k["x_shape"],
        k["stride"], k["padding"]))
    assert np.array_equal(dx.ravel(), np.array(k["dx"], np.float32))
    k = kats["conv_bwd_weight_ones"]
    dw = host(ops().conv2d_backward_weight(
        dev(np.array(k["dy"], np.float32).reshape(k["dy_shape"])),
        dev(np.array(k["x"], np.float32).reshape(k["x_shape"])), k["w_shape"],
        k["stride"], k["padding"]))
    assert np.array_equal(dw.ravel(), np.array(k["dw"], np.float32))


BWD_GEOMS = [  # (B, C, H, W, OC, KH, KW, SH, SW, PH, PW)
    (2, 3, 8, 9, 4, 3, 3, 1, 1, 1, 1),
    (1, 2, 7, 7, 3, 3, 5, 2, 1, 2, 0),
    (3, 4, 6, 5, 5, 2, 2, 1, 1, 1, 0),
    (4, 16, 28, 28, 32, 3, 3, 1, 1, 1, 1),
    (2, 8, 15, 17, 6, 1, 1, 2, 2, 0, 0),
    # stride 1: flipped-filter forward route, incl. padding = kernel - 1,
    # 1x1, and padding above kernel - 1 (falls back to GEMM + col2im)
    (2, 5, 9, 4, 3, 5, 3, 1, 1, 4, 1),
    (1, 8, 15, 17, 6, 1, 1, 1, 1, 0, 0),
    (2, 3, 6, 7, 4, 3, 3, 1, 1, 3, 0),
    (2, 33, 10, 30, 65, 3, 3, 1, 1, 0, 2),
    # 3x3 stride 1 row-window weight gradient: rows wider than 64 pixels (two
    # segments), 61-pixel rows, pad 2 with partial channel tiles
    (1, 4, 5, 70, 8, 3, 3, 1, 1, 1, 1),
    (2, 16, 9, 61, 16, 3, 3, 1, 1, 1, 1),
    (1, 20, 6, 33, 70, 3, 3, 1, 1, 2, 2),
    # backward data through 128- and 112-pixel row-window tiles
    (48, 8, 20, 32, 16, 3, 3, 1, 1, 1, 1),
    (42, 8, 20, 32, 16, 3, 3, 1, 1, 1, 1),
]


@pytest.mark.parametrize("g", BWD_GEOMS)
@pytest.mark.parametrize("prec", [0, 1])
def test_conv_backward_parity(g, prec):
    Bn, C, H, W, OC, KH, KW, SH, SW, PH, PW = g
    rng = np.random.default_rng(200 + sum(g))
    x = normal(rng, (Bn, C, H, W))
    w = normal(rng, (OC, C, KH, KW), std=np.sqrt(2.0 / (C * KH * KW)))
    OH = oracle.conv_out_size(H, KH, SH, PH)
    OW = oracle.conv_out_size(W, KW, SW, PW)
    dy = normal(rng, (Bn, OC, OH, OW))
    st, pd = (SH, SW), (PH, PW)
    say("conv bwd", g, "prec", prec)
    dx = host(ops().conv2d_backward_data(dev(dy), dev(w), x.shape, st, pd, precision=prec))
    dw = host(ops().conv2d_backward_weight(dev(dy), dev(x), w.shape, st, pd, precision=prec))
    db = host(ops().conv2d_backward_bias(dev(dy)))
    dx64 = oracle.conv2d_backward_data64(dy, w, x.shape, st, pd)
    dw64 = oracle.conv2d_backward_weight64(dy, x, w.shape, st, pd)
    if prec == 0:
        ex_ref = oracle.rel_fro(oracle.conv2d_backward_data_ref(dy, w, x.shape, st, pd), dx64)
        ew_ref = oracle.rel_fro(oracle.conv2d_backward_weight_ref(dy, x, w.shape, st, pd), dw64)
        floor = 2.0 ** -24
        assert oracle.rel_fro(dx, dx64) <= 2 * ex_ref + floor
        assert oracle.rel_fro(dw, dw64) <= 2 * ew_ref + floor
    else:
        ex_ref = min(oracle.rel_fro(oracle.conv2d_backward_data_ref(dy, w, x.shape, st, pd, m), dx64)
                     for m in ("rz", "rne"))
        ew_ref = min(oracle.rel_fro(oracle.conv2d_backward_weight_ref(dy, x, w.shape, st, pd, m), dw64)
                     for m in ("rz", "rne"))
        assert oracle.rel_fro(dx, dx64) <= ex_ref
        assert oracle.rel_fro(dw, dw64) <= ew_ref
    db64 = dy.astype(np.float64).sum(axis=(0, 2, 3))
    # reference: NumPy float32 sum over (0, 2, 3) (tensor.py:718-721)
    e_ref = oracle.rel_fro(dy.sum(axis=(0, 2, 3)).astype(np.float32), db64)
    assert oracle.rel_fro(db, db64) <= 2 * e_ref + 2.0 ** -24


@pytest.mark.parametrize("g,ws_expect", [
    ((128, 64, 32, 32, 64, 3, 3, 1, 1, 1, 1), 256 * 64 * 576 * 4),
    ((64, 128, 20, 20, 70, 3, 3, 1, 1, 1, 1), 64 * 70 * 1152 * 4)])
def test_conv_backward_weight_64_channel_tile(g, ws_expect):
    """3x3 stride-1 layers with a multiple of 64 input channels and long
    K slices take the row-window kernel's 64-channel tile (the workspace
    size pins the route: 256 / 64 slices of the whole OC x 9 IC partial):
    dW against the fp64 oracle at 2x the reference route's error, in both
    precision modes' gates (ragged OC in the second layer)."""
    Bn, C, H, W, OC, KH, KW, SH, SW, PH, PW = g
    rng = np.random.default_rng(sum(g))
    x = normal(rng, (Bn, C, H, W))
    OH, OW = oracle.conv_out_size(H, KH, SH, PH), oracle.conv_out_size(W, KW, SW, PW)
    dy = normal(rng, (Bn, OC, OH, OW))
    w_shape = (OC, C, KH, KW)
    assert ops().conv2d_backward_weight_workspace_bytes(x.shape, w_shape, (SH, SW),
                                                        (PH, PW)) == ws_expect
    say("wgrad 64-channel tile", g)
    dw = host(ops().conv2d_backward_weight(dev(dy), dev(x), w_shape, (SH, SW), (PH, PW)))
    dw64 = oracle.conv2d_backward_weight64(dy, x, w_shape, (SH, SW), (PH, PW))
    ew_ref = oracle.rel_fro(oracle.conv2d_backward_weight_ref(dy, x, w_shape, (SH, SW), (PH, PW)),
                            dw64)
    assert oracle.rel_fro(dw, dw64) <= 2 * ew_ref


def test_conv_backward_c5_full():
    """C5 backward at full size: N=32, C=64, 56x56, OC=64, 3x3, s1, p1.
    dW checked against the fp64 oracle in full (it reduces over the whole
    batch); dX on batch items 0 and 31."""
    rng = np.random.default_rng(5151)
    x = normal(rng, (32, 64, 56, 56))
    w = normal(rng, (64, 64, 3, 3), std=np.sqrt(2.0 / 576))
    dy = normal(rng, (32, 64, 56, 56))
    say("conv bwd C5 full")
    dx = host(ops().conv2d_backward_data(dev(dy), dev(w), x.shape, (1, 1), (1, 1)))
    dw = host(ops().conv2d_backward_weight(dev(dy), dev(x), w.shape, (1, 1), (1, 1)))
    dw64 = oracle.conv2d_backward_weight64(dy, x, w.shape, (1, 1), (1, 1))
    ew_ref = oracle.rel_fro(oracle.conv2d_backward_weight_ref(dy, x, w.shape, (1, 1), (1, 1)), dw64)
    ew = oracle.rel_fro(dw, dw64)
    print(f"C5 dW relFro gpu={ew:.3e} ref-route={ew_ref:.3e}")
    assert ew <= 2 * ew_ref
    for i in (0, 31):
        d64 = oracle.conv2d_backward_data64(dy[i:i + 1], w, (1, 64, 56, 56), (1, 1), (1, 1))
        e_ref = oracle.rel_fro(oracle.conv2d_backward_data_ref(dy[i:i + 1], w, (1, 64, 56, 56),
                                                               (1, 1), (1, 1)), d64)
        assert oracle.rel_fro(dx[i:i + 1], d64) <= 2 * e_ref


# ---------------------------------------------------------------------------
# float64 conv (the reference's double instantiations)
# ---------------------------------------------------------------------------

def _conv64_calls(x, w, b, dy, stride, padding):
    """The four fp64 C-ABI entry points on device copies of the operands."""
    import torch
    from cudeep_amd import _lib as L
    Bn, C, H, W = x.shape
    OC, _, KH, KW = w.shape
    SH, SW = stride
    PH, PW = padding
    X, Wt, Y = dev(x), dev(w), dev(dy)
    Bt = dev(b) if b is not None else None
    geo = (Bn, C, OC, H, W, KH, KW, SH, SW, PH, PW)
    out = torch.empty(dy.shape, dtype=torch.float64, device="cuda")
    dx = torch.empty(x.shape, dtype=torch.float64, device="cuda")
    dw = torch.empty(w.shape, dtype=torch.float64, device="cuda")
    db = torch.empty((OC,), dtype=torch.float64, device="cuda")
    s = torch.cuda.current_stream().cuda_stream
    L.call("cdx_conv2d_forward_f64", X.data_ptr(), Wt.data_ptr(),
           Bt.data_ptr() if Bt is not None else None, out.data_ptr(), *geo, s)
    L.call("cdx_conv2d_backward_data_f64", Y.data_ptr(), Wt.data_ptr(), dx.data_ptr(), *geo, s)
    L.call("cdx_conv2d_backward_weight_f64", Y.data_ptr(), X.data_ptr(), dw.data_ptr(), *geo, s)
    L.call("cdx_conv2d_backward_bias_f64", Y.data_ptr(), db.data_ptr(), Bn, OC,
           dy.shape[2] * dy.shape[3], s)
    return host(out), host(dx), host(dw), host(db)


F64_GEOMS = [  # (B, C, H, W, OC, KH, KW, SH, SW, PH, PW)
    (2, 3, 8, 9, 4, 3, 3, 1, 1, 1, 1),
    (1, 2, 7, 7, 3, 3, 5, 2, 1, 2, 0),
    (3, 4, 6, 5, 5, 2, 2, 1, 1, 1, 0),
    (2, 8, 15, 17, 6, 1, 1, 2, 2, 0, 0),
    (2, 16, 28, 28, 32, 3, 3, 1, 1, 1, 1),
]


@pytest.mark.parametrize("g", F64_GEOMS)
def test_conv_f64_parity(g):
    """fp64 forward / backward data / backward weight / bias gradient against the
    fp64 oracles.  Operands are fp32 values held in fp64 (the oracles read fp32),
    so every product is exact and only the summation order differs."""
    Bn, C, H, W, OC, KH, KW, SH, SW, PH, PW = g
    rng = np.random.default_rng(640 + sum(g))
    x = normal(rng, (Bn, C, H, W)).astype(np.float64)
    w = normal(rng, (OC, C, KH, KW), std=np.sqrt(2.0 / (C * KH * KW))).astype(np.float64)
    b = normal(rng, (OC,), std=0.1).astype(np.float64)
    OH = oracle.conv_out_size(H, KH, SH, PH)
    OW = oracle.conv_out_size(W, KW, SW, PW)
    dy = normal(rng, (Bn, OC, OH, OW)).astype(np.float64)
    st, pd = (SH, SW), (PH, PW)
    say("conv f64", g)
    out, dx, dw, db = _conv64_calls(x, w, b, dy, st, pd)
    assert out.dtype == np.float64
    assert oracle.rel_fro(out, oracle.conv2d_direct64(x, w, b, st, pd)) < 1e-14
    assert oracle.rel_fro(dx, oracle.conv2d_backward_data64(dy, w, x.shape, st, pd)) < 1e-14
    assert oracle.rel_fro(dw, oracle.conv2d_backward_weight64(dy, x, w.shape, st, pd)) < 1e-14
    assert oracle.rel_fro(db, dy.sum(axis=(0, 2, 3))) < 1e-14


def _conv_fwd_numpy64(x, w, b, stride, padding):
    """Independent fp64 cross-correlation: zero-pad, then one tensor contraction
    per filter tap."""
    SH, SW = stride
    PH, PW = padding
    Bn, C, H, W = x.shape
    OC, _, KH, KW = w.shape
    OH, OW = (H + 2 * PH - KH) // SH + 1, (W + 2 * PW - KW) // SW + 1
    xp = np.zeros((Bn, C, H + 2 * PH, W + 2 * PW))
    xp[:, :, PH:PH + H, PW:PW + W] = x
    out = np.zeros((Bn, OC, OH, OW))
    for kh in range(KH):
        for kw in range(KW):
            win = xp[:, :, kh:kh + SH * (OH - 1) + 1:SH, kw:kw + SW * (OW - 1) + 1:SW]
            out += np.einsum("oc,bchw->bohw", w[:, :, kh, kw], win)
    return out + b[None, :, None, None]


def test_conv_f64_full_precision_operands():
    """Full 53-bit operands (not fp32 values): forward against an independent
    NumPy fp64 contraction, backward through the adjoint identity
    <conv(x), dy> = <x, dX(dy)> = <w, dW(dy, x)>, all in fp64."""
    rng = np.random.default_rng(6464)
    x = rng.standard_normal((2, 5, 11, 13))
    w = rng.standard_normal((7, 5, 3, 3)) / 6.0
    b = rng.standard_normal(7)
    st, pd = (2, 1), (1, 2)
    ref = _conv_fwd_numpy64(x, w, b, st, pd)
    dy = rng.standard_normal(ref.shape)
    say("conv f64 full precision")
    out, dx, dw, db = _conv64_calls(x, w, b, dy, st, pd)
    assert oracle.rel_fro(out, ref) < 1e-14
    lin = float(np.sum((ref - b[None, :, None, None]) * dy))   # <conv without bias, dy>
    assert abs(float(np.sum(x * dx)) - lin) <= 1e-12 * abs(lin)
    assert abs(float(np.sum(w * dw)) - lin) <= 1e-12 * abs(lin)
    assert np.allclose(db, dy.sum(axis=(0, 2, 3)), rtol=1e-14, atol=0)


@pytest.mark.parametrize("prec", [0, 1])
def test_conv_three_rounds_same_bits_as_single_images(prec):
    """A batch of 40 C5-size images runs the im2col route in three rounds of
    15 + 15 + 10 images through one 15-image column buffer (the round size
    with the fewest waves of GEMM tiles): images at both round boundaries and
    at the ends come out bit for bit as when convolved alone."""
    rng = np.random.default_rng(5252)
    x = normal(rng, (40, 64, 56, 56))
    w = normal(rng, (64, 64, 3, 3), std=np.sqrt(2.0 / 576))
    b = normal(rng, (64,), 0.1)
    say("conv 40 images three rounds prec", prec)
    assert ops().conv2d_workspace_bytes(x.shape, w.shape, (1, 1), (1, 1)) == 15 * 576 * 3136 * 4
    gx, gw, gb = dev(x), dev(w), dev(b)
    y = host(ops().conv2d_forward(gx, gw, gb, (1, 1), (1, 1), precision=prec))
    for i in (0, 14, 15, 29, 30, 39):
        yi = host(ops().conv2d_forward(gx[i:i + 1].contiguous(), gw, gb, (1, 1), (1, 1),
                                       precision=prec))
        assert np.array_equal(yi[0].view(np.uint32), y[i].view(np.uint32)), i


@pytest.mark.parametrize("H,W", [(22, 1024), (20, 1024)])
def test_conv_backward_data_wide_rows_gemm_route(H, W):
    """Stride-1 backward data of 1024-pixel-wide rows takes the im2col + GEMM
    route of the transposed convolution (its row window does not fit in
    LDS) with a two-level k sum: 64 output channels x 352 / 320 column tiles,
    whose last round over the 256 CUs (96 / 64 tiles) runs as half / quarter
    tiles.  FP32 against the reference's route (GEMM + col2im) to 2x its
    error vs fp64."""
    rng = np.random.default_rng(H * 1000 + W)
    C = OC = 64
    w = normal(rng, (OC, C, 3, 3), std=np.sqrt(2.0 / (C * 9)))
    dy = normal(rng, (1, OC, H, W))
    xs = (1, C, H, W)
    assert ops().conv2d_backward_data_workspace_bytes(xs, w.shape, (1, 1), (1, 1)) > w.size * 4
    say("conv bwd data wide rows", H, W)
    dx = host(ops().conv2d_backward_data(dev(dy), dev(w), xs, (1, 1), (1, 1), precision=0))
    dx64 = oracle.conv2d_backward_data64(dy, w, xs, (1, 1), (1, 1))
    e_ref = oracle.rel_fro(oracle.conv2d_backward_data_ref(dy, w, xs, (1, 1), (1, 1)), dx64)
    e = oracle.rel_fro(dx, dx64)
    print(f"bwd data {H}x{W}: gpu={e:.3e} reference route={e_ref:.3e}")
    assert e <= 2 * e_ref + 2.0 ** -24
