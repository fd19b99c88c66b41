"""The allocation-free backward-weight entry point
(cdx_conv2d_backward_weight_f32_noalloc) against the allocating one
(cdx_conv2d_backward_weight_f32, workspace NULL): the same kernels on the
same inputs, so the results must agree bit for bit -- on calls in a row
whose scratch use shrinks (stale partials of the previous call must not
leak into the next), on both backward-weight kernels, in every precision
mode.  Layers whose scratch exceeds the fixed per-GPU array are refused
before any launch."""

import numpy as np
import pytest

from tests.gpu_util import dev, host, normal, require_gpu, say

NOALLOC_BYTES = 40 << 20


def _lib():
    from cudeep_amd import _lib as L
    return L


def _geom_out(g):
    Bn, C, H, W, OC, KH, KW, SH, SW, PH, PW = g
    return (H + 2 * PH - KH) // SH + 1, (W + 2 * PW - KW) // SW + 1


def _args(g):
    Bn, C, H, W, OC, KH, KW, SH, SW, PH, PW = g
    return (Bn, C, OC, H, W, KH, KW, SH, SW, PH, PW)


def test_implicit_route_layers_fit_the_scratch():
    """The implicit kernels split K over about 256 workgroups, so their
    partials stay near 9-10 MiB (36 MiB on the 64-channel row-window
    kernel) whatever the layer: all of these fit."""
    L = _lib()
    for g in [(32, 64, 56, 56, 64, 3, 3, 1, 1, 1, 1), (32, 512, 14, 14, 512, 3, 3, 1, 1, 1, 1),
              (64, 128, 56, 56, 128, 3, 3, 1, 1, 1, 1), (32, 512, 14, 14, 512, 1, 1, 1, 1, 0, 0),
              (8, 256, 28, 28, 512, 3, 3, 2, 2, 1, 1), (16, 3, 224, 224, 64, 7, 7, 2, 2, 3, 3)]:
        assert L.lib().cdx_conv2d_backward_weight_workspace_size(*_args(g)) <= NOALLOC_BYTES, g


def test_refuses_layers_beyond_the_scratch_before_any_launch():
    """A layer beyond the implicit kernels' 32-bit index range (a 2^15 x 2^15
    plane) takes the column-buffer route, whose 4 GiB of scratch the array
    cannot hold: refused with CDX_ERR_UNSUPPORTED and a message naming the
    limit (no device call happens, so this runs without a GPU too)."""
    L = _lib()
    big = (1, 1, 2 ** 15, 2 ** 15, 1, 1, 1, 1, 1, 0, 0)
    need = L.lib().cdx_conv2d_backward_weight_workspace_size(*_args(big))
    assert need > NOALLOC_BYTES
    # NULL tensors: the refusal comes before any pointer is used; were it to
    # regress, the general entry point's NULL check would stop the call
    # before any kernel launch.
    st = L.lib().cdx_conv2d_backward_weight_f32_noalloc(None, None, None, *_args(big), 0, None)
    assert st == L.CDX_ERR_UNSUPPORTED
    msg = L.lib().cdx_last_error().decode()
    assert str(need) in msg and str(NOALLOC_BYTES) in msg


CALLS = [  # (B, C, H, W, OC, KH, KW, SH, SW, PH, PW), in this order
    (128, 64, 32, 32, 64, 3, 3, 1, 1, 1, 1),   # 64-channel row-window tile, 256 slices (36 MiB)
    (32, 64, 56, 56, 64, 3, 3, 1, 1, 1, 1),    # C5: row-window kernel, 64 partial slices
    (4, 32, 28, 28, 16, 3, 3, 1, 1, 1, 1),     # smaller: fewer, smaller slices
    (2, 5, 13, 11, 7, 3, 2, 2, 1, 1, 0),       # gather kernel, ragged
]


@pytest.mark.gpu
@pytest.mark.parametrize("prec", [0, 1])
def test_noalloc_equals_allocating_entry_point(prec):
    require_gpu()
    import torch
    L = _lib()
    stream = torch.cuda.current_stream().cuda_stream
    for i, g in enumerate(CALLS):
        Bn, C, H, W, OC, KH, KW, SH, SW, PH, PW = g
        OH, OW = _geom_out(g)
        rng = np.random.default_rng(100 * prec + i)
        x = dev(normal(rng, (Bn, C, H, W)))
        dy = dev(normal(rng, (Bn, OC, OH, OW)))
        need = L.lib().cdx_conv2d_backward_weight_workspace_size(*_args(g))
        assert need <= NOALLOC_BYTES           # 0 for the unsplit third call
        say("noalloc wgrad", i, g, "precision", prec, "scratch", need)
        ref = torch.empty((OC, C, KH, KW), device="cuda")
        got = torch.full((OC, C, KH, KW), float("nan"), device="cuda")
        L.call("cdx_conv2d_backward_weight_f32", dy.data_ptr(), x.data_ptr(), ref.data_ptr(),
               *_args(g), prec, None, 0, stream)
        L.call("cdx_conv2d_backward_weight_f32_noalloc", dy.data_ptr(), x.data_ptr(),
               got.data_ptr(), *_args(g), prec, stream)
        a, b = host(got), host(ref)
        assert np.isfinite(a).all()
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (i, g)
