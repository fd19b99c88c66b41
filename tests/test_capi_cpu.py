"""CPU-side checks of the C-ABI boundary (no GPU, no compute calls):
the library loads, exports every entry point include/cudeep_amd.h declares,
and rejects bad arguments with status codes before any HIP call."""
import ctypes
import os
import re

import pytest

from cudeep_amd import _lib as L

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "cudeep_amd.h")


def declared_symbols():
    txt = open(HEADER).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(cdx_[a-z0-9_]+)\s*\(", txt)))


def test_header_declares_expected_entry_points():
    syms = declared_symbols()
    for must in ("cdx_sgemm_f32", "cdx_gemm_tf32mode", "cdx_gemm_ex", "cdx_im2col_f32",
                 "cdx_conv2d_forward_f32", "cdx_sum_reduce_rows_f32", "cdx_dgemm"):
        assert must in syms


def test_library_exports_every_declared_symbol():
    lib = L.lib()
    missing = [s for s in declared_symbols() if not hasattr(lib, s)]
    assert not missing, missing
    # and the Python signature table covers exactly the header
    assert sorted(L.SIGNATURES) == declared_symbols()


def test_version_string():
    assert b"gfx950" in L.lib().cdx_version()


def _status(name, *args):
    return getattr(L.lib(), name)(*args)


def test_gemm_argument_validation():
    fake = ctypes.c_void_p(0x1000)   # never dereferenced: validation fails first
    assert _status("cdx_gemm_ex", 0, 7, 0, 4, 4, 4, fake, 4, fake, 4, fake, 4, None, 0, 0, None) \
        == L.CDX_ERR_INVALID_ARG
    assert b"opA" in L.lib().cdx_last_error()
    assert _status("cdx_gemm_ex", 0, 0, 0, -1, 4, 4, fake, 4, fake, 4, fake, 4, None, 0, 0, None) \
        == L.CDX_ERR_INVALID_ARG
    assert _status("cdx_gemm_ex", 0, 0, 0, 4, 4, 4, fake, 3, fake, 4, fake, 4, None, 0, 0, None) \
        == L.CDX_ERR_INVALID_ARG          # lda < K
    assert _status("cdx_gemm_ex", 0, 0, 0, 4, 4, 4, None, 4, fake, 4, fake, 4, None, 0, 0, None) \
        == L.CDX_ERR_INVALID_ARG          # NULL A
    for prec in (9, 3, -1):
        assert _status("cdx_gemm_ex", prec, 0, 0, 4, 4, 4, fake, 4, fake, 4, fake, 4, None, 0, 0,
                       None) == L.CDX_ERR_INVALID_ARG          # precision
    assert _status("cdx_gemm_ex", 0, 0, 0, 4, 4, 4, fake, 4, fake, 4, fake, 4, None, 2, 0, None) \
        == L.CDX_ERR_INVALID_ARG          # bias mode without bias
    assert _status("cdx_gemm_ex", 0, 0, 0, 4, 4, 4, fake, 4, fake, 4, fake, 4, None, 0, 5, None) \
        == L.CDX_ERR_INVALID_ARG          # epilogue
    assert _status("cdx_sgemm_f32", fake, fake, None, 4, 4, 4, None) == L.CDX_ERR_INVALID_ARG
    # empty problems are a successful no-op and touch nothing
    assert _status("cdx_sgemm_f32", None, None, None, 0, 4, 4, None) == L.CDX_OK
    assert _status("cdx_gemm_tf32mode", None, None, None, 4, 0, 4, None) == L.CDX_OK
    assert _status("cdx_dgemm", 0, 0, 0, 0, 0, None, 1, None, 1, None, 1, None) == L.CDX_OK


def test_conv_argument_validation():
    fake = ctypes.c_void_p(0x1000)
    # kernel larger than padded input
    assert _status("cdx_im2col_f32", fake, fake, 1, 1, 2, 2, 5, 5, 1, 1, 0, 0, None) \
        == L.CDX_ERR_INVALID_ARG
    # zero stride
    assert _status("cdx_conv2d_forward_f32", fake, fake, None, fake, 1, 1, 1, 4, 4, 3, 3,
                   0, 1, 0, 0, 0, None, 0, None) == L.CDX_ERR_INVALID_ARG
    # workspace too small
    assert _status("cdx_conv2d_forward_f32", fake, fake, None, fake, 1, 1, 1, 4, 4, 3, 3,
                   1, 1, 0, 0, 0, fake, 4, None) == L.CDX_ERR_WORKSPACE
    # workspace size query = K_col * OH * OW * 4 per image of a round: the whole
    # batch while its column buffer fits 128 MiB, else rounds of at most 18
    # C5 images (7.2 MB each), sized for whole waves of 64-column GEMM tiles:
    # C5 32 -> 18 + 14 (882 + 686 tiles, 4 + 3 waves of 256; 16 + 16 needs 8),
    # 33 -> 18 + 15 (17 + 16 needs 8 waves)
    assert L.lib().cdx_conv2d_forward_workspace_size(32, 64, 56, 56, 3, 3, 1, 1, 1, 1) \
        == 576 * 18 * 56 * 56 * 4
    assert L.lib().cdx_conv2d_forward_workspace_size(2, 3, 9, 9, 3, 3, 1, 1, 1, 1) \
        == 27 * 2 * 81 * 4
    assert L.lib().cdx_conv2d_forward_workspace_size(33, 64, 56, 56, 3, 3, 1, 1, 1, 1) \
        == 576 * 18 * 56 * 56 * 4
    # 40 images -> 15 + 15 + 10 (3 + 3 + 2 waves; 18 + 18 + 4 needs 4 + 4 + 1)
    assert L.lib().cdx_conv2d_forward_workspace_size(40, 64, 56, 56, 3, 3, 1, 1, 1, 1) \
        == 576 * 15 * 56 * 56 * 4
    # backward data, stride 1 (row-window implicit kernel): the flipped filter only
    assert L.lib().cdx_conv2d_backward_data_workspace_size(32, 64, 64, 56, 56, 3, 3, 1, 1, 1, 1) \
        == 64 * 64 * 9 * 4
    # stride 2: grad_col [K_col, B*S] + grad_out in [OC, B*S]
    assert L.lib().cdx_conv2d_backward_data_workspace_size(2, 3, 4, 9, 9, 3, 3, 2, 2, 1, 1) \
        == (27 * 2 * 25 + 4 * 2 * 25) * 4
    # padding above kernel - 1 keeps the col2im route
    assert L.lib().cdx_conv2d_backward_data_workspace_size(1, 3, 4, 5, 5, 3, 3, 1, 1, 3, 0) \
        == 27 * 9 * 3 * 4
    # backward weight: exactly the route the launch takes.  C5 takes the
    # implicit kernel: 64 k-slices of [OC, K_col] partials (no column buffer)
    c5 = (32, 64, 64, 56, 56, 3, 3, 1, 1, 1, 1)
    need = L.lib().cdx_conv2d_backward_weight_workspace_size(*c5)
    assert need == 64 * 64 * 576 * 4
    assert _status("cdx_conv2d_backward_weight_f32", fake, fake, fake, *c5, 0, fake, need - 1,
                   None) == L.CDX_ERR_WORKSPACE
    # beyond the implicit kernel's 32-bit range (a 2^15 x 2^15 plane): the GEMM
    # route's column buffer, then its split-K partials (768 slices of 1 x 1)
    assert L.lib().cdx_conv2d_backward_weight_workspace_size(1, 1, 1, 2 ** 15, 2 ** 15, 1, 1,
                                                             1, 1, 0, 0) \
        == 2 ** 30 * 4 + 768 * 4
    # Winograd backward data: the transposed problem (OC in, IC out, IH x IW tiles)
    assert L.lib().cdx_conv2d_backward_data_winograd_workspace_size(32, 64, 64, 56, 56, 1, 1) \
        == 36 * (64 * 64 + 2 * 64 * 32 * 14 * 14) * 4
    assert L.lib().cdx_conv2d_backward_data_winograd_workspace_size(1, 2, 2, 8, 8, 3, 3) == 0
    assert _status("cdx_conv2d_backward_data_winograd_f32", fake, fake, fake, 1, 2, 2, 8, 8, 3, 0,
                   0, None, 0, None) == L.CDX_ERR_UNSUPPORTED
    assert _status("cdx_conv2d_backward_data_winograd_f32", fake, fake, fake, 1, 2, 2, 8, 8, 1, 1,
                   0, fake, 4, None) == L.CDX_ERR_WORKSPACE
    # GEMM split-K scratch: C4's dW1 (256 x 784 x 8192, TN) in FP32 runs 29
    # slices of 288 k on the 128x64 split-K tile (26 tiles); 4096^3 never splits
    assert L.lib().cdx_gemm_workspace_size(0, 1, 0, 256, 784, 8192) == 29 * 256 * 784 * 4
    assert L.lib().cdx_gemm_workspace_size(0, 0, 0, 4096, 4096, 4096) == 0
    assert L.lib().cdx_gemm_workspace_size(1, 0, 0, 4096, 4096, 4096) == 0
    assert L.lib().cdx_gemm_workspace_size(0, 0, 0, 0, 4096, 4096) == 0
    assert L.lib().cdx_gemm_workspace_size(7, 0, 0, 16, 16, 16) == 0     # bad precision
    assert _status("cdx_gemm_ex_ws", 0, 1, 0, 256, 784, 8192, fake, 256, fake, 784, fake, 784,
                   None, 0, 0, fake, 4, None) == L.CDX_ERR_WORKSPACE
    # 8192 rows -> 256 chunks of 32 rows; partials sized for fp64
    assert L.lib().cdx_sum_reduce_rows_workspace_size(8192, 256) == 256 * 256 * 8
    assert L.lib().cdx_sum_reduce_rows_workspace_size(10 ** 7, 3) == 1024 * 3 * 8
    assert _status("cdx_activation_forward_f32", fake, fake, 4, 0, 0.01, None) == L.CDX_ERR_INVALID_ARG
    assert _status("cdx_activation_forward_f32", fake, fake, 4, 7, 0.01, None) == L.CDX_ERR_INVALID_ARG
    assert _status("cdx_activation_backward_f64", fake, fake, fake, 4, 7, 0.01, None) \
        == L.CDX_ERR_INVALID_ARG
    assert _status("cdx_activation_forward_f32", None, fake, 4, L.ACT_TANH, 0.01, None) \
        == L.CDX_ERR_INVALID_ARG
    assert _status("cdx_sum_reduce_rows_f32", None, fake, 4, 4, None, 0, None) \
        == L.CDX_ERR_INVALID_ARG


def test_missing_library_raises(monkeypatch, tmp_path):
    monkeypatch.setattr(L, "_lib", None)
    monkeypatch.setattr(L, "LIB_PATH", str(tmp_path / "nope.so"))
    with pytest.raises(ImportError):
        L.lib()


def test_fused_gemm_argument_validation():
    fake = ctypes.c_void_p(0x1000)
    args = (0, 0, 0, 4, 4, 4, fake, 4, fake, 4, fake, 4)

    def st(bias, bias_mode, epi, aux, ldaux, colsum):
        return _status("cdx_gemm_fused", *args, bias, bias_mode, epi, aux, ldaux, colsum,
                       None, 0, None)
    assert st(fake, L.BIAS_COL, L.EPI_BWD_RELU, fake, 4, None) == L.CDX_ERR_INVALID_ARG
    assert b"bias" in L.lib().cdx_last_error()
    assert st(None, 0, L.EPI_BWD_GELU, None, 4, None) == L.CDX_ERR_INVALID_ARG      # no aux
    assert st(None, 0, L.EPI_BWD_RELU, fake, 3, None) == L.CDX_ERR_INVALID_ARG      # ldaux < N
    assert st(None, 0, L.EPI_RELU, fake, 4, None) == L.CDX_ERR_INVALID_ARG          # aux w/o BWD
    assert st(None, 0, 12, None, 0, None) == L.CDX_ERR_INVALID_ARG                  # bad epilogue
    assert st(None, 0, L.EPI_RELU, None, 0, fake) == L.CDX_ERR_INVALID_ARG          # colsum + act
    assert st(fake, L.BIAS_ROW, 0, None, 0, fake) == L.CDX_ERR_INVALID_ARG          # colsum + bias
    # workspace: C4's dW1 with its bias gradient -- 29 k-slices of [256, 785]
    assert L.lib().cdx_gemm_fused_workspace_size(0, 1, 0, 256, 784, 8192, 1) == 29 * 256 * 785 * 4
    assert L.lib().cdx_gemm_fused_workspace_size(1, 1, 0, 256, 784, 8192, 1) == 29 * 256 * 785 * 4
    assert L.lib().cdx_gemm_fused_workspace_size(0, 1, 0, 256, 784, 8192, 0) == 29 * 256 * 784 * 4
