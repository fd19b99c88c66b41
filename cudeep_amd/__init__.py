"""cudeep_amd -- MI355X (gfx950) implementation of cuDeep's dense-contraction
hot path: FP32 MFMA SGEMM, TF32-mode (bf16x3) GEMM, fused bias/ReLU/GELU
epilogues, im2col + Conv2d forward, and the Linear helpers, behind the C-ABI
in include/cudeep_amd.h (libcudeep_amd.so)."""
from ._runtime import share_torch_hip_runtime

# before any native library of this package is loaded
HIP_RUNTIME = share_torch_hip_runtime()

from . import _lib  # noqa: E402,F401
from ._lib import (ACT_LEAKY_RELU, ACT_TANH, CdxError, EPI_GELU, EPI_NONE, EPI_RELU,  # noqa: F401
                   EPI_SIGMOID, EPI_SILU, EPI_BWD_GELU, EPI_BWD_RELU, EPI_BWD_SIGMOID,
                   EPI_BWD_SILU,
                   BIAS_COL, BIAS_NONE, BIAS_ROW, OP_N, OP_T, PREC_FP32, PREC_TF32MODE,
                   PREC_TF32MODE4)

__version__ = "0.1.0"
