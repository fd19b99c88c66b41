"""Bridge to the compiled extension, as python/cuDeep/_core.py:3-35 of the
reference: imports the native `_cudeep_core` module (built in-tree next to
libcudeep.so / libcudeep_amd.so) and fails loudly if it is missing."""

try:
    from cudeep_amd._cudeep_core import (  # type: ignore[import-not-found]
        Tensor,
        DType,
        Layout,
        Stream,
        Event,
        MemoryPool,
        relu, gelu, sigmoid, silu, tanh_act, leaky_relu, activation_backward,
        broadcast_add, sum_reduce_rows, sum,
        matmul_ex, linear_forward, linear_weight_grad, linear_input_grad,
        conv2d_forward, conv2d_backward_data, conv2d_backward_weight, conv2d_backward_bias,
        set_matmul_precision, get_matmul_precision, set_conv_algorithm, get_conv_algorithm,
        device_info,
    )
except ImportError as e:  # pragma: no cover - exercised when the build is missing
    raise ImportError(
        "cuDeep native extension (_cudeep_core) not found. Build it first: "
        "python -c 'import __graft_entry__ as g; g.build()' (make -C cudeep_amd/csrc)"
    ) from e
