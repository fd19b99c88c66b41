"""CPU-side checks of the drop-in Python surface: the native module and the
cuDeep package import without a GPU, expose the reference's names, and
fail loudly (RuntimeError) instead of falling back when no GPU exists."""
import pytest


def test_import_surface():
    from cudeep_amd import cuDeep, _cudeep_core
    for name in ("Tensor", "DType", "Layout", "Stream", "Event", "MemoryPool", "relu", "gelu",
                 "activation_backward", "broadcast_add", "sum_reduce_rows", "sum",
                 "conv2d_forward", "conv2d_backward_data", "conv2d_backward_weight",
                 "device_info", "linear_forward", "matmul_ex", "conv2d_backward_bias",
                 "linear_weight_grad"):
        assert hasattr(_cudeep_core, name), name
    for name in ("Tensor", "nn", "init", "autograd", "no_grad", "conv2d", "linear",
                 "broadcast_add", "relu", "gelu"):
        assert hasattr(cuDeep, name), name
    assert {"Linear", "Conv2d", "ReLU", "GELU", "Sequential", "Module", "Parameter"} <= set(
        dir(cuDeep.nn))
    assert {"xavier_uniform_", "kaiming_normal_", "zeros_"} <= set(dir(cuDeep.init))


def test_precision_switch():
    from cudeep_amd import cuDeep
    prev = cuDeep.get_matmul_precision()
    assert prev in ("fp32", "tf32")
    cuDeep.set_matmul_precision("fp32")
    assert cuDeep.get_matmul_precision() == "fp32"
    cuDeep.set_matmul_precision("tf32")
    assert cuDeep.get_matmul_precision() == "tf32"
    with pytest.raises(RuntimeError):
        cuDeep.set_matmul_precision("bf16")
    cuDeep.set_matmul_precision(prev)


def test_no_cpu_fallback_without_gpu():
    torch = pytest.importorskip("torch")
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    from cudeep_amd import cuDeep
    with pytest.raises(RuntimeError):
        cuDeep.Tensor.zeros([2, 2])


def test_one_hip_runtime_whatever_the_import_order():
    """Importing this package before torch must not map a second HIP runtime
    (torch's wheel bundles its own libamdhip64.so; two runtimes in one
    process leave one of them without a device)."""
    import os
    import subprocess
    import sys
    pytest.importorskip("torch")
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    code = ("import os, cudeep_amd.cuDeep, torch\n"
            "maps = open(f'/proc/{os.getpid()}/maps').read().splitlines()\n"
            "print(len({l.split()[-1] for l in maps if 'libamdhip64' in l}))\n")
    out = subprocess.run([sys.executable, "-c", code], cwd=root, capture_output=True,
                         text=True, timeout=300, env=dict(os.environ, PYTHONPATH=root))
    assert out.returncode == 0, out.stderr
    assert out.stdout.strip() == "1"
