#!/usr/bin/env python3
"""Benchmark of the MI355X dense-contraction path (one GPU).

Headline (BASELINE.json metric): FP32 GEMM TFLOP/s at M=N=K=4096 (config
C2, A, B ~ N(0,1), beta=0) and its fraction of the MI355X FP32 MFMA peak
(157.3 TFLOP/s).  A "step" is one 4096^3 FP32 GEMM through cdx_sgemm_f32,
with A, B, C resident in HBM.  The same run also reports, under "extra":
TF32-mode (bf16x3) GEMM at 2048^3 / 4096^3 (C3), the MLP Linear stack (C4)
and the im2col + GEMM Conv2d (C5).

Timing: W untimed warmup steps, then K back-to-back steps between one HIP
event pair recorded on the stream the library launches on (torch's current
stream), bracketed by torch.cuda.synchronize().  The headline's roofline
figure divides the FLOPs of one launch by the timed region's duration over
K (its average launch duration); per-launch event pairs, timed after the
region, are reported beside it.

cpu_baseline: the repo's host reference SGEMM (oracle/, the sequential-FMA
restatement of the reference SGEMM, OpenMP over all host cores) timed on
the same 4096^3 problem: 1 warmup + median of 3.  It is a reported
baseline, not the optimisation target.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--headline-only]
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

FP32_PEAK_TFLOPS = 157.3      # MI355X dense FP32 MFMA
BF16_PEAK_TFLOPS = 2516.6     # MI355X dense BF16 MFMA; bf16x3 logical ceiling = /3
HEAD_SETTLE_S = 0.3           # untimed clock-settling launches before the headline
HBM_PEAK_GBS = 8000.0
MLP_SETTLE_S = 0.3            # untimed settling launches before each C4 step line


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    # 100 warmup launches (0.1 s at 4096^3): the clock settles over the first
    # ~10-40 ms of sustained MFMA work (4096^3 FP32: 1.037 ms per launch with
    # 10 warmup launches, 1.016 ms with 100)
    p.add_argument("--warmup", type=int, default=100)
    p.add_argument("--headline-only", action="store_true",
                   help="time only the 4096^3 FP32 GEMM (for profiler runs)")
    p.add_argument("--tf32-only", action="store_true",
                   help="time only the 4096^3 TF32-mode GEMM (for profiler runs); prints "
                        "its line to stderr and no JSON")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    p.add_argument("--copy-calibration", action="store_true",
                   help="also run a plain 256 MiB device copy (reference point for "
                        "rocprofv3 FETCH_SIZE / WRITE_SIZE counters)")
    return p.parse_args()


def time_launches(fn, steps, warmup, min_warm_s=0.0, per_call=False):
    """Runs fn() warmup times (and, with min_warm_s, keeps going in batches
    of 10 until that much wall time has passed), then times exactly `steps`
    back-to-back calls between one HIP event pair on the current stream,
    with a device synchronisation on both sides.  Returns (mean ms per step,
    per-launch ms list or None).  per_call: afterwards, `steps` more calls,
    each between an event pair of its own, give per-launch durations.  Those
    calls are not the timed region: on this runtime a timing event recorded
    between two calls leaves the GPU idle for 6-10 us (C5 conv route in TF32
    mode: 109 us per call with a pair per call, 100 us without; 4096^3 FP32
    GEMM: 987 against 981 us)."""
    import torch
    t0 = time.perf_counter()
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    while time.perf_counter() - t0 < min_warm_s:
        for _ in range(10):
            fn()
        torch.cuda.synchronize()
    outer0 = torch.cuda.Event(enable_timing=True)
    outer1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    outer0.record()
    for _ in range(steps):
        fn()
    outer1.record()
    torch.cuda.synchronize()
    ms = outer0.elapsed_time(outer1) / steps
    if not per_call:
        return ms, None
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(steps)]
    for e0, e1 in evs:
        e0.record()
        fn()
        e1.record()
    torch.cuda.synchronize()
    return ms, [e0.elapsed_time(e1) for e0, e1 in evs]


def per_launch_ms(steps, warmup, fn, reps=20):
    """Kernel time of fn's launches: a HIP graph of `reps` back-to-back calls,
    replayed `steps` times after `warmup` replays (no per-launch host cost;
    fn must take its scratch from preallocated buffers)."""
    import torch
    for _ in range(3):
        fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(reps):
            fn()
    ms, _ = time_launches(g.replay, steps, warmup)
    return ms / reps


def bench_gemm(n, precision, steps, warmup, seed, min_warm_s=0.0):
    import torch
    import cudeep_amd.ops as ops
    import cudeep_amd as cd
    g = torch.Generator(device="cuda").manual_seed(seed)
    A = torch.randn((n, n), device="cuda", generator=g)
    B = torch.randn((n, n), device="cuda", generator=g)
    C = torch.empty((n, n), device="cuda")
    if precision == cd.PREC_FP32:
        def f():
            ops.sgemm(A, B, out=C)           # cdx_sgemm_f32
    else:
        def f():
            ops.gemm(A, B, precision=precision, out=C)
    ms, per = time_launches(f, steps, warmup, min_warm_s, per_call=True)
    flops = 2.0 * n ** 3
    return {"n": n, "ms_per_step": ms, "kernel_ms_mean": statistics.mean(per),
            "kernel_ms_median": statistics.median(per),
            "tflops": flops / (ms * 1e-3) / 1e12,
            "tflops_kernel_median": flops / (statistics.median(per) * 1e-3) / 1e12}


def bench_gemm16(n, dtype, steps, warmup, seed, min_warm_s=0.0):
    """16-bit-operand GEMM (cdx_gemm16_ex): fp16 / bf16 A, B, fp32 C."""
    import torch
    import cudeep_amd.ops as ops
    g = torch.Generator(device="cuda").manual_seed(seed)
    td = torch.float16 if dtype == "f16" else torch.bfloat16
    A = torch.randn((n, n), device="cuda", generator=g).to(td)
    B = torch.randn((n, n), device="cuda", generator=g).to(td)
    C = torch.empty((n, n), device="cuda")
    ms, per = time_launches(lambda: ops.gemm16(A, B, out=C), steps, warmup, min_warm_s,
                            per_call=True)
    flops = 2.0 * n ** 3
    return {"n": n, "ms_per_step": ms, "kernel_ms_median": statistics.median(per),
            "tflops": flops / (ms * 1e-3) / 1e12,
            "frac_of_bf16_peak": flops / (ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS}


def bench_mlp(steps, warmup, precision):
    """C4: 784 -> 256 -> 10, batch 8192: fused forward (bias+ReLU epilogue)
    and backward: dW GEMMs that also form the bias gradients (ones column),
    the ReLU mask in the epilogue of dH = dY2 W2, dX = dZ W1."""
    import torch
    import cudeep_amd.ops as ops
    import cudeep_amd as cd
    g = torch.Generator(device="cuda").manual_seed(4)
    X = torch.randn((8192, 784), device="cuda", generator=g)
    W1 = (torch.rand((256, 784), device="cuda", generator=g) * 2 - 1) * (6 / (784 + 256)) ** 0.5
    W2 = (torch.rand((10, 256), device="cuda", generator=g) * 2 - 1) * (6 / (256 + 10)) ** 0.5
    b1 = torch.randn((256,), device="cuda", generator=g) * 0.1
    b2 = torch.randn((10,), device="cuda", generator=g) * 0.1
    dY2 = torch.randn((8192, 10), device="cuda", generator=g)
    H = torch.empty((8192, 256), device="cuda")
    Y = torch.empty((8192, 10), device="cuda")
    dZ = torch.empty((8192, 256), device="cuda")
    gW2 = torch.empty((10, 256), device="cuda")
    gW1 = torch.empty((256, 784), device="cuda")
    gX = torch.empty((8192, 784), device="cuda")
    gb1 = torch.empty((256,), device="cuda")
    gb2 = torch.empty((10,), device="cuda")

    # Every launch takes its scratch from a preallocated workspace, so the
    # step allocates nothing and can be captured as a HIP graph.
    def wsp(nbytes):
        return torch.empty(max(nbytes, 4) // 4 + 1, device="cuda")
    ws_w2 = wsp(ops.gemm_workspace_bytes(10, 256, 8192, precision=precision, transA=True,
                                         colsum=True))
    ws_w1 = wsp(ops.gemm_workspace_bytes(256, 784, 8192, precision=precision, transA=True,
                                         colsum=True))
    ws_x = wsp(ops.gemm_workspace_bytes(8192, 784, 256, precision=precision))
    ws_h = wsp(ops.gemm_workspace_bytes(8192, 256, 10, precision=precision))
    ws_f1 = wsp(ops.gemm_workspace_bytes(8192, 256, 784, precision=precision, transB=True))
    ws_f2 = wsp(ops.gemm_workspace_bytes(8192, 10, 256, precision=precision, transB=True))

    def fwd1():
        ops.gemm(X, W1, transB=True, bias=b1, bias_mode=cd.BIAS_COL, epilogue=cd.EPI_RELU,
                 precision=precision, out=H, workspace=ws_f1)

    def fwd2():
        ops.gemm(H, W2, transB=True, bias=b2, bias_mode=cd.BIAS_COL, precision=precision, out=Y,
                 workspace=ws_f2)

    def fwd():
        fwd1()
        fwd2()

    def bwd_layer2():
        # dW2 = dY2^T H and db2 = column sums of dY2, one launch (+ split-K reduction)
        ops.gemm(dY2, H, transA=True, precision=precision, out=gW2, colsum=gb2, workspace=ws_w2)

    def bwd_mask():
        # dZ = (dY2 W2) * (H > 0): the ReLU backward in the GEMM's epilogue
        ops.gemm(dY2, W2, precision=precision, out=dZ, epilogue=cd.EPI_BWD_RELU, aux=H,
                 workspace=ws_h)

    def bwd_layer1():
        # dW1 = dZ^T X and db1 = column sums of dZ, one launch (+ reduction)
        ops.gemm(dZ, X, transA=True, precision=precision, out=gW1, colsum=gb1, workspace=ws_w1)

    def bwd_dx():
        ops.gemm(dZ, W1, precision=precision, out=gX, workspace=ws_x)          # dX = dZ W1

    def bwd():
        bwd_layer2()
        bwd_mask()
        bwd_layer1()
        bwd_dx()

    # (each step line keeps launching untimed for MLP_SETTLE_S after its warmup:
    # the first C4 lines of a process otherwise read ~10 us per step slower, for
    # a few hundred ms after the previous line's load, with every kernel's own
    # graph-timed duration unchanged)
    fwd_ms, _ = time_launches(fwd, steps, warmup, min_warm_s=MLP_SETTLE_S)
    bwd_ms, _ = time_launches(bwd, steps, warmup, min_warm_s=MLP_SETTLE_S)
    fwd_flops = 2.0 * 8192 * (784 * 256 + 256 * 10)
    bwd_flops = 2 * fwd_flops

    # The same step as one HIP graph: at this size the eager step is bound by
    # per-launch host work (Python + ctypes), which replaying a captured
    # graph removes.
    def step():
        fwd()
        bwd()

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            step()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    graph_ms, _ = time_launches(graph.replay, steps, warmup, min_warm_s=MLP_SETTLE_S)

    # The same step with its independent branches on two side streams, each
    # launch on its own workspace: with the output gradient dY2 given, layer
    # 2's forward and its weight + bias gradient need only H, so they run
    # beside the masked dH; layer 1's weight + bias gradient beside dX.
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()

    def step_forked():
        main = torch.cuda.current_stream()
        fwd1()
        s1.wait_stream(main)
        with torch.cuda.stream(s1):
            fwd2()
            bwd_layer2()
        bwd_mask()
        s2.wait_stream(main)
        with torch.cuda.stream(s2):
            bwd_layer1()
        bwd_dx()
        main.wait_stream(s1)
        main.wait_stream(s2)

    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            step_forked()
    torch.cuda.current_stream().wait_stream(side)
    graph2 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph2):
        step_forked()
    graph2_ms, _ = time_launches(graph2.replay, steps, warmup, min_warm_s=MLP_SETTLE_S)
    # the big forward GEMM and the two narrow products on their own, each as
    # a HIP graph of 20 back-to-back launches (kernel time, not the ~20 us
    # per-launch host cost of an eager ctypes call)
    l1_ms = per_launch_ms(steps, warmup, lambda: ops.gemm(X, W1, transB=True, bias=b1, bias_mode=cd.BIAS_COL,
                                           epilogue=cd.EPI_RELU, precision=precision, out=H,
                                           workspace=ws_f1))
    l2_ms = per_launch_ms(steps, warmup, lambda: ops.gemm(H, W2, transB=True, bias=b2, bias_mode=cd.BIAS_COL,
                                           precision=precision, out=Y, workspace=ws_f2))
    dh_ms = per_launch_ms(steps, warmup, bwd_mask)
    return {"fwd_ms": fwd_ms, "bwd_ms": bwd_ms,
            "fwd_tflops": fwd_flops / (fwd_ms * 1e-3) / 1e12,
            "bwd_tflops": bwd_flops / (bwd_ms * 1e-3) / 1e12,
            "step_graph_ms": graph_ms,
            "step_graph_tflops": (fwd_flops + bwd_flops) / (graph_ms * 1e-3) / 1e12,
            "step_graph_forked_ms": graph2_ms,
            "step_graph_forked_tflops": (fwd_flops + bwd_flops) / (graph2_ms * 1e-3) / 1e12,
            "fwd1_fused_ms": l1_ms,
            "fwd1_fused_tflops": 2.0 * 8192 * 784 * 256 / (l1_ms * 1e-3) / 1e12,
            "fwd2_ms": l2_ms, "dh_masked_ms": dh_ms, "settle_s": MLP_SETTLE_S}


def bench_mlp_api(steps, warmup, precision):
    """C4 forward + backward through the drop-in Python API: cuDeep.nn
    Sequential(Linear(784, 256), ReLU, Linear(256, 10)) -> _cudeep_core ->
    libcudeep.so -> the C-ABI, with the output gradient given (y.backward(dY)),
    timed eagerly, host work included."""
    import numpy as np
    import torch
    from cudeep_amd import cuDeep
    prev = cuDeep.get_matmul_precision()
    cuDeep.set_matmul_precision("fp32" if precision == 0 else "tf32")
    nn, T = cuDeep.nn, cuDeep.Tensor
    rng = np.random.default_rng(4)
    model = nn.Sequential(nn.Linear(784, 256), nn.ReLU(), nn.Linear(256, 10))
    cuDeep.init.xavier_uniform_(model[0].weight)
    cuDeep.init.xavier_uniform_(model[2].weight)
    # the input requires its gradient: C4's backward includes dX of the first
    # layer (dX = dY W)
    X = T.from_numpy(rng.standard_normal((8192, 784), dtype=np.float32), requires_grad=True)
    dY = T.from_numpy(rng.standard_normal((8192, 10), dtype=np.float32))

    def step():
        model.zero_grad()
        X.grad = None
        y = model(X)
        y.backward(dY)

    # (untimed settling: the first steps fill the runtime's allocation caches)
    ms, _ = time_launches(step, steps, warmup, min_warm_s=0.2)
    cuDeep.set_matmul_precision(prev)
    flops = 3 * 2.0 * 8192 * (784 * 256 + 256 * 10)
    return {"step_ms": ms, "step_tflops": flops / (ms * 1e-3) / 1e12}


def bench_conv(steps, warmup, precision):
    """C5: N=32, C=64, 56x56 -> 64, 3x3, s1, p1: im2col + GEMM (bias in the
    epilogue, output written NCHW), Winograd, the implicit GEMM, the backward
    routes; and a 7x7 layer of the same size (implicit route)."""
    import torch
    import cudeep_amd as cd
    import cudeep_amd.ops as ops
    g = torch.Generator(device="cuda").manual_seed(5)
    x = torch.randn((32, 64, 56, 56), device="cuda", generator=g)
    w = torch.randn((64, 64, 3, 3), device="cuda", generator=g) * (2.0 / 576) ** 0.5
    b = torch.randn((64,), device="cuda", generator=g) * 0.1
    ws = torch.empty(ops.conv2d_workspace_bytes(x.shape, w.shape, (1, 1), (1, 1)) // 4,
                     device="cuda")
    y = torch.empty((32, 64, 56, 56), device="cuda")
    col = torch.empty((576, 100352), device="cuda")   # the whole batch's column buffer
    conv_ms, _ = time_launches(lambda: ops.conv2d_forward(x, w, b, (1, 1), (1, 1), precision,
                                                          workspace=ws, out=y), steps, warmup,
                               min_warm_s=0.2)
    im_ms = per_launch_ms(steps, warmup, lambda: ops.im2col(x, 3, 3, (1, 1), (1, 1), out=col))
    flops = 2.0 * 32 * 64 * 56 * 56 * 64 * 9
    im2col_bytes = 576 * 100352 * 4 + 32 * 64 * 56 * 56 * 4
    # Winograd F(4x4, 3x3) route (the reference's route for this layer); TFLOP/s
    # counted with the direct-convolution FLOPs, as for the im2col route
    wws = torch.empty(ops.conv2d_winograd_workspace_bytes(x.shape, 64, (1, 1)) // 4,
                      device="cuda")
    wino_ms, _ = time_launches(lambda: ops.conv2d_winograd(x, w, b, (1, 1), precision,
                                                           workspace=wws, out=y), steps, warmup)
    # backward: data (stride 1: the row-window implicit conv of dY with the
    # flipped filter; or Winograd on the transposed conv), weight (the
    # row-window implicit weight-gradient kernel), bias
    dy = torch.randn((32, 64, 56, 56), device="cuda", generator=g)
    dx = torch.empty_like(x)
    dw = torch.empty_like(w)
    db = torch.empty_like(b)
    dws = torch.empty(ops.conv2d_backward_data_winograd_workspace_bytes(x.shape, 64, (1, 1)) // 4,
                      device="cuda")

    def bwd_data():
        ops.conv2d_backward_data(dy, w, x.shape, (1, 1), (1, 1), precision, out=dx)

    def bwd_data_wino():
        ops.conv2d_backward_data_winograd(dy, w, x.shape, (1, 1), precision, workspace=dws, out=dx)

    def bwd_weight():
        ops.conv2d_backward_weight(dy, x, w.shape, (1, 1), (1, 1), precision, out=dw)

    # the routes launch_conv2d_backward_data_kernel takes (Auto): Winograd in
    # the TF32 modes, the flipped-filter implicit conv in FP32
    bwd_data_auto = bwd_data if precision == cd.PREC_FP32 else bwd_data_wino

    def bwd():
        bwd_data_auto()
        bwd_weight()
        ops.conv2d_backward_bias(dy, out=db)
    bwd_ms, _ = time_launches(bwd, steps, warmup)
    bd_ms, _ = time_launches(bwd_data, steps, warmup)
    bdw_ms, _ = time_launches(bwd_data_wino, steps, warmup)
    bw_ms, _ = time_launches(bwd_weight, steps, warmup)
    # the im2col route's GEMM on its own (weight [64, 576] x col [576, 100352],
    # plain row-major output instead of the NCHW map; same kernel family)
    gflat = torch.empty((64, 100352), device="cuda")
    gemm_ms = per_launch_ms(steps, warmup, lambda: ops.gemm(w.view(64, 576), col,
                                                           precision=precision, out=gflat))
    # implicit GEMM (no column buffer): this layer forced through it, and a
    # 7x7 layer of the same size, which the forward routes there (its column
    # buffer would be 1.26 GB)
    imp_ms, _ = time_launches(lambda: ops.conv2d_implicit(x, w, b, (1, 1), (1, 1), out=y),
                              steps, warmup)
    imp_kernel_ms = per_launch_ms(steps, warmup,
                                  lambda: ops.conv2d_implicit(x, w, b, (1, 1), (1, 1), out=y))
    w7 = torch.randn((64, 64, 7, 7), device="cuda", generator=g) * (2.0 / 3136) ** 0.5
    c7_ms, _ = time_launches(lambda: ops.conv2d_forward(x, w7, b, (1, 1), (3, 3), precision,
                                                        out=y), max(3, steps // 5), 3)
    flops7 = 2.0 * 32 * 64 * 56 * 56 * 64 * 49
    return {"conv_ms": conv_ms, "conv_tflops": flops / (conv_ms * 1e-3) / 1e12,
            "gemm_ms": gemm_ms, "gemm_tflops": flops / (gemm_ms * 1e-3) / 1e12,
            "implicit_3x3_ms": imp_ms, "implicit_3x3_tflops": flops / (imp_ms * 1e-3) / 1e12,
            "implicit_3x3_kernel_ms": imp_kernel_ms,
            "implicit_3x3_kernel_tflops": flops / (imp_kernel_ms * 1e-3) / 1e12,
            "conv7x7_implicit_ms": c7_ms,
            "conv7x7_implicit_tflops": flops7 / (c7_ms * 1e-3) / 1e12,
            "bwd_ms": bwd_ms, "bwd_tflops": 2 * flops / (bwd_ms * 1e-3) / 1e12,
            "bwd_data_implicit_ms": bd_ms, "bwd_data_winograd_ms": bdw_ms,
            "bwd_weight_ms": bw_ms,
            "im2col_ms": im_ms, "im2col_gbs": im2col_bytes / (im_ms * 1e-3) / 1e9,
            "winograd_ms": wino_ms, "winograd_tflops_equiv": flops / (wino_ms * 1e-3) / 1e12}


def bench_conv_api(steps, warmup, precision):
    """C5 forward (and forward + backward) through the drop-in Python API:
    cuDeep.nn.Conv2d(64, 64, 3, padding=1) on [32, 64, 56, 56] ->
    _cudeep_core -> libcudeep.so -> the C-ABI (the reference's routing: Winograd
    for this 3x3 stride-1 layer), timed eagerly, host work included."""
    import numpy as np
    from cudeep_amd import cuDeep
    prev = cuDeep.get_matmul_precision()
    cuDeep.set_matmul_precision("fp32" if precision == 0 else "tf32")
    T = cuDeep.Tensor
    rng = np.random.default_rng(5)
    conv = cuDeep.nn.Conv2d(64, 64, 3, padding=1)
    cuDeep.init.kaiming_normal_(conv.weight)
    x = T.from_numpy(rng.standard_normal((32, 64, 56, 56), dtype=np.float32))
    dy = T.from_numpy(rng.standard_normal((32, 64, 56, 56), dtype=np.float32))
    with cuDeep.no_grad():
        fwd_ms, _ = time_launches(lambda: conv(x), steps, warmup, min_warm_s=0.2)
    xg = T.from_numpy(rng.standard_normal((32, 64, 56, 56), dtype=np.float32), requires_grad=True)

    def step():
        conv.zero_grad()
        xg.grad = None
        conv(xg).backward(dy)

    step_ms, _ = time_launches(step, steps, warmup, min_warm_s=0.2)
    cuDeep.set_matmul_precision(prev)
    fl = 2.0 * 32 * 64 * 56 * 56 * 64 * 9
    return {"fwd_ms": fwd_ms, "fwd_tflops": fl / (fwd_ms * 1e-3) / 1e12,
            "step_ms": step_ms, "step_tflops": 3 * fl / (step_ms * 1e-3) / 1e12}


def cpu_baseline(n=4096):
    """Repo host reference SGEMM (oracle, seq-FMA restatement), all cores."""
    import numpy as np
    import oracle
    oracle.build()
    cores = os.cpu_count() or 1
    oracle.set_num_threads(cores)
    rng = np.random.default_rng(2)
    A = rng.standard_normal((n, n)).astype(np.float32)
    B = rng.standard_normal((n, n)).astype(np.float32)
    t_med = _cpu_time(lambda: oracle.sgemm_seqfma(A, B))
    # the other configs on the same (still warm) OpenMP threads, before NumPy:
    # its BLAS threads keep spinning for a while after a call and then compete
    # with the oracle's threads for the cores
    configs = cpu_configs()
    t_np = _cpu_time(lambda: A @ B)
    flops = 2.0 * n ** 3
    return {"value": flops / t_med / 1e12, "unit": "TFLOP/s", "cores": oracle.num_threads(),
            "kind": "port",
            "sample": f"full {n}^3 FP32 GEMM, seq-FMA host reference (oracle/oracle.c), "
                      f"1 warmup + median of 3 ({t_med:.2f} s each)",
            "numpy_f32_tflops": flops / t_np / 1e12,
            "numpy_sample": "NumPy float32 A @ B on the same operands, all cores, "
                            "1 warmup + median of 3, timed after the host reference",
            "configs": configs}


def _cpu_time(fn, reps=3):
    fn()
    ts = []
    for _ in range(reps):
        t = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t)
    return statistics.median(ts)


def cpu_configs():
    """The same host reference (oracle/: seq-FMA SGEMM, im2col + SGEMM conv)
    on the other configs, bounded samples: C1 in full; C4 forward + backward
    on 1024 of the 8192 batch rows; C5 forward on 2 of the 32 images.  Rates
    are the sample's algorithmic FLOPs / median wall time (1 warmup + 3)."""
    import numpy as np
    import oracle
    rng = np.random.default_rng(7)
    out = {}
    A = rng.uniform(-1, 1, (512, 512)).astype(np.float32)
    B = rng.uniform(-1, 1, (512, 512)).astype(np.float32)
    t = _cpu_time(lambda: oracle.sgemm_seqfma(A, B), reps=5)
    out["c1_512"] = {"tflops": 2.0 * 512 ** 3 / t / 1e12, "ms": t * 1e3, "sample": "full 512^3"}

    rows = 1024
    X = rng.standard_normal((rows, 784)).astype(np.float32)
    W1 = rng.uniform(-0.07596, 0.07596, (256, 784)).astype(np.float32)
    W2 = rng.uniform(-0.1502, 0.1502, (10, 256)).astype(np.float32)
    b1 = (rng.standard_normal(256) * 0.1).astype(np.float32)
    b2 = (rng.standard_normal(10) * 0.1).astype(np.float32)
    dY2 = rng.standard_normal((rows, 10)).astype(np.float32)

    def mlp_step():
        H = np.maximum(oracle.sgemm_seqfma(X, W1, transB=True) + b1, 0)
        oracle.sgemm_seqfma(H, W2, transB=True) + b2
        dH = oracle.sgemm_seqfma(dY2, W2)
        oracle.sgemm_seqfma(dY2, H, transA=True)
        dY2.sum(0)
        dZ = dH * (H > 0)
        oracle.sgemm_seqfma(dZ, W1)
        oracle.sgemm_seqfma(dZ, X, transA=True)
        dZ.sum(0)
    t = _cpu_time(mlp_step)
    fl = 3 * 2.0 * rows * (784 * 256 + 256 * 10)
    out["c4_mlp_step"] = {"tflops": fl / t / 1e12, "ms": t * 1e3,
                          "sample": f"forward + backward, {rows} of 8192 batch rows"}

    imgs = 2
    x = rng.standard_normal((imgs, 64, 56, 56)).astype(np.float32)
    w = (rng.standard_normal((64, 64, 3, 3)) * (2.0 / 576) ** 0.5).astype(np.float32)
    b = (rng.standard_normal(64) * 0.1).astype(np.float32)
    t = _cpu_time(lambda: oracle.conv2d_ref_im2col(x, w, b, (1, 1), (1, 1)))
    fl = 2.0 * imgs * 64 * 56 * 56 * 64 * 9
    out["c5_conv_fwd"] = {"tflops": fl / t / 1e12, "ms": t * 1e3,
                          "sample": f"im2col + seq-FMA GEMM + bias, {imgs} of 32 images"}
    return out


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs the hot path on one GPU; --gpus must be 1 "
                                   "(no multi-GPU path is built or run)"}))
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU visible"}))
        sys.exit(1)
    import cudeep_amd as cd
    props = torch.cuda.get_device_properties(0)
    log("device", props.name, getattr(props, "gcnArchName", ""), "CUs", props.multi_processor_count)

    if args.copy_calibration:
        src = torch.randn((64, 1024, 1024), device="cuda")     # 256 MiB
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        log("copy calibration: 3 x 256 MiB device copies (268435456 B read + written each)")

    if args.tf32_only:
        r = bench_gemm(4096, cd.PREC_TF32MODE, args.steps, max(args.warmup, 50), seed=3,
                       min_warm_s=0.1)
        log("tf32mode 4096^3:", r)
        return
    extra = {}
    # The reduced-precision GEMMs run ~12 % slower for their first ~20 ms of
    # back-to-back launches (the clock settles under the new load; measured
    # 344 -> 300 us per 4096^3 TF32-mode launch), so these lines warm up for
    # at least 50 launches and 0.1 s and report the settled rate.
    w_extra = max(args.warmup, 50)
    warm_s = 0.1
    if not args.headline_only:
        for n in (4096, 2048):
            r = bench_gemm(n, cd.PREC_TF32MODE, args.steps, w_extra, seed=3, min_warm_s=warm_s)
            r["frac_of_bf16x3_ceiling"] = r["tflops"] / (BF16_PEAK_TFLOPS / 3)
            extra[f"tf32mode_{n}"] = r
            log(f"tf32mode {n}^3:", r)
        r = bench_gemm(4096, cd.PREC_TF32MODE4, args.steps, w_extra, seed=3, min_warm_s=warm_s)
        r["frac_of_bf16x4_ceiling"] = r["tflops"] / (BF16_PEAK_TFLOPS / 4)
        extra["tf32mode4_4096"] = r
        log("tf32mode4 (bf16x4) 4096^3:", r)
        for dt in ("f16", "bf16"):
            r = bench_gemm16(4096, dt, args.steps, w_extra, seed=6, min_warm_s=warm_s)
            extra[f"{dt}_gemm_4096"] = r
            log(f"{dt} GEMM 4096^3:", r)
    # The headline is timed while the clock is settled under sustained MFMA
    # work: measured on one MI355X, 4096^3 FP32 launches run at 125-126
    # TFLOP/s from idle (or after 0.5 s idle) and at 135 TFLOP/s after 0.3 s
    # of back-to-back MFMA launches.  So it runs straight after the
    # reduced-precision GEMM lines, and after its W warmup launches keeps
    # launching untimed until HEAD_SETTLE_S has passed; the timed region is
    # still exactly K launches.
    log("headline: fp32 4096^3")
    head = bench_gemm(4096, cd.PREC_FP32, args.steps, args.warmup, seed=2,
                      min_warm_s=HEAD_SETTLE_S)
    log("fp32 4096^3:", head)
    if not args.headline_only:
        for prec, name in ((cd.PREC_FP32, "fp32"), (cd.PREC_TF32MODE, "tf32mode")):
            extra[f"mlp_c4_{name}"] = bench_mlp(args.steps, args.warmup, prec)
            log(f"mlp {name}:", extra[f"mlp_c4_{name}"])
            extra[f"conv_c5_{name}"] = bench_conv(args.steps, args.warmup, prec)
            log(f"conv {name}:", extra[f"conv_c5_{name}"])
            extra[f"mlp_c4_api_{name}"] = bench_mlp_api(args.steps, args.warmup, prec)
            log(f"mlp via cuDeep.nn {name}:", extra[f"mlp_c4_api_{name}"])
            extra[f"conv_c5_api_{name}"] = bench_conv_api(args.steps, args.warmup, prec)
            log(f"conv via cuDeep.nn {name}:", extra[f"conv_c5_api_{name}"])
        r = bench_gemm(512, cd.PREC_FP32, 200, 50, seed=1)
        extra["fp32_512"] = r
    cpu = None
    if not args.no_cpu:
        log("cpu baseline")
        cpu = cpu_baseline()
        log("cpu:", cpu)

    # average launch duration of the headline kernel over the timed region
    # (K launches of cdx_sgemm_f32's one kernel, back to back)
    achieved = 2.0 * 4096 ** 3 / (head["ms_per_step"] * 1e-3) / 1e12
    # HBM bytes per launch of the headline kernel, measured offline with two
    # rocprofv3 --pmc runs (FETCH_SIZE, WRITE_SIZE) scaled by a plain-copy
    # calibration; see profiles/gemm_f32_4096_pmc_traffic.md.
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "gemm_f32_4096_traffic.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            traffic = round(json.load(f)["traffic_bytes"])
    out = {
        "metric": "FP32 GEMM TFLOP/s at 4096^3 (+% of FP32 MFMA peak); TF32-mode TFLOP/s",
        "value": round(head["tflops"], 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "warmup_settle_s": HEAD_SETTLE_S,
        "ms_per_step": round(head["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic N(0,1) fp32 operands generated on the GPU (seeded)",
        "config": {"workload": "C2: FP32 SGEMM C=A*B, M=N=K=4096, row-major, beta=0",
                   "M": 4096, "N": 4096, "K": 4096, "entry_point": "cdx_sgemm_f32"},
        "pct_of_fp32_mfma_peak": round(100 * head["tflops"] / FP32_PEAK_TFLOPS, 2),
        "tf32mode_4096_tflops": (round(extra["tf32mode_4096"]["tflops"], 3)
                                 if "tf32mode_4096" in extra else None),
        "roofline": {"bound": "mfma", "achieved": round(achieved, 3), "peak": FP32_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / FP32_PEAK_TFLOPS, 4),
                     "traffic": traffic},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
