"""Allocation-free launches and HIP-graph capture.

cdx_gemm_ex_ws / cdx_sum_reduce_rows_f32 with caller workspaces must give
the same bits as the self-allocating calls, reject a workspace that is too
small, and be capturable: a captured C4-style step (Linear 784 -> 256 -> 10
forward and backward, batch 1024) is replayed several times, with eager work
and synchronisation between replays, and every replay is compared with the
eager step on the same inputs."""
import numpy as np
import pytest

from tests.gpu_util import require_gpu, say

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    require_gpu()


def _ops():
    import cudeep_amd.ops as o
    return o


SPLIT_SHAPES = [  # (M, N, K, transA, transB): long K, few tiles -> split-K
    (256, 784, 8192, True, False),
    (10, 256, 8192, True, False),
    (64, 576, 20000, False, True),
    (33, 70, 4099, False, False),
]


@pytest.mark.parametrize("shape", SPLIT_SHAPES)
@pytest.mark.parametrize("prec", [0, 1, 2])
def test_gemm_workspace_matches_allocating_call(shape, prec):
    import torch
    ops = _ops()
    M, N, K, tA, tB = shape
    g = torch.Generator(device="cuda").manual_seed(M + N + K + prec)
    A = torch.randn((K, M) if tA else (M, K), device="cuda", generator=g)
    B = torch.randn((N, K) if tB else (K, N), device="cuda", generator=g)
    nbytes = ops.gemm_workspace_bytes(M, N, K, precision=prec, transA=tA, transB=tB)
    assert nbytes > 0, "shape chosen to split K"
    say("gemm workspace", shape, "prec", prec, "bytes", nbytes)
    ref = ops.gemm(A, B, precision=prec, transA=tA, transB=tB)
    ws = torch.empty(nbytes // 4, device="cuda")
    got = ops.gemm(A, B, precision=prec, transA=tA, transB=tB, workspace=ws)
    torch.cuda.synchronize()
    assert torch.equal(got, ref)
    small = torch.empty(nbytes // 4 - 1, device="cuda")
    with pytest.raises(Exception):
        ops.gemm(A, B, precision=prec, transA=tA, transB=tB, workspace=small)


def test_gemm_workspace_zero_when_no_split():
    ops = _ops()
    for prec in (0, 1, 2):
        assert ops.gemm_workspace_bytes(4096, 4096, 4096, precision=prec) == 0
        assert ops.gemm_workspace_bytes(8192, 784, 256, precision=prec) == 0


@pytest.mark.parametrize("forked", [False, True])
@pytest.mark.parametrize("prec", [0, 1])
def test_captured_step_replays_match_eager(prec, forked):
    """forked: the backward's independent branches (dW2 + its bias sum beside
    dH and the ReLU mask; dW1 + its bias sum beside dX) captured on two side
    streams, each branch on its own workspaces."""
    import torch
    import cudeep_amd as cd
    ops = _ops()
    Bn = 1024
    g = torch.Generator(device="cuda").manual_seed(40 + prec)
    W1 = torch.randn((256, 784), device="cuda", generator=g) * 0.05
    W2 = torch.randn((10, 256), device="cuda", generator=g) * 0.1
    b1 = torch.randn((256,), device="cuda", generator=g) * 0.1
    b2 = torch.randn((10,), device="cuda", generator=g) * 0.1
    X = torch.empty((Bn, 784), device="cuda")
    dY2 = torch.empty((Bn, 10), device="cuda")
    outs = {k: torch.empty(s, device="cuda") for k, s in
            (("H", (Bn, 256)), ("Y", (Bn, 10)), ("dH", (Bn, 256)), ("dZ", (Bn, 256)),
             ("gW2", (10, 256)), ("gW1", (256, 784)), ("gX", (Bn, 784)), ("gb1", (256,)),
             ("gb2", (10,)))}

    def wsp(nbytes):
        return torch.empty(max(nbytes, 4) // 4 + 1, device="cuda")
    ws = {"w2": wsp(ops.gemm_workspace_bytes(10, 256, Bn, precision=prec, transA=True)),
          "w1": wsp(ops.gemm_workspace_bytes(256, 784, Bn, precision=prec, transA=True)),
          "x": wsp(ops.gemm_workspace_bytes(Bn, 784, 256, precision=prec)),
          "h": wsp(ops.gemm_workspace_bytes(Bn, 256, 10, precision=prec)),
          "f1": wsp(ops.gemm_workspace_bytes(Bn, 256, 784, precision=prec, transB=True)),
          "f2": wsp(ops.gemm_workspace_bytes(Bn, 10, 256, precision=prec, transB=True)),
          "b2": wsp(ops.sum_reduce_rows_workspace_bytes(Bn, 10)),
          "b1": wsp(ops.sum_reduce_rows_workspace_bytes(Bn, 256))}

    def step(o):
        ops.gemm(X, W1, transB=True, bias=b1, bias_mode=cd.BIAS_COL, epilogue=cd.EPI_RELU,
                 precision=prec, out=o["H"], workspace=ws["f1"])
        ops.gemm(o["H"], W2, transB=True, bias=b2, bias_mode=cd.BIAS_COL, precision=prec,
                 out=o["Y"], workspace=ws["f2"])
        ops.gemm(dY2, W2, precision=prec, out=o["dH"], workspace=ws["h"])
        ops.gemm(dY2, o["H"], transA=True, precision=prec, out=o["gW2"], workspace=ws["w2"])
        ops.sum_reduce_rows(dY2, out=o["gb2"], workspace=ws["b2"])
        ops.activation_backward(o["dH"], o["H"], cd.EPI_RELU, out=o["dZ"])
        ops.gemm(o["dZ"], W1, precision=prec, out=o["gX"], workspace=ws["x"])
        ops.gemm(o["dZ"], X, transA=True, precision=prec, out=o["gW1"], workspace=ws["w1"])
        ops.sum_reduce_rows(o["dZ"], out=o["gb1"], workspace=ws["b1"])

    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()

    def step_forked(o):
        main = torch.cuda.current_stream()
        ops.gemm(X, W1, transB=True, bias=b1, bias_mode=cd.BIAS_COL, epilogue=cd.EPI_RELU,
                 precision=prec, out=o["H"], workspace=ws["f1"])
        ops.gemm(o["H"], W2, transB=True, bias=b2, bias_mode=cd.BIAS_COL, precision=prec,
                 out=o["Y"], workspace=ws["f2"])
        s1.wait_stream(main)
        with torch.cuda.stream(s1):
            ops.gemm(dY2, o["H"], transA=True, precision=prec, out=o["gW2"], workspace=ws["w2"])
            ops.sum_reduce_rows(dY2, out=o["gb2"], workspace=ws["b2"])
        ops.gemm(dY2, W2, precision=prec, out=o["dH"], workspace=ws["h"])
        ops.activation_backward(o["dH"], o["H"], cd.EPI_RELU, out=o["dZ"])
        s2.wait_stream(main)
        with torch.cuda.stream(s2):
            ops.gemm(o["dZ"], X, transA=True, precision=prec, out=o["gW1"], workspace=ws["w1"])
            ops.sum_reduce_rows(o["dZ"], out=o["gb1"], workspace=ws["b1"])
        ops.gemm(o["dZ"], W1, precision=prec, out=o["gX"], workspace=ws["x"])
        main.wait_stream(s1)
        main.wait_stream(s2)

    captured = step_forked if forked else step
    X.normal_(generator=g)
    dY2.normal_(generator=g)
    say("graph capture", "prec", prec, "forked", forked)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        captured(outs)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured(outs)
    torch.cuda.synchronize()
    eager = {k: torch.empty_like(v) for k, v in outs.items()}
    for r in range(4):
        X.normal_(generator=g)        # new inputs, written eagerly between replays
        dY2.normal_(generator=g)
        for v in outs.values():
            v.fill_(float("nan"))
        torch.cuda.synchronize()
        say("graph replay", r)
        graph.replay()
        torch.cuda.synchronize()
        step(eager)                   # eager step on the same inputs
        torch.cuda.synchronize()
        for k in outs:
            assert torch.equal(outs[k], eager[k]), (r, k)
        # the eager result is right, not just repeatable: fp64 closed forms
        Xd, W1d, W2d = X.double(), W1.double(), W2.double()
        Hd = torch.relu(Xd @ W1d.T + b1.double())
        dZd = (dY2.double() @ W2d) * (Hd > 0)
        gW1 = (dZd.T @ Xd).float()
        assert (eager["gW1"] - gW1).norm() <= 1e-4 * gW1.norm()
    assert np.isfinite(eager["gX"].cpu().numpy()).all()


@pytest.mark.parametrize("prec", [0, 1])
def test_conv_step_graph_capture_replays(prec):
    """A conv layer's forward (implicit route, no workspace) and backward
    (data: the flipped-filter row-window kernel, FP32 products in both
    precision modes; weight: implicit kernel with its split partials; bias) on caller
    workspaces, captured once and replayed with new inputs written eagerly
    between replays: every replay equals the eager step bit for bit, and the
    eager gradients pass fp64 checks."""
    import torch
    import torch.nn.functional as F
    ops = _ops()
    g = torch.Generator(device="cuda").manual_seed(11)
    B, C, H, W, OC = 4, 24, 20, 22, 32
    x = torch.randn((B, C, H, W), device="cuda", generator=g)
    w = torch.randn((OC, C, 3, 3), device="cuda", generator=g) * 0.1
    b = torch.randn((OC,), device="cuda", generator=g) * 0.1
    dy = torch.randn((B, OC, H, W), device="cuda", generator=g)
    st, pd = (1, 1), (1, 1)
    ws_d = torch.empty(ops.conv2d_backward_data_workspace_bytes(x.shape, w.shape, st, pd) // 4 + 1,
                       device="cuda")
    ws_w = torch.empty(ops.conv2d_backward_weight_workspace_bytes(x.shape, w.shape, st, pd) // 4 + 1,
                       device="cuda")
    outs = {"y": torch.empty((B, OC, H, W), device="cuda"), "dx": torch.empty_like(x),
            "dw": torch.empty_like(w), "db": torch.empty_like(b)}

    def step(o):
        ops.conv2d_implicit(x, w, b, st, pd, out=o["y"])
        ops.conv2d_backward_data(dy, w, x.shape, st, pd, prec, out=o["dx"], workspace=ws_d)
        ops.conv2d_backward_weight(dy, x, w.shape, st, pd, prec, out=o["dw"], workspace=ws_w)
        ops.conv2d_backward_bias(dy, out=o["db"])

    say("conv graph capture", "prec", prec)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step(outs)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step(outs)
    torch.cuda.synchronize()
    eager = {k: torch.empty_like(v) for k, v in outs.items()}
    for r in range(3):
        x.normal_(generator=g)
        dy.normal_(generator=g)
        for v in outs.values():
            v.fill_(float("nan"))
        torch.cuda.synchronize()
        say("conv graph replay", r)
        graph.replay()
        torch.cuda.synchronize()
        step(eager)
        torch.cuda.synchronize()
        for k in outs:
            assert torch.equal(outs[k], eager[k]), (r, k)
        xd, wd, dyd = x.double().cpu(), w.double().cpu(), dy.double().cpu()
        y64 = F.conv2d(xd, wd, b.double().cpu(), padding=1)
        dx64 = F.conv_transpose2d(dyd, wd, padding=1)
        dw64 = F.conv2d(xd.transpose(0, 1), dyd.transpose(0, 1), padding=1).transpose(0, 1)
        tol = 1e-5 if prec == 0 else 1e-3
        for got, want in ((eager["y"], y64), (eager["dx"], dx64), (eager["dw"], dw64)):
            got = got.double().cpu()
            assert (got - want).norm() <= tol * want.norm()
