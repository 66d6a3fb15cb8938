"""The one-call backward (katsu_hip_conv2d_bwd_f32[_dev]) against the two
separate passes.  Where dX and dW share one launch the kernels and their
summation order are those of the separate launches, so the results must be
identical bit for bit; shapes the fused launch does not take (stride 2,
small channel counts, other filter sizes) go through the separate passes and
must match them too.  beta = 1 accumulates into both outputs."""
import numpy as np
import pytest

from katsu_amd import synth
from oracle import oracle as O
from tests.parity import assert_within

pytestmark = pytest.mark.gpu

CASES = [
    ((32, 64, 56, 56), (64, 64, 3, 3), 1, 1),   # config 3: fused launch
    ((32, 64, 30, 30), (64, 64, 3, 3), 1, 1),   # fused, rows not a multiple of 4 (masked dW)
    ((32, 80, 28, 28), (96, 80, 3, 3), 1, 1),   # fused, channel counts off the tiles
    ((2, 80, 17, 9), (96, 80, 3, 3), 1, 0),     # too few blocks to fuse: separate passes
    ((4, 128, 28, 28), (256, 128, 3, 3), 2, 1),  # stride 2: separate passes
    ((2, 3, 40, 40), (64, 3, 7, 7), 2, 3),      # stem-like: separate passes
    ((2, 16, 12, 12), (8, 16, 1, 1), 1, 0),     # 1x1: separate passes
]


def _tensors(xs, ws, st, p, dev):
    import torch
    c = {"x": xs, "w": ws, "stride": st, "pad": p}
    x = synth.uniform(synth.SEED_X, xs, -1.0, 1.0)
    w = synth.normal(synth.SEED_W, ws)
    g = synth.normal(synth.SEED_G, synth.out_shape(c))
    return [torch.from_numpy(a).to(dev) for a in (x, w, g)]


@pytest.mark.parametrize("xs,ws,st,p", CASES)
def test_fused_matches_separate(xs, ws, st, p, dev):
    import torch

    from katsu_amd import ops
    x, w, g = _tensors(xs, ws, st, p, dev)
    for beta in (0.0, 1.0):
        dx0 = torch.randn(x.shape, device=dev) if beta else None
        dw0 = torch.randn(w.shape, device=dev) if beta else None
        dx_s = ops.conv2d_backward_data(g, w, x.shape, st, p,
                                        out=None if dx0 is None else dx0.clone(), beta=beta)
        dw_s = ops.conv2d_backward_filter(x, g, w.shape, st, p,
                                          out=None if dw0 is None else dw0.clone(), beta=beta)
        dx_f, dw_f = ops.conv2d_backward(x, w, g, st, p,
                                         dx=None if dx0 is None else dx0.clone(),
                                         dw=None if dw0 is None else dw0.clone(), beta=beta)
        torch.cuda.synchronize()
        assert torch.equal(dx_f, dx_s), f"dX beta={beta}"
        assert torch.equal(dw_f, dw_s), f"dW beta={beta}"


def test_fused_caller_workspace_and_graph_replay(dev):
    import torch

    from katsu_amd import ops
    xs, ws, st, p = (8, 64, 56, 56), (64, 64, 3, 3), 1, 1
    x, w, g = _tensors(xs, ws, st, p, dev)
    nbytes = ops.bwd_filter_workspace_bytes(xs, ws, st, p)
    work = torch.empty(max(1, nbytes), device=dev, dtype=torch.uint8)
    dx = torch.empty_like(x)
    dw = torch.empty_like(w)
    ops.conv2d_backward(x, w, g, st, p, dx=dx, dw=dw, workspace=work)
    torch.cuda.synchronize()
    ref = (dx.clone(), dw.clone())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        ops.conv2d_backward(x, w, g, st, p, dx=dx, dw=dw, workspace=work)
    for _ in range(3):
        dx.fill_(float("nan"))
        dw.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(dx, ref[0]) and torch.equal(dw, ref[1])


def test_fused_host_entry_against_oracle():
    """The host-pointer form (what katsu-core's backward_buffers would call)
    against the CPU oracle."""
    from katsu_amd import host
    xs, ws, st, p = (2, 64, 14, 14), (64, 64, 3, 3), 1, 1
    c = {"x": xs, "w": ws, "stride": st, "pad": p}
    x = synth.uniform(synth.SEED_X, xs, -1.0, 1.0)
    w = synth.normal(synth.SEED_W, ws)
    g = synth.normal(synth.SEED_G, synth.out_shape(c))
    dx, dw = host.conv2d_backward(x, w, g, st, p)
    dx_ref, dw_ref = O.conv2d_backward(x, w, g, st, p)
    dxs, dws = O.conv2d_backward(np.abs(x), np.abs(w), np.abs(g), st, p)
    assert_within(dx, dx_ref, dxs, 64 * 9, "fused host dX")
    assert_within(dw, dw_ref, dws, 2 * 14 * 14, "fused host dW")
