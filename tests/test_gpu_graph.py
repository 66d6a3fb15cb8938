"""HIP-graph capture of the path (how bench.py times it): every replay must
reproduce the eager result bit for bit.  Replays are separated by eager work
and synchronisations, and each one is checked."""
import numpy as np
import pytest

from katsu_amd import synth

pytestmark = pytest.mark.gpu


def _capture(fn):
    import torch
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    return g


@pytest.mark.parametrize("name,batch", [("c3_resnet", 4), ("c4a_down3x3", 2), ("c1_example", 1)])
def test_conv_step_graph_replays(name, batch, dev):
    import torch

    from katsu_amd import ops
    c = dict(synth.CONV_CONFIGS[name])
    c["x"] = (batch,) + c["x"][1:]
    x, w = synth.conv_inputs(c)
    st, p = c["stride"], c["pad"]
    g = synth.normal(synth.SEED_G, synth.out_shape(c))
    xd, wd, gd = (torch.from_numpy(a).to(dev) for a in (x, w, g))
    y = torch.empty(synth.out_shape(c), device=dev)
    dx = torch.empty_like(xd)
    dw = torch.empty_like(wd)
    ws = torch.empty(max(1, ops.bwd_filter_workspace_bytes(x.shape, w.shape, st, p)),
                     device=dev, dtype=torch.uint8)

    def step():
        ops.conv2d_forward(xd, wd, st, p, out=y)
        ops.conv2d_backward_data(gd, wd, x.shape, st, p, out=dx)
        ops.conv2d_backward_filter(xd, gd, w.shape, st, p, out=dw, workspace=ws)

    step()
    torch.cuda.synchronize()
    ref = (y.clone(), dx.clone(), dw.clone())
    graph = _capture(step)
    for _ in range(3):
        for t in (y, dx, dw):
            t.fill_(float("nan"))  # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for got, want in zip((y, dx, dw), ref):
            assert torch.equal(got, want)


@pytest.mark.parametrize("name,batch", [("c4b_down1x1", 32), ("c5_stem", 2)])
def test_one_call_backward_graph_replays(name, batch, dev):
    """The forward and the one-call backward of the 1x1 layer at full size
    (register-direct forward; dX and dW in one launch with two k-tiles of
    buffer loads in flight, non-temporal dX stores; the dW reduce) and of the
    stem (flat-reduction forward; rolling-row dX, dW and reduce)."""
    import torch

    from katsu_amd import ops
    c = dict(synth.CONV_CONFIGS[name])
    c["x"] = (batch,) + c["x"][1:]
    x, w = synth.conv_inputs(c)
    st, p = c["stride"], c["pad"]
    g = synth.normal(synth.SEED_G, synth.out_shape(c))
    xd, wd, gd = (torch.from_numpy(a).to(dev) for a in (x, w, g))
    y = torch.empty(synth.out_shape(c), device=dev)
    dx = torch.empty_like(xd)
    dw = torch.empty_like(wd)

    def step():
        ops.conv2d_forward(xd, wd, st, p, out=y)
        ops.conv2d_backward(xd, wd, gd, st, p, dx=dx, dw=dw)

    step()
    torch.cuda.synchronize()
    ref = (y.clone(), dx.clone(), dw.clone())
    graph = _capture(step)
    for _ in range(3):
        for t in (y, dx, dw):
            t.fill_(float("nan"))  # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for got, want in zip((y, dx, dw), ref):
            assert torch.equal(got, want)


def test_matmul_vjp_graph_replays(dev):
    import torch

    from katsu_amd import ops
    m, k, n = 300, 200, 260
    a = torch.from_numpy(synth.uniform(1, (m, k))).to(dev)
    b = torch.from_numpy(synth.uniform(2, (k, n))).to(dev)
    g = torch.from_numpy(synth.uniform(3, (m, n))).to(dev)
    c = torch.empty((m, n), device=dev)
    da = torch.zeros_like(a)
    db = torch.zeros_like(b)

    def mstep():
        ops.gemm(a, b, m, n, k, out=c)
        ops.matmul_vjp(a, b, g, da, db)

    mstep()
    torch.cuda.synchronize()
    ref = (c.clone(), da.clone(), db.clone())
    graph = _capture(mstep)
    for _ in range(3):
        c.fill_(float("nan"))
        da.zero_()
        db.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for got, want in zip((c, da, db), ref):
            assert torch.equal(got, want)
    assert np.isfinite(c.cpu().numpy()).all()
