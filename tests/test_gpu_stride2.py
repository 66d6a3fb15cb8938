"""Stride-2 direct kernels against the CPU oracle: the 3x3 stride-2 forward
(32-float halo rows) and the data gradient by super-pixels (a stride-1
convolution of G over 2x2 pixel blocks, then scattered back).  Shapes are
chosen so the planner takes these kernels (enough workgroups to fill the
GPU), at sizes the oracle finishes in seconds; odd input sizes exercise the
scatter's edge, where a super-pixel's second row or column lies outside."""
import numpy as np
import pytest

from katsu_amd import synth
from oracle import oracle as O
from tests.parity import assert_within, edge_samples, random_samples, sample_dx

pytestmark = pytest.mark.gpu


def _inputs(xs, ws, st, p):
    c = {"x": xs, "w": ws, "stride": st, "pad": p}
    x = synth.normal(synth.SEED_X, xs)
    w = synth.he_normal(synth.SEED_W, ws)
    g = synth.normal(synth.SEED_G, synth.out_shape(c))
    return x, w, g


@pytest.mark.parametrize("xs,ws", [((16, 8, 28, 28), (256, 8, 3, 3)),
                                   ((16, 8, 27, 29), (256, 8, 3, 3))])
def test_forward_stride2(xs, ws, dev):
    import torch

    from katsu_amd import ops
    x, w, _ = _inputs(xs, ws, 2, 1)
    y = ops.conv2d_forward(torch.from_numpy(x).to(dev), torch.from_numpy(w).to(dev), 2, 1)
    torch.cuda.synchronize()
    ref = O.conv2d_forward(x, w, 2, 1)
    sab = O.conv2d_forward(np.abs(x), np.abs(w), 2, 1)
    assert_within(y.cpu().numpy(), ref, sab, ws[1] * 9, f"fwd s2 {xs}")


@pytest.mark.parametrize("xs,ws,p", [((32, 64, 28, 28), (128, 64, 3, 3), 1),
                                     ((32, 64, 27, 27), (128, 64, 3, 3), 1),
                                     ((32, 64, 28, 28), (128, 64, 3, 3), 0)])
def test_data_gradient_superpixel_3x3(xs, ws, p, dev):
    import torch

    from katsu_amd import ops
    x, w, g = _inputs(xs, ws, 2, p)
    dx = ops.conv2d_backward_data(torch.from_numpy(g).to(dev), torch.from_numpy(w).to(dev),
                                  xs, 2, p)
    dx1 = torch.randn(xs, device=dev)
    dx1c = dx1.clone()
    ops.conv2d_backward_data(torch.from_numpy(g).to(dev), torch.from_numpy(w).to(dev), xs, 2, p,
                             out=dx1, beta=1.0)
    torch.cuda.synchronize()
    ref = O.conv2d_backward_data(xs, w, g, 2, p)
    sab = O.conv2d_backward_data(xs, np.abs(w), np.abs(g), 2, p)
    assert_within(dx.cpu().numpy(), ref, sab, ws[0] * 9, f"dX s2 {xs} p{p}")
    # beta = 1: each element is the old value plus the same sum, rounded once
    assert torch.equal(dx1, dx1c + dx)


def test_data_gradient_superpixel_stem(dev):
    """7x7 stride-2 padding-3 layer with 3 input channels (the stem's shape at
    half resolution): sampled outputs, edges and corners included, against
    exact f64 dot products."""
    import torch

    from katsu_amd import ops
    xs, ws = (64, 3, 112, 112), (64, 3, 7, 7)
    x, w, g = _inputs(xs, ws, 2, 3)
    dx = ops.conv2d_backward_data(torch.from_numpy(g).to(dev), torch.from_numpy(w).to(dev),
                                  xs, 2, 3)
    torch.cuda.synchronize()
    dx = dx.cpu().numpy()
    pts = random_samples(xs, 2000, 7) + edge_samples(xs)
    ref, sab = sample_dx(g, w, xs, 2, 3, pts)
    assert_within(np.array([dx[t] for t in pts]), ref, sab, 64 * 49, "stem dX")
