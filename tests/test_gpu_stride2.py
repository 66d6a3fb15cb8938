"""Stride-2 direct kernels against the CPU oracle.

Forward: the 3x3 stride-2 kernel (32-float halo rows split by column
parity), and on rows of at most 16 output pixels the row-fragment tiles;
cases cover 14- and 15-pixel rows and input channel counts with and without
16-byte weight rows.  Data gradient: a 3x3, padding-1 layer with at least 16
input channels takes the phase form (every MFMA a real tap, all four output
phases of a channel block in one block); other stride-2 layers take the
super-pixel form (a stride-1 convolution of G over 2x2 pixel blocks, then
scattered back), except the stem's own channel counts (3 in, 64 out), which
take the rolling-row kernel (each output row summed over its four G rows in
the accumulators).  Phase-form cases cover odd image sizes (a super-pixel's
second row or column outside the image), channel counts off the 16-channel
blocks and stages, rows of exactly 16 super-pixels, tiles of 5 rows with a
short last tile, and beta = 1.  Shapes are chosen so the planner takes these
kernels (enough workgroups to fill the GPU), at sizes the oracle finishes in
seconds."""
import numpy as np
import pytest

from katsu_amd import synth
from oracle import oracle as O
from tests.parity import assert_within, edge_samples, random_samples, sample_dx
from tests.test_gpu_conv import _check_full

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
def test_data_gradient_3x3(xs, ws, p, dev):
    """Padding 1 takes the phase form, padding 0 the super-pixel form."""
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


def test_data_gradient_stem_half_resolution(dev):
    """7x7 stride-2 padding-3 layer with 3 input channels (the stem's shape at
    half resolution, rolling-row kernel): sampled outputs, edges and corners
    included, against exact f64 dot products."""
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


DX_CASES = [
    ((32, 64, 28, 28), (32, 64, 3, 3)),   # 14 x 14 super-pixels, 7-row tiles
    ((32, 40, 27, 25), (24, 40, 3, 3)),   # odd sizes; 3 channel blocks; 5-row tiles
    ((64, 64, 9, 31), (33, 64, 3, 3)),    # 16-wide super rows; a 1-channel last stage
]


@pytest.mark.parametrize("xs,ws", DX_CASES)
def test_stride2_data_gradient_phases(xs, ws, dev):
    import torch

    from katsu_amd import ops
    x = synth.uniform(301, xs)
    w = synth.uniform(302, ws)
    oh, ow = (xs[2] - 1) // 2 + 1, (xs[3] - 1) // 2 + 1
    g = synth.uniform(303, (xs[0], ws[0], oh, ow))
    wd, gd = torch.from_numpy(w).to(dev), torch.from_numpy(g).to(dev)
    dx = ops.conv2d_backward_data(gd, wd, xs, 2, 1)
    torch.cuda.synchronize()
    dx_ref = O.conv2d_backward_data(xs, w, g, 2, 1)
    dxs = O.conv2d_backward_data(xs, np.abs(w), np.abs(g), 2, 1)
    assert_within(dx.cpu().numpy(), dx_ref, dxs, ws[0] * 9, f"{xs}*{ws} dX")


def test_stride2_data_gradient_accumulates(dev):
    """beta = 1 adds the gradient to what dX holds, in every phase."""
    import torch

    from katsu_amd import ops
    xs, ws = DX_CASES[1]
    w = synth.uniform(311, ws)
    g = synth.uniform(313, (xs[0], ws[0], 14, 13))
    dx0 = synth.uniform(314, xs)
    dx = torch.from_numpy(dx0.copy()).to(dev)
    ops.conv2d_backward_data(torch.from_numpy(g).to(dev), torch.from_numpy(w).to(dev), xs, 2, 1,
                             out=dx, beta=1.0)
    torch.cuda.synchronize()
    dx_ref = O.conv2d_backward_data(xs, w, g, 2, 1)
    dxs = O.conv2d_backward_data(xs, np.abs(w), np.abs(g), 2, 1)
    assert_within(dx.cpu().numpy(), dx0.astype(np.float64) + dx_ref, dxs + np.abs(dx0),
                  ws[0] * 9 + 1, "dX beta=1")


FWD_CASES = [
    ((64, 16, 28, 28), (128, 16, 3, 3)),  # 14-pixel rows, 7-row tiles
    ((64, 20, 27, 29), (100, 20, 3, 3)),  # 15-pixel rows; a partial channel block
    ((64, 22, 28, 30), (96, 22, 3, 3)),   # 22 channels: 4-byte weight loads
    ((64, 40, 28, 28), (64, 40, 3, 3)),   # three 16-channel stages; 4-row tiles
]


@pytest.mark.parametrize("xs,ws", FWD_CASES)
def test_stride2_small_image_all_passes(xs, ws, dev):
    x = synth.uniform(321, xs)
    w = synth.uniform(322, ws)
    oh, ow = (xs[2] - 1) // 2 + 1, (xs[3] - 1) // 2 + 1
    g = synth.uniform(323, (xs[0], ws[0], oh, ow))
    _check_full(x, w, g, 2, 1, dev, f"{xs}*{ws} s2")


# 7x7 stride-2 padding-3 data gradient of layers with at most 4 input
# channels (stem-like), full oracle comparison: odd sizes clip the last
# super-pixel's second row and column, an odd K, C = 1 and C = 4, beta = 1.
STEM_DX_CASES = [
    ((32, 3, 99, 101), (25, 3, 7, 7)),
    ((64, 4, 64, 72), (16, 4, 7, 7)),
    ((20, 1, 224, 60), (8, 1, 7, 7)),
    # The stem's own channels (3 in, 64 out: the rolling-row kernel): bands
    # of 2 and 4 flattened super-rows whose segments start and end at image
    # edges and inside images, a clipped last row, a clipped last column,
    # bands of one row on small maps, a partial column tile, a 1 x 1 map.
    ((2, 3, 224, 224), (64, 3, 7, 7)),
    ((5, 3, 223, 224), (64, 3, 7, 7)),
    ((3, 3, 224, 223), (64, 3, 7, 7)),
    ((7, 3, 20, 36), (64, 3, 7, 7)),
    ((3, 3, 223, 35), (64, 3, 7, 7)),
    ((2, 3, 9, 9), (64, 3, 7, 7)),
    ((2, 3, 2, 1), (64, 3, 7, 7)),
]


@pytest.mark.parametrize("xs,ws", STEM_DX_CASES)
def test_stem_data_gradient(xs, ws, dev):
    import torch

    from katsu_amd import ops
    w = synth.uniform(331, ws)
    oh, ow = (xs[2] - 1) // 2 + 1, (xs[3] - 1) // 2 + 1
    g = synth.uniform(333, (xs[0], ws[0], oh, ow))
    wd, gd = torch.from_numpy(w).to(dev), torch.from_numpy(g).to(dev)
    dx = ops.conv2d_backward_data(gd, wd, xs, 2, 3)
    dx0 = synth.uniform(334, xs)
    dx1 = torch.from_numpy(dx0.copy()).to(dev)
    ops.conv2d_backward_data(gd, wd, xs, 2, 3, out=dx1, beta=1.0)
    torch.cuda.synchronize()
    ref = O.conv2d_backward_data(xs, w, g, 2, 3)
    sab = O.conv2d_backward_data(xs, np.abs(w), np.abs(g), 2, 3)
    assert_within(dx.cpu().numpy(), ref, sab, ws[0] * 49, f"stem dX {xs}*{ws}")
    assert_within(dx1.cpu().numpy(), dx0.astype(np.float64) + ref, sab + np.abs(dx0),
                  ws[0] * 49 + 1, f"stem dX beta=1 {xs}*{ws}")


def test_stem_full_size_sampled_rows(dev):
    """The stem's dX at its full size (64 images of 224 x 224): every row of
    three images (so every band and image boundary of a kernel that works in
    bands of rows), sampled against exact f64 dot products at the first,
    middle and last columns of each 16-column tile edge and all channels;
    the result is the same bit for bit on every call."""
    import torch

    from katsu_amd import ops
    from tests.parity import sample_dx
    c = synth.CONV_CONFIGS["c5_stem"]
    xs, ws = c["x"], c["w"]
    w = synth.he_normal(synth.SEED_W, ws)
    g = synth.normal(synth.SEED_G, synth.out_shape(c))
    wd, gd = torch.from_numpy(w).to(dev), torch.from_numpy(g).to(dev)
    dx = ops.conv2d_backward_data(gd, wd, xs, 2, 3)
    again = ops.conv2d_backward_data(gd, wd, xs, 2, 3)
    torch.cuda.synchronize()
    assert torch.equal(dx, again), "stem dX differs between calls"
    rows = range(xs[2])
    pts = [(n, ch, iy, ix) for n in (0, 17, 63) for ch in range(3) for iy in rows
           for ix in (0, 1, 31, 32, 111, 112, 191, 192, 222, 223)]
    ref, sab = sample_dx(g, w, xs, 2, 3, pts)
    dxh = dx.cpu().numpy()
    assert_within(np.array([dxh[t] for t in pts]), ref, sab, 64 * 49, "stem dX strip rows")
