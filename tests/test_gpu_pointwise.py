"""1x1 convolutions without padding (pw_kernel) against the CPU oracle.

These layers take the pointwise GEMM path for all three passes: the forward
gathers input pixel (oy*s, ox*s), dX writes each output pixel's value at the
corner of the s x s input block it owns and zeros in the rest of the block,
and dW sums over every output pixel with a fixed split order.  With 64, 128
or 256 input channels and a block per CU the forward is register-direct
(pw_rd_fwd_kernel: operands loaded straight into MFMA registers).  Cases cover
strides 1-3 (blocks clipped at the image edge), channel counts off the 32-
and 64-wide tiles, pixel tiles that straddle images, the split dW, and
beta = 1 accumulation (the zero positions of dX are left as they were)."""
import numpy as np
import pytest

from katsu_amd import synth
from oracle import oracle as O
from tests.parity import assert_within
from tests.test_gpu_conv import _check_full

pytestmark = pytest.mark.gpu

CASES = [
    ((2, 16, 15, 15), (130, 16, 1, 1), 2),    # odd image: last row/column block clipped
    ((3, 70, 9, 11), (33, 70, 1, 1), 1),      # stride 1, channels off the tiles
    ((2, 24, 13, 10), (40, 24, 1, 1), 3),     # stride 3: 3x3 blocks, clipped
    ((1, 300, 7, 7), (20, 300, 1, 1), 1),     # reduction not a multiple of 32
    ((4, 128, 28, 28), (256, 128, 1, 1), 2),  # config 4b's layer on 4 images
    ((16, 32, 32, 32), (64, 32, 1, 1), 1),    # long pixel reduction: split dW
    ((1, 1, 1, 1), (1, 1, 1, 1), 1),
    # Register-direct forward (64, 128 or 256 input channels, a block per CU
    # at least): config 4b at full size; 64 channels with a partial output
    # channel block and pixel tiles straddling images; 256 channels at
    # stride 2 with a partial last pixel tile.
    ((32, 128, 28, 28), (256, 128, 1, 1), 2),
    ((16, 64, 30, 30), (130, 64, 1, 1), 1),
    ((24, 256, 40, 42), (70, 256, 1, 1), 2),
    # Full-size grids for the tiled backward: 40 input channels (a partial
    # 64-wide dW tile), and 256 channels onto whole stride-2 blocks.
    ((16, 40, 30, 32), (64, 40, 1, 1), 1),
    ((32, 256, 28, 28), (64, 256, 1, 1), 2),
]


@pytest.mark.parametrize("xs,ws,st", CASES)
def test_pointwise_parity(xs, ws, st, dev):
    x = synth.uniform(201, xs)
    w = synth.uniform(202, ws)
    oh = (xs[2] - 1) // st + 1
    ow = (xs[3] - 1) // st + 1
    g = synth.uniform(203, (xs[0], ws[0], oh, ow))
    _check_full(x, w, g, st, 0, dev, f"{xs}*{ws} s{st}")


@pytest.mark.parametrize("st,xs,ws", [(1, (3, 40, 11, 12), (24, 40, 1, 1)),
                                      (2, (3, 40, 11, 12), (24, 40, 1, 1)),
                                      (1, (16, 40, 30, 32), (64, 40, 1, 1)),
                                      (1, (1, 8, 4, 4), (8, 8, 1, 1))])
def test_pointwise_accumulate(st, xs, ws, dev):
    """beta = 1: dX and dW add into what the buffers hold; with stride 2 the
    input pixels no tap reaches keep their old values.  The last case has one
    dW slice, written straight into dw."""
    import torch

    from katsu_amd import ops
    x = synth.uniform(211, xs)
    w = synth.uniform(212, ws)
    oh, ow = (xs[2] - 1) // st + 1, (xs[3] - 1) // st + 1
    g = synth.uniform(213, (xs[0], ws[0], oh, ow))
    dx0 = synth.uniform(214, xs)
    dw0 = synth.uniform(215, ws)
    xd, wd, gd = (torch.from_numpy(a).to(dev) for a in (x, w, g))
    dx = torch.from_numpy(dx0.copy()).to(dev)
    dw = torch.from_numpy(dw0.copy()).to(dev)
    ops.conv2d_backward_data(gd, wd, xs, st, 0, out=dx, beta=1.0)
    ops.conv2d_backward_filter(xd, gd, ws, st, 0, out=dw, beta=1.0)
    torch.cuda.synchronize()
    dx_ref, dw_ref = O.conv2d_backward(x, w, g, st, 0)
    dxs, dws = O.conv2d_backward(np.abs(x), np.abs(w), np.abs(g), st, 0)
    # One more rounding for the final add: bound on |dx0| + |sum| terms.
    assert_within(dx.cpu().numpy(), dx0.astype(np.float64) + dx_ref, dxs + np.abs(dx0),
                  ws[0] + 1, "dX beta=1")
    assert_within(dw.cpu().numpy(), dw0.astype(np.float64) + dw_ref, dws + np.abs(dw0),
                  xs[0] * oh * ow + 1, "dW beta=1")
    if st == 2:
        odd = dx.cpu().numpy()[:, :, 1::2, :]
        assert np.array_equal(odd, dx0[:, :, 1::2, :]), "untouched rows changed"


@pytest.mark.parametrize("xs", [(2, 16, 9, 9), (2, 16, 12, 12)])
def test_pointwise_zero_fill_overwrites(xs, dev):
    """beta = 0 writes every dX element, zeros included, over stale contents:
    an odd image (scalar stores, blocks clipped) and an even one (whole 2 x 4
    blocks as 16-byte stores)."""
    import torch

    from katsu_amd import ops
    ws, st = (8, 16, 1, 1), 2
    oh, ow = (xs[2] + 1) // 2, (xs[3] + 1) // 2
    w = synth.uniform(221, ws)
    g = synth.uniform(223, (2, 8, oh, ow))
    dx = torch.full(xs, float("nan"), device=dev)
    ops.conv2d_backward_data(torch.from_numpy(g).to(dev), torch.from_numpy(w).to(dev), xs, st,
                             0, out=dx)
    torch.cuda.synchronize()
    got = dx.cpu().numpy()
    assert np.all(np.isfinite(got))
    assert np.all(got[:, :, 1::2, :] == 0) and np.all(got[:, :, :, 1::2] == 0)
    ref = O.conv2d_backward_data(xs, w, g, st, 0)
    sab = O.conv2d_backward_data(xs, np.abs(w), np.abs(g), st, 0)
    assert_within(got, ref, sab, ws[0], f"dX {xs}")
