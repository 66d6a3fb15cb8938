"""Operands over 1 GiB.

The direct convolution kernels and the dedicated GEMM address one image (or
one operand) through a buffer resource with 32-bit byte offsets, so the
planners refuse those kernels when a buffer reaches 1 GiB and the call falls
back to the generic engine, whose addresses are 64-bit; outputs are
addressed with 64-bit offsets everywhere.  These tests run past the limit:
a 3x3 convolution whose one image is 1.07 GB (the forward and dW read it on
the generic engine; dX reads the 537 MB G on the direct kernel and writes the
1.07 GB image), and a matmul whose A (and so dA) is 1.07 GB (the forward and
dB on the generic engine, dA on the dedicated GEMM with a 1.07 GB output).
Sampled outputs, edges and corners included, are compared with exact f64
dot products within the f32 bound."""
import numpy as np
import pytest

from tests.parity import (assert_within, edge_samples, random_samples, sample_dw, sample_dx,
                          sample_fwd)

pytestmark = pytest.mark.gpu

GIB = 1 << 30


def test_convolution_image_over_1gib(dev):
    import torch

    from katsu_amd import ops
    xs, ws, st, p = (1, 64, 2048, 2050), (32, 64, 3, 3), 1, 1
    assert np.prod(xs[1:]) * 4 >= GIB
    rng = np.random.default_rng(71)
    x = rng.standard_normal(xs, dtype=np.float32)
    w = rng.standard_normal(ws, dtype=np.float32) * np.float32(1 / 24)
    gs = (1, ws[0], xs[2], xs[3])
    g = rng.standard_normal(gs, dtype=np.float32)
    xd, wd, gd = (torch.from_numpy(t).to(dev) for t in (x, w, g))
    y = ops.conv2d_forward(xd, wd, st, p).cpu().numpy()
    dx = ops.conv2d_backward_data(gd, wd, xs, st, p).cpu().numpy()
    dw = ops.conv2d_backward_filter(xd, gd, ws, st, p).cpu().numpy()
    # The one-call backward runs the same plans: the same bits.
    bdx, bdw = ops.conv2d_backward(xd, wd, gd, st, p)
    assert np.array_equal(bdx.cpu().numpy(), dx) and np.array_equal(bdw.cpu().numpy(), dw)
    del xd, gd, bdx, bdw
    k, c, r, s = ws
    pts = random_samples(gs, 200, 1) + edge_samples(gs)
    ref, sab = sample_fwd(x, w, st, p, pts)
    assert_within(np.array([y[t] for t in pts]), ref, sab, c * r * s, "fwd > 1 GiB")
    pts = random_samples(xs, 200, 2) + edge_samples(xs)
    ref, sab = sample_dx(g, w, xs, st, p, pts)
    assert_within(np.array([dx[t] for t in pts]), ref, sab, k * r * s, "dX > 1 GiB")
    pts = random_samples(ws, 24, 3) + [(0, 0, 0, 0), (k - 1, c - 1, r - 1, s - 1)]
    ref, sab = sample_dw(x, g, ws, st, p, pts)
    assert_within(np.array([dw[t] for t in pts]), ref, sab, xs[2] * xs[3], "dW > 1 GiB")


def test_matmul_operand_over_1gib(dev):
    import torch

    from katsu_amd import ops
    m, k, n = 16384, 16400, 256
    assert m * k * 4 >= GIB
    rng = np.random.default_rng(72)
    a = rng.standard_normal((m, k), dtype=np.float32)
    b = rng.standard_normal((k, n), dtype=np.float32)
    g = rng.standard_normal((m, n), dtype=np.float32)
    ad, bd, gd = (torch.from_numpy(t).to(dev) for t in (a, b, g))
    c = ops.matmul(ad, bd).cpu().numpy()
    da = torch.zeros((m, k), device=dev)
    db = torch.zeros((k, n), device=dev)
    ops.matmul_vjp(ad, bd, gd, da, db)
    da, db = da.cpu().numpy(), db.cpu().numpy()
    a64, b64, g64 = a.astype(np.float64), b.astype(np.float64), g.astype(np.float64)

    def check(got, rows, cols, kred, what, seed):
        pts = random_samples(got.shape, 200, seed)
        pts += [(0, 0), (0, got.shape[1] - 1), (got.shape[0] - 1, 0),
                (got.shape[0] - 1, got.shape[1] - 1)]
        ref = np.array([np.dot(rows(i), cols(j)) for i, j in pts])
        sab = np.array([np.dot(np.abs(rows(i)), np.abs(cols(j))) for i, j in pts])
        assert_within(np.array([got[t] for t in pts]), ref, sab, kred, what)

    check(c, lambda i: a64[i], lambda j: b64[:, j], k, "C = A B", 4)
    check(da, lambda i: g64[i], lambda j: b64[j], n, "dA = G B^T", 5)
    check(db, lambda i: a64[:, i], lambda j: g64[:, j], m, "dB = A^T G", 6)
