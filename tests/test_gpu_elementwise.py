"""The device engine's elementwise kernels through the C ABI: the ops whose
reference loops are one rounding per element (add, mul, the VJP
accumulations, fill, the scalar broadcast) must match numpy's f32 results
bit for bit, aligned or not, with and without a ragged tail; the reductions
(sum, row mean) must lie within the f32 summation bound of an exact f64 sum
and be identical run to run."""
import numpy as np
import pytest

from katsu_amd import synth
from tests.parity import gamma

pytestmark = pytest.mark.gpu

SIZES = [0, 1, 3, 4, 5, 1000, 4099, 1 << 20]


def _vec(seed, n):
    return synth.uniform(seed, (n,)) if n else np.zeros(0, np.float32)


@pytest.mark.parametrize("n", SIZES)
@pytest.mark.parametrize("offset", [0, 1])
def test_binary_and_accumulate_exact(n, offset, dev):
    import torch

    from katsu_amd import ops
    a = _vec(1, n + offset)
    b = _vec(2, n + offset)
    c0 = _vec(3, n + offset)
    ta, tb, tc = (torch.from_numpy(v).to(dev)[offset:] for v in (a, b, c0))  # offset 1: unaligned
    a, b, c0 = a[offset:], b[offset:], c0[offset:]
    assert np.array_equal(ops.add(ta, tb).cpu().numpy(), a + b)
    assert np.array_equal(ops.mul(ta, tb).cpu().numpy(), a * b)
    out = tc.clone()
    ops.mul(ta, tb, out=out, beta=1.0)
    assert np.array_equal(out.cpu().numpy(), c0 + a * b)
    out = tc.clone()
    ops.add(ta, tb, out=out, beta=1.0)
    assert np.array_equal(out.cpu().numpy(), c0 + (a + b))
    out = tc.clone()
    ops.accumulate(ta, out)
    assert np.array_equal(out.cpu().numpy(), c0 + a)
    ops.accumulate(ta, out, beta=0.0)
    assert np.array_equal(out.cpu().numpy(), a)
    out = tc.clone()
    ops.fill(out, 0.0)
    assert not out.any()
    s = torch.tensor([0.25], device=dev)
    out = tc.clone()
    ops.add_scalar(s, out)
    assert np.array_equal(out.cpu().numpy(), c0 + np.float32(0.25))
    ops.add_scalar(s, out, beta=0.0)
    assert np.array_equal(out.cpu().numpy(), np.full(n, 0.25, np.float32))


@pytest.mark.parametrize("n", [0, 1, 7, 4096, 4097, 1 << 20, 25690112])
def test_sum_within_bound_and_deterministic(n, dev):
    import torch

    from katsu_amd import ops
    x = _vec(5, n)
    tx = torch.from_numpy(x).to(dev)
    got = ops.sum(tx).item()
    again = ops.sum(tx).item()
    assert got == again
    exact = float(np.sum(x.astype(np.float64)))
    # The library's tree: chunks of max(4096, n/1024) elements per block, 256
    # strided sequential sums per chunk, a 256-lane tree, then the same over
    # the chunk sums; its longest chain of additions bounds the error.
    chunk = max(4096, -(-n // 1024))
    parts = max(1, -(-n // chunk))
    depth = -(-chunk // 256) + 8 + -(-parts // 256) + 8
    bound = gamma(depth) * float(np.sum(np.abs(x.astype(np.float64))))
    assert abs(got - exact) <= bound
    out = torch.tensor([1.5], device=dev)
    ops.sum(tx, out=out, beta=1.0)
    assert abs(out.item() - (1.5 + exact)) <= bound + 2 ** -23 * (1.5 + abs(exact))


def test_mean_rows_and_broadcast(dev):
    import torch

    from katsu_amd import ops
    rows, cols = 4096, 12544 // 16
    y = synth.uniform(7, (rows, cols))
    ty = torch.from_numpy(y).to(dev)
    m = ops.mean_rows(ty, rows, cols).cpu().numpy()
    exact = y.astype(np.float64).sum(1) / cols
    bound = 2 * gamma(cols) * np.abs(y.astype(np.float64)).sum(1) / cols + np.abs(exact) * 2 ** -23
    assert np.all(np.abs(m - exact) <= bound)
    g = synth.uniform(8, (rows,))
    dy = ops.broadcast_rows(torch.from_numpy(g).to(dev), rows, cols, 1.0 / cols).cpu().numpy()
    assert np.array_equal(dy.reshape(rows, cols), np.repeat((g * np.float32(1.0 / cols))[:, None],
                                                            cols, 1))


def test_grad_cam(dev):
    """katsu_hip_gradcam_f32_dev against the formula in float64: channel
    weights = spatial means of the gradient, ReLU of the weighted channel sum,
    each map divided by its maximum; an all-negative map stays zero."""
    import torch

    from katsu_amd import ops
    n, c, h, w = 3, 16, 14, 15
    act = synth.uniform(11, (n, c, h, w))
    grad = synth.uniform(12, (n, c, h, w))
    act[2] = -np.abs(act[2])
    grad[2] = np.abs(grad[2])  # image 2: every weighted sum negative
    cam = ops.grad_cam(torch.from_numpy(act).to(dev), torch.from_numpy(grad).to(dev)).cpu().numpy()
    a64, g64 = act.astype(np.float64), grad.astype(np.float64)
    alpha = g64.reshape(n, c, -1).mean(2)
    ref = np.maximum(np.einsum("nc,nchw->nhw", alpha, a64), 0.0)
    mx = ref.reshape(n, -1).max(1)
    ref = np.where(mx[:, None, None] > 0, ref / np.where(mx > 0, mx, 1)[:, None, None], 0.0)
    assert np.all(cam[2] == 0.0)
    assert np.max(np.abs(cam - ref)) <= 1e-5


@pytest.mark.parametrize("src,dst", [((14, 15), (28, 30)), ((112, 112), (224, 224)),
                                     ((14, 15), (7, 4)), ((6, 5), (6, 5)), ((1, 3), (5, 9))])
def test_resize_bilinear(dev, src, dst):
    """katsu_hip_resize_bilinear_f32_dev (Grad-CAM's resize to the input image)
    against torch's CPU bilinear interpolation in float64 with half-pixel
    centres (align_corners=False), an independent implementation of the same
    formula; equal sizes copy bit for bit."""
    import torch
    import torch.nn.functional as F

    from katsu_amd import ops
    n = 3
    maps = np.abs(synth.uniform(21, (n, *src)))
    got = ops.resize_bilinear(torch.from_numpy(maps).to(dev), dst).cpu().numpy()
    ref = F.interpolate(torch.from_numpy(maps.astype(np.float64))[:, None], size=dst,
                        mode="bilinear", align_corners=False)[:, 0].numpy()
    assert got.shape == (n, *dst)
    assert np.max(np.abs(got - ref)) <= 2e-7
    assert np.array_equal(got, _resize_f32(maps, dst))
    if src == dst:
        assert np.array_equal(got, maps)


def _resize_f32(maps, size):
    """The kernel's formula evaluated in float32 by numpy, rounding as written:
    per blend (1 - f)*a + f*b, a weight of exactly 0 leaving its neighbour
    out; equal sizes copy."""
    n, ih, iw = maps.shape
    oh, ow = size
    if (ih, iw) == (oh, ow):
        return maps.copy()
    f32 = np.float32

    def axis(o, i):
        s = np.maximum((np.arange(o, dtype=f32) + f32(0.5)) * (f32(i) / f32(o)) - f32(0.5), f32(0))
        lo = np.minimum(s.astype(np.int64), i - 1)
        hi = np.minimum(lo + 1, i - 1)
        return lo, hi, np.minimum(s - lo.astype(f32), f32(1))

    def blend(a, b, f):
        with np.errstate(invalid="ignore", over="ignore"):
            mix = (f32(1) - f) * a + f * b
        return np.where(f == 0, a, np.where(f == 1, b, mix)).astype(f32)

    y0, y1, fy = axis(oh, ih)
    x0, x1, fx = axis(ow, iw)
    top = blend(maps[:, y0][:, :, x0], maps[:, y0][:, :, x1], fx[None, None, :])
    bot = blend(maps[:, y1][:, :, x0], maps[:, y1][:, :, x1], fx[None, None, :])
    return blend(top, bot, fy[None, :, None])


@pytest.mark.parametrize("src,dst", [((7, 9), (14, 18)), ((7, 9), (7, 9)), ((5, 6), (11, 4))])
def test_resize_bilinear_nonfinite(dev, src, dst):
    """Inf and NaN pixels: an equal-size resize copies them; otherwise they
    reach only the outputs whose blend gives them a non-zero weight (the
    float32 formula's masks and values, exactly)."""
    import torch

    from katsu_amd import ops
    maps = np.abs(synth.uniform(22, (2, *src)))
    maps[0, 0, 0] = np.inf
    maps[1, src[0] // 2, src[1] - 1] = np.nan
    maps[1, src[0] - 1, 1] = -np.inf
    got = ops.resize_bilinear(torch.from_numpy(maps).to(dev), dst).cpu().numpy()
    ref = _resize_f32(maps, dst)
    assert np.isfinite(ref).any() and not np.isfinite(ref).all()
    assert np.array_equal(got, ref, equal_nan=True)


def test_grad_cam_resized(dev):
    """Grad-CAM with the resize: the unresized maps, then resized, equal the
    maps computed with size= in one call; and the resized maps are within
    1e-5 of the float64 formula followed by torch's float64 bilinear resize."""
    import torch
    import torch.nn.functional as F

    from katsu_amd import ops
    n, c, h, w = 2, 8, 7, 9
    act = synth.uniform(31, (n, c, h, w))
    grad = synth.uniform(32, (n, c, h, w))
    a, g = torch.from_numpy(act).to(dev), torch.from_numpy(grad).to(dev)
    small = ops.grad_cam(a, g)
    big = ops.grad_cam(a, g, size=(14, 18)).cpu().numpy()
    assert np.array_equal(big, ops.resize_bilinear(small, (14, 18)).cpu().numpy())
    a64, g64 = act.astype(np.float64), grad.astype(np.float64)
    alpha = g64.reshape(n, c, -1).mean(2)
    ref = np.maximum(np.einsum("nc,nchw->nhw", alpha, a64), 0.0)
    mx = ref.reshape(n, -1).max(1)
    ref = np.where(mx[:, None, None] > 0, ref / np.where(mx > 0, mx, 1)[:, None, None], 0.0)
    ref = F.interpolate(torch.from_numpy(ref)[:, None], size=(14, 18), mode="bilinear",
                        align_corners=False)[:, 0].numpy()
    assert np.max(np.abs(big - ref)) <= 1e-5

