"""The HIP path against the committed golden fixtures (tests/golden): every
pass through the C ABI (device entry points, the one-call backward and the
host-pointer entry points), within the f32 dot-product bound of the fixture
outputs; the reference's known answers exactly."""
import hashlib
import json
import os

import numpy as np
import pytest

from oracle import oracle as O
from tests.parity import assert_within

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
MANIFEST = json.load(open(os.path.join(GOLDEN, "MANIFEST.json")))
CONV = [m["file"] for m in MANIFEST["conv"]]
MM = [m["file"] for m in MANIFEST["matmul"]]


def load(fn):
    return np.load(os.path.join(GOLDEN, fn))


def _bounds(f, st, p):
    ys = O.conv2d_forward(np.abs(f["x"]), np.abs(f["w"]), st, p)
    dxs, dws = O.conv2d_backward(np.abs(f["x"]), np.abs(f["w"]), np.abs(f["g"]), st, p)
    return ys, dxs, dws


@pytest.mark.parametrize("fn", CONV)
def test_conv_fixture(fn, dev):
    import torch

    from katsu_amd import host, ops
    f = load(fn)
    st, p = int(f["stride"]), int(f["pad"])
    k, c, r, s = f["w"].shape
    n, _, oh, ow = f["g"].shape
    ys, dxs, dws = _bounds(f, st, p)
    x, w, g = (torch.from_numpy(f[a]).to(dev) for a in ("x", "w", "g"))
    y = ops.conv2d_forward(x, w, st, p)
    dx, dw = ops.conv2d_backward(x, w, g, st, p)
    dx2 = ops.conv2d_backward_data(g, w, f["x"].shape, st, p)
    dw2 = ops.conv2d_backward_filter(x, g, f["w"].shape, st, p)
    torch.cuda.synchronize()
    for got, key, sabs, kred in ((y, "y", ys, c * r * s), (dx, "dx", dxs, k * r * s),
                                 (dw, "dw", dws, n * oh * ow), (dx2, "dx", dxs, k * r * s),
                                 (dw2, "dw", dws, n * oh * ow)):
        assert_within(got.cpu().numpy(), f[key], sabs, max(1, kred), f"{fn} {key}")
    # host-pointer entry points (the drop-in seams)
    yh = host.conv2d_forward(f["x"], f["w"], st, p)
    dxh, dwh = host.conv2d_backward(f["x"], f["w"], f["g"], st, p)
    assert_within(yh, f["y"], ys, c * r * s, f"{fn} host y")
    assert_within(dxh, f["dx"], dxs, k * r * s, f"{fn} host dx")
    assert_within(dwh, f["dw"], dws, max(1, n * oh * ow), f"{fn} host dw")


@pytest.mark.parametrize("fn", MM)
def test_matmul_fixture(fn, dev):
    import torch

    from katsu_amd import ops
    f = load(fn)
    m, k = f["a"].shape
    n = f["b"].shape[1]
    a, b, g = (torch.from_numpy(f[v]).to(dev) for v in ("a", "b", "g"))
    c = ops.matmul(a, b)
    da = torch.zeros_like(a)
    db = torch.zeros_like(b)
    ops.matmul_vjp(a, b, g, da, db)
    torch.cuda.synchronize()
    A, B, G = (np.abs(f[v]).astype(np.float64) for v in ("a", "b", "g"))
    assert_within(c.cpu().numpy(), f["c"], A @ B, k, fn + " c")
    assert_within(da.cpu().numpy(), f["da"], G @ B.T, n, fn + " da")
    assert_within(db.cpu().numpy(), f["db"], A.T @ G, m, fn + " db")


def test_reference_kats_exact():
    from katsu_amd import host
    for kat in json.load(open(os.path.join(GOLDEN, "reference_kats.json"))):
        if kat["op"] == "conv2d":
            x = np.array(kat["x"]["data"], np.float32).reshape(kat["x"]["shape"])
            w = np.array(kat["w"]["data"], np.float32).reshape(kat["w"]["shape"])
            y = host.conv2d_forward(x, w, kat["stride"], kat["pad"])
            assert y.ravel().tolist() == kat["y"], kat["src"]
            if "dx" in kat:
                dx, dw = host.conv2d_backward(x, w, np.ones_like(y), kat["stride"], kat["pad"])
                assert dx.ravel().tolist() == kat["dx"], kat["src"]
                assert dw.ravel().tolist() == kat["dw"], kat["src"]
        elif kat["op"] == "matmul":
            a = np.array(kat["a"]["data"], np.float32).reshape(kat["a"]["shape"])
            b = np.array(kat["b"]["data"], np.float32).reshape(kat["b"]["shape"])
            assert host.matmul(a, b).ravel().tolist() == kat["c"], kat["src"]
        else:
            a = np.array(kat["a"]["data"], np.float32).reshape(kat["a"]["shape"])
            pend = np.zeros_like(a)
            host.matmul_vjp(a, a, np.ones_like(a), pend, pend)
            assert pend.ravel().tolist() == kat["pending_after"], kat["src"]


def test_example_1b(dev):
    """The repository example on the GPU against the oracle, whose outputs
    the fixture pins by digest."""
    from katsu_amd import host
    ex = json.load(open(os.path.join(GOLDEN, "example_1b.json")))
    x = (np.arange(3 * 224 * 224) % 256).astype(np.float32) / np.float32(255.0)
    x = x.reshape(1, 3, 224, 224)
    w = np.array(ex["w"], np.float32).reshape(8, 3, 3, 3)
    y_ref = O.conv2d_forward(x, w, 1, 1)
    dx_ref, _ = O.conv2d_backward(x, w, (y_ref + y_ref).astype(np.float32), 1, 1)
    assert hashlib.sha256(y_ref.tobytes()).hexdigest() == ex["sha256_y_f32"]
    assert hashlib.sha256(dx_ref.tobytes()).hexdigest() == ex["sha256_dx_f32"]
    y = host.conv2d_forward(x, w, 1, 1)
    ys = O.conv2d_forward(np.abs(x), np.abs(w), 1, 1)
    assert_within(y, y_ref, ys, 27, "example y")
    g = (y + y).astype(np.float32)  # the GPU's own G, as the autograd chain makes it
    dx, dw = host.conv2d_backward(x, w, g, 1, 1)
    # the backward checked on the same G (the oracle's own G differs from it
    # by the forward's rounding, which the digests above already cover)
    dx_g, dw_g = O.conv2d_backward(x, w, g, 1, 1)
    dxs, dws = O.conv2d_backward(np.abs(x), np.abs(w), np.abs(g), 1, 1)
    assert_within(dx, dx_g, dxs, 8 * 9, "example dx")
    assert_within(dw, dw_g, dws, 224 * 224, "example dw")
