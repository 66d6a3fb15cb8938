"""The committed golden fixtures (tests/golden, written by make_golden.py)
against the CPU oracle, CPU only: the oracle must reproduce every fixture
bit for bit, the fixtures must stay within the f32 dot-product bound of an
independent float64 evaluation, and the reference's known answers must hold
exactly."""
import hashlib
import json
import os

import numpy as np
import pytest

from oracle import oracle as O
from tests.parity import assert_within

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
MANIFEST = json.load(open(os.path.join(GOLDEN, "MANIFEST.json")))
CONV = [m["file"] for m in MANIFEST["conv"]]
MM = [m["file"] for m in MANIFEST["matmul"]]


def load(fn):
    return np.load(os.path.join(GOLDEN, fn))  # allow_pickle=False (numpy default)


def test_manifest_digests():
    for fn, digest in MANIFEST["sha256"].items():
        assert hashlib.sha256(open(os.path.join(GOLDEN, fn), "rb").read()).hexdigest() == digest, fn


@pytest.mark.parametrize("fn", CONV)
def test_oracle_reproduces_conv_fixture(fn):
    f = load(fn)
    st, p = int(f["stride"]), int(f["pad"])
    y = O.conv2d_forward(f["x"], f["w"], st, p)
    dx, dw = O.conv2d_backward(f["x"], f["w"], f["g"], st, p)
    assert np.array_equal(y, f["y"]) and np.array_equal(dx, f["dx"]) and np.array_equal(dw, f["dw"])
    # the split passes are bit-identical to the one-visit backward
    assert np.array_equal(O.conv2d_backward_data(f["x"].shape, f["w"], f["g"], st, p), f["dx"])
    assert np.array_equal(O.conv2d_backward_filter(f["x"], f["w"].shape, f["g"], st, p), f["dw"])


@pytest.mark.parametrize("fn", CONV)
def test_conv_fixture_against_f64(fn):
    import torch
    f = load(fn)
    st, p = int(f["stride"]), int(f["pad"])
    x, w, g = (torch.from_numpy(f[k]).double() for k in ("x", "w", "g"))
    ax, aw, ag = x.abs(), w.abs(), g.abs()
    k, c, r, s = f["w"].shape
    n, _, oh, ow = f["g"].shape
    conv = torch.nn.functional.conv2d
    gi, gw = torch.nn.grad.conv2d_input, torch.nn.grad.conv2d_weight
    assert_within(f["y"], conv(x, w, stride=st, padding=p).numpy(),
                  conv(ax, aw, stride=st, padding=p).numpy(), c * r * s, fn + " y")
    assert_within(f["dx"], gi(x.shape, w, g, stride=st, padding=p).numpy(),
                  gi(x.shape, aw, ag, stride=st, padding=p).numpy(), k * r * s, fn + " dx")
    assert_within(f["dw"], gw(x, w.shape, g, stride=st, padding=p).numpy(),
                  gw(ax, w.shape, ag, stride=st, padding=p).numpy(), max(1, n * oh * ow),
                  fn + " dw")


@pytest.mark.parametrize("fn", MM)
def test_oracle_reproduces_matmul_fixture(fn):
    f = load(fn)
    assert np.array_equal(O.matmul(f["a"], f["b"]), f["c"])
    da, db = O.matmul_vjp(f["a"], f["b"], f["g"])
    assert np.array_equal(da, f["da"]) and np.array_equal(db, f["db"])
    a, b, g = (f[k].astype(np.float64) for k in ("a", "b", "g"))
    m, k = a.shape
    n = b.shape[1]
    assert_within(f["c"], a @ b, np.abs(a) @ np.abs(b), k, fn + " c")
    assert_within(f["da"], g @ b.T, np.abs(g) @ np.abs(b).T, n, fn + " da")
    assert_within(f["db"], a.T @ g, np.abs(a).T @ np.abs(g), m, fn + " db")


def test_reference_kats():
    for kat in json.load(open(os.path.join(GOLDEN, "reference_kats.json"))):
        if kat["op"] == "conv2d":
            x = np.array(kat["x"]["data"], np.float32).reshape(kat["x"]["shape"])
            w = np.array(kat["w"]["data"], np.float32).reshape(kat["w"]["shape"])
            y = O.conv2d_forward(x, w, kat["stride"], kat["pad"])
            assert y.ravel().tolist() == kat["y"], kat["src"]
            if "dx" in kat:
                dx, dw = O.conv2d_backward(x, w, np.ones_like(y), kat["stride"], kat["pad"])
                assert dx.ravel().tolist() == kat["dx"], kat["src"]
                assert dw.ravel().tolist() == kat["dw"], kat["src"]
        elif kat["op"] == "matmul":
            a = np.array(kat["a"]["data"], np.float32).reshape(kat["a"]["shape"])
            b = np.array(kat["b"]["data"], np.float32).reshape(kat["b"]["shape"])
            assert O.matmul(a, b).ravel().tolist() == kat["c"], kat["src"]
        else:
            a = np.array(kat["a"]["data"], np.float32).reshape(kat["a"]["shape"])
            pend = np.zeros_like(a)
            O.matmul_vjp(a, a, np.ones_like(a), pend, pend)
            assert pend.ravel().tolist() == kat["pending_after"], kat["src"]


def test_oracle_reproduces_example_1b():
    ex = json.load(open(os.path.join(GOLDEN, "example_1b.json")))
    x = (np.arange(3 * 224 * 224) % 256).astype(np.float32) / np.float32(255.0)
    x = x.reshape(1, 3, 224, 224)
    w = O.seeded_weights(3, 8, (3, 3), 123)
    assert w.ravel().tolist() == ex["w"]
    y = O.conv2d_forward(x, w, 1, 1)
    dx, dw = O.conv2d_backward(x, w, (y + y).astype(np.float32), 1, 1)
    assert hashlib.sha256(y.tobytes()).hexdigest() == ex["sha256_y_f32"]
    assert hashlib.sha256(dx.tobytes()).hexdigest() == ex["sha256_dx_f32"]
    assert dw.ravel().tolist() == ex["dw"]
    assert O.fsum((y * y).astype(np.float32)) == ex["loss_sum_y_sq"]
