"""The allocation-free one-call backward (katsu_hip_conv2d_bwd_f32_dev_noalloc)
against the allocating entry point (katsu_hip_conv2d_bwd_f32_dev): same
kernels and plans, so the same bits.  Two calls in a row on the static
scratch, the second with a smaller input, and calls of every backward path
(direct one-launch at stride 1 and 2, the 1x1 kernels, the stem's two
launches, the few-channel kernels, the generic engine, one buffer for dX and
dW).  A fresh process that calls it first, on every path, must see the
library's device-allocation count stay at zero."""
import ctypes
import json
import os
import subprocess
import sys

import numpy as np
import pytest

from katsu_amd import _abi, ops, synth

pytestmark = pytest.mark.gpu


def _both(c, dev, beta):
    import torch
    x, w = synth.conv_inputs(c)
    g = synth.normal(synth.SEED_G, synth.out_shape(c))
    st, p = c["stride"], c["pad"]
    xd, wd, gd = (torch.from_numpy(a).to(dev) for a in (x, w, g))
    init_x = torch.from_numpy(synth.uniform(51, x.shape)).to(dev)
    init_w = torch.from_numpy(synth.uniform(52, w.shape)).to(dev)
    ref_dx, ref_dw = init_x.clone(), init_w.clone()
    ops.conv2d_backward(xd, wd, gd, st, p, dx=ref_dx, dw=ref_dw, beta=beta)
    dx, dw = init_x.clone(), init_w.clone()
    geo = ops.conv_geom(x.shape, w.shape, st, p)
    torch.cuda.synchronize()
    rc = _abi.lib().katsu_hip_conv2d_bwd_f32_dev_noalloc(
        ops._p(xd), ops._p(wd), ops._p(gd), ops._p(dx), ops._p(dw), ctypes.byref(geo),
        float(beta), ops._stream())
    assert rc == _abi.OK, _abi.strerror(rc)
    torch.cuda.synchronize()
    return (dx, dw), (ref_dx, ref_dw)


def _cfg(name, batch):
    c = dict(synth.CONV_CONFIGS[name])
    c["x"] = (batch,) + c["x"][1:]
    return c


def test_two_calls_second_smaller(dev):
    """Config 3 at its full batch, then a smaller batch: the static scratch
    keeps the first call's partials, and the second must not read them."""
    import torch
    assert _abi.lib().katsu_hip_noalloc_scratch_bytes() == 40 << 20
    for batch, beta in ((32, 0.0), (12, 1.0)):
        print(f"c3_resnet N={batch} beta={beta}", flush=True)
        (dx, dw), (rx, rw) = _both(_cfg("c3_resnet", batch), dev, beta)
        assert torch.equal(dx, rx)
        assert torch.equal(dw, rw)


@pytest.mark.parametrize("name,batch", [("c4a_down3x3", 32), ("c4b_down1x1", 32),
                                        ("c5_stem", 8), ("c1_example", 1), ("c3_resnet", 2)])
def test_every_backward_path(name, batch, dev):
    import torch
    print(f"{name} N={batch}", flush=True)
    for beta in (0.0, 1.0):
        (dx, dw), (rx, rw) = _both(_cfg(name, batch), dev, beta)
        assert torch.equal(dx, rx)
        assert torch.equal(dw, rw)


def test_shared_dx_dw_buffer(dev):
    """The weights are the input (tests/conv2d.rs:109-116): one buffer
    receives beta*buf + dX + dW, dX added first."""
    import torch
    a = synth.uniform(53, (2, 3, 3, 3))
    g = synth.normal(synth.SEED_G, (2, 2, 3, 3))
    ad, gd = torch.from_numpy(a).to(dev), torch.from_numpy(g).to(dev)
    init = torch.from_numpy(synth.uniform(54, a.shape)).to(dev)
    ref = init.clone()
    ops.conv2d_backward(ad, ad, gd, 1, 1, dx=ref, dw=ref, beta=1.0)
    buf = init.clone()
    geo = ops.conv_geom(a.shape, a.shape, 1, 1)
    torch.cuda.synchronize()
    rc = _abi.lib().katsu_hip_conv2d_bwd_f32_dev_noalloc(
        ops._p(ad), ops._p(ad), ops._p(gd), ops._p(buf), ops._p(buf), ctypes.byref(geo), 1.0,
        ops._stream())
    assert rc == _abi.OK, _abi.strerror(rc)
    torch.cuda.synchronize()
    assert torch.equal(buf, ref)


# Run in a fresh interpreter: the allocation-free entry point on every
# backward path before anything else of the library runs, then one
# allocating call (library scratch for the dW partials) to show the count
# moves when the library does allocate.
_FRESH = r"""
import ctypes, json, sys
sys.path.insert(0, sys.argv[1])
import torch
from katsu_amd import _abi, ops, synth
L = _abi.lib()
dev = torch.device("cuda:0")
counts = {"start": L.katsu_hip_device_allocations()}

def cfg(name, batch):
    c = dict(synth.CONV_CONFIGS[name])
    c["x"] = (batch,) + c["x"][1:]
    return c

def call(xd, wd, gd, dx, dw, st, p, beta):
    geo = ops.conv_geom(tuple(xd.shape), tuple(wd.shape), st, p)
    rc = L.katsu_hip_conv2d_bwd_f32_dev_noalloc(ops._p(xd), ops._p(wd), ops._p(gd), ops._p(dx),
                                               ops._p(dw), ctypes.byref(geo), float(beta),
                                               ops._stream())
    torch.cuda.synchronize()
    assert rc == 0, _abi.strerror(rc)

for name, batch in (("c3_resnet", 32), ("c4a_down3x3", 32), ("c4b_down1x1", 32),
                    ("c5_stem", 8), ("c1_example", 1), ("c3_resnet", 2)):
    c = cfg(name, batch)
    x, w = synth.conv_inputs(c)
    g = synth.normal(synth.SEED_G, synth.out_shape(c))
    xd, wd, gd = (torch.from_numpy(a).to(dev) for a in (x, w, g))
    for beta in (0.0, 1.0):
        call(xd, wd, gd, torch.zeros_like(xd), torch.zeros_like(wd), c["stride"], c["pad"], beta)
    counts[f"{name} N={batch}"] = L.katsu_hip_device_allocations()
a = torch.from_numpy(synth.uniform(53, (2, 3, 3, 3))).to(dev)
g = torch.from_numpy(synth.normal(synth.SEED_G, (2, 2, 3, 3))).to(dev)
buf = torch.zeros_like(a)
call(a, a, g, buf, buf, 1, 1, 1.0)
counts["shared dx/dw buffer"] = L.katsu_hip_device_allocations()
c = cfg("c3_resnet", 32)
x, w = synth.conv_inputs(c)
xd, wd = torch.from_numpy(x).to(dev), torch.from_numpy(w).to(dev)
ops.conv2d_backward(xd, wd, torch.ones(synth.out_shape(c), device=dev), 1, 1)
torch.cuda.synchronize()
counts["allocating entry point"] = L.katsu_hip_device_allocations()
print(json.dumps(counts), flush=True)
"""


def test_fresh_process_allocates_nothing():
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, "-c", _FRESH, root], capture_output=True, text=True,
                       timeout=300, cwd=root)
    assert r.returncode == 0, r.stderr[-2000:]
    counts = json.loads([l for l in r.stdout.splitlines() if l.startswith("{")][-1])
    print(counts)
    after = counts.pop("allocating entry point")
    assert all(v == 0 for v in counts.values()), counts
    assert after > 0, "the allocating entry point should have allocated its dW scratch"
