"""The allocation-free one-call backward (katsu_hip_conv2d_bwd_f32_dev_noalloc)
against the allocating entry point (katsu_hip_conv2d_bwd_f32_dev): same
kernels and plans, so the same bits.  Two calls in a row on the static
scratch, the second with a smaller input, and calls of every backward path
(direct one-launch at stride 1 and 2, the 1x1 kernels, the stem's two
launches, the few-channel kernels, the generic engine)."""
import ctypes

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


def test_workspace_bound_covers_every_plan():
    """Every BASELINE layer's workspace fits the static scratch (no GPU)."""
    lim = _abi.lib().katsu_hip_noalloc_scratch_bytes()
    for name, c in synth.CONV_CONFIGS.items():
        need = ops.bwd_filter_workspace_bytes(c["x"], c["w"], c["stride"], c["pad"])
        assert 0 <= need <= lim, (name, need)
