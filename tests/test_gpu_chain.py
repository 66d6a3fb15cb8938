"""The config-5 chain at its real shapes, every step on the device through the
C ABI, each against an independent reference:

  y  = stem(x)            x [64,3,224,224] U[0,1), w [64,3,7,7] He-normal, s2 p3
  P  = meanpool(y)        [64,64], over 112*112 = 12544 pixels per row
  C  = P . H              H [64,1000] He-normal (fan_in 64)   (tensor.rs:264-273)
  L  = sum(C)             so G = 1                            (tensor.rs:242-247, 410-417)
  dP = G . H^T, dH = P^T . G                                  (tensor.rs:424-444)
  dY = dP / 12544 spread over each row
  dX, dW = backward_buffers(x, w, dY)                         (conv2d.rs:265-292)

(The benchmark's config-5 chain: Katsu has no pool op, so the pool and its
VJP are the caller's glue between two public calls.)  The matmul head and its VJP are
compared in full with the CPU oracle; the stem passes on sampled elements
with exact f64 dot products; the pool with an f64 mean of the device's y."""
import numpy as np
import pytest

from katsu_amd import synth
from oracle import oracle as O
from tests.parity import (assert_within, edge_samples, gamma, random_samples, sample_dw,
                          sample_dx, sample_fwd)

pytestmark = pytest.mark.gpu


def test_stem_chain_real_shapes(dev):
    import torch

    from katsu_amd import ops
    c = synth.CONV_CONFIGS["c5_stem"]
    x, w = synth.conv_inputs(c)
    h = synth.he_normal(synth.SEED_HEAD, (64, 1000))
    st, p = c["stride"], c["pad"]
    xd, wd, hd = (torch.from_numpy(a).to(dev) for a in (x, w, h))
    y = ops.conv2d_forward(xd, wd, st, p)
    n, k, oh, ow = y.shape
    hw = oh * ow
    assert (n, k, hw) == (64, 64, 12544)
    pool = ops.mean_rows(y, n * k, hw).reshape(n, k)
    cmat = ops.matmul(pool, hd)
    loss = ops.sum(cmat)
    gmat = torch.ones_like(cmat)
    dpool = torch.zeros_like(pool)
    dh = torch.zeros_like(hd)
    ops.matmul_vjp(pool, hd, gmat, dpool, dh)
    scale = np.float32(1.0) / np.float32(hw)
    dy = ops.broadcast_rows(dpool.reshape(-1), n * k, hw, float(scale)).reshape(y.shape)
    dx, dw = ops.conv2d_backward(xd, wd, dy, st, p)
    torch.cuda.synchronize()
    y_h, pool_h, c_h = y.cpu().numpy(), pool.cpu().numpy(), cmat.cpu().numpy()
    dpool_h, dh_h, dy_h = dpool.cpu().numpy(), dh.cpu().numpy(), dy.cpu().numpy()
    dx_h, dw_h = dx.cpu().numpy(), dw.cpu().numpy()

    # Stem forward, sampled.
    ys = random_samples(y_h.shape, 300, 11) + edge_samples(y_h.shape)
    ref, sab = sample_fwd(x, w, st, p, ys)
    assert_within(np.array([y_h[t] for t in ys]), ref, sab, 3 * 49, "stem fwd")
    # Pool: f64 mean of the device's y, bound of an f32 sum of 12544 terms
    # plus the division's rounding.
    rows = y_h.reshape(n * k, hw).astype(np.float64)
    exact = rows.sum(axis=1) / hw
    lim = gamma(hw) * np.abs(rows).sum(axis=1) / hw + 2.0 ** -24 * np.abs(exact)
    assert np.all(np.abs(pool_h.ravel() - exact) <= 2 * lim), "mean pool"
    # Head and its VJP: full oracle comparison.
    assert_within(c_h, O.matmul(pool_h, h), np.abs(pool_h) @ np.abs(h), 64, "head C")
    da_ref, db_ref = O.matmul_vjp(pool_h, h, np.ones((64, 1000), np.float32))
    assert_within(dpool_h, da_ref, np.ones((64, 1000)) @ np.abs(h).T, 1000, "head dA")
    assert_within(dh_h, db_ref, np.abs(pool_h).T @ np.ones((64, 1000)), 64, "head dB")
    # With G = 1 every row of dA is H's row sums.
    assert np.all(dpool_h == dpool_h[0:1])
    # The loss: the oracle's sequential sum of the device's C, within the
    # bound of a 64000-term sum.
    ls = float(loss.cpu().numpy()[0])
    assert abs(ls - O.fsum(c_h)) <= 2 * gamma(64000) * float(np.abs(c_h).sum())
    # Spread: dY = dP * (1/12544), one rounding.
    assert np.array_equal(dy_h, (dpool_h.reshape(n, k, 1, 1) * scale) *
                          np.ones((1, 1, oh, ow), np.float32))
    # Stem backward seeded with dY, sampled.
    xs = random_samples(x.shape, 300, 12) + edge_samples(x.shape)
    ref, sab = sample_dx(dy_h, w, x.shape, st, p, xs)
    assert_within(np.array([dx_h[t] for t in xs]), ref, sab, 64 * 49, "stem dX")
    wsamp = random_samples(w.shape, 48, 13) + [(0, 0, 0, 0), (63, 2, 6, 6), (5, 1, 3, 0)]
    ref, sab = sample_dw(x, dy_h, w.shape, st, p, wsamp)
    assert_within(np.array([dw_h[t] for t in wsamp]), ref, sab, n * hw, "stem dW")
