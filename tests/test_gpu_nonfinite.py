"""Non-finite inputs: the GPU convolutions against the CPU oracle.

The reference visits only valid (input, weight, output) triples and skips
padded taps (crates/katsu-core/src/conv2d.rs:240-255); NaN and Inf then
follow f32 arithmetic over the visited products (docs/api.md:34).  The MFMA
kernels multiply a padded halo's zeros (and a gathered filter's absent taps,
and zeroed tile lanes) as well, which is harmless for finite data but turns
0 * Inf into NaN.  The kernels recompute such outputs over the visited
products, so the results must match the oracle's class by class: the NaN,
+Inf and -Inf masks exactly, and every finite value within the f32 bound.

Inf, -Inf and NaN are planted in x, w and G at border taps (a corner of the
filter, the first and last rows and columns of the images) and in the
interior.  Batches are chosen so each layer takes the kernels the planner
uses at the BASELINE size (the direct halo kernels need enough tiles to fill
the chip): config 3 at N = 9, config 4a at N = 16, the stem at N = 9; a
config-3 layer at N = 2 takes the generic engine, config 4b the 1x1 kernels
and config 1 the few-channel kernels."""
import numpy as np
import pytest

from katsu_amd import synth
from oracle import oracle as O
from tests.parity import assert_within

pytestmark = pytest.mark.gpu

INF = np.float32(np.inf)
NAN = np.float32(np.nan)


def _plant(c):
    """Seeded inputs of config c with non-finite values planted."""
    x, w = synth.conv_inputs(c)
    g = synth.normal(synth.SEED_G, synth.out_shape(c))
    n, ci, h, wd = x.shape
    k, _, r, s = w.shape
    _, _, oh, ow = g.shape
    # Filter: a corner tap (padded at the top-left border outputs), the
    # opposite corner of another output channel, and a NaN at the centre of a
    # third (k >= 3 in every case below).
    w[0, 0, 0, 0] = INF
    w[min(1, k - 1), min(2, ci - 1), r - 1, s - 1] = -INF
    w[min(2, k - 1), min(1, ci - 1), r // 2, s // 2] = NAN
    # Input: corners and edges of the image, one interior NaN.
    x[0, 0, 0, 0] = INF
    x[0, min(1, ci - 1), 0, wd - 1] = -INF
    x[n - 1, ci - 1, h - 1, wd // 2] = INF
    x[n - 1, ci - 1, h // 2, wd // 3] = NAN
    # Upstream gradient: border and interior, several channels.
    g[0, 0, 0, 0] = INF
    g[0, min(3, k - 1), oh - 1, ow // 2] = -INF
    g[n - 1, k - 1, oh // 2, ow - 1] = INF
    g[n - 1, min(5, k - 1), oh // 2, ow // 2] = NAN
    return x, w, g


def _finite0(a):
    return np.where(np.isfinite(a), np.abs(a), 0).astype(np.float32)


def _check(got, ref, s, kred, what):
    got = np.asarray(got)
    for name, mask in (("NaN", np.isnan), ("+Inf", np.isposinf), ("-Inf", np.isneginf)):
        gm, rm = mask(got), mask(ref)
        if not np.array_equal(gm, rm):
            diff = np.argwhere(gm != rm)
            idx = tuple(diff[0])
            raise AssertionError(f"{what}: {name} mask differs at {len(diff)} elements; first "
                                 f"{idx}: gpu {got[idx]!r} oracle {ref[idx]!r}")
    fin = np.isfinite(ref)
    assert_within(got[fin], ref[fin], s[fin], kred, what)


def _run_all(x, w, g, st, p, dev):
    import torch

    from katsu_amd import ops
    xd, wd, gd = (torch.from_numpy(np.ascontiguousarray(a)).to(dev) for a in (x, w, g))
    y = ops.conv2d_forward(xd, wd, st, p)
    dx = ops.conv2d_backward_data(gd, wd, x.shape, st, p)
    dw = ops.conv2d_backward_filter(xd, gd, w.shape, st, p)
    dx1, dw1 = ops.conv2d_backward(xd, wd, gd, st, p)
    # beta = 1 into finite pending buffers: the original value plus the
    # recomputed one.
    init_x = torch.from_numpy(synth.uniform(61, x.shape)).to(dev)
    init_w = torch.from_numpy(synth.uniform(62, w.shape)).to(dev)
    dxa, dwa = ops.conv2d_backward(xd, wd, gd, st, p, dx=init_x.clone(), dw=init_w.clone(),
                                   beta=1.0)
    torch.cuda.synchronize()
    out = [t.cpu().numpy() for t in (y, dx, dw, dx1, dw1, dxa, dwa)]
    return out, init_x.cpu().numpy(), init_w.cpu().numpy()


CASES = [
    ("c3_resnet", 9),     # direct forward, stride-1 dX, one-launch backward
    ("c3_resnet", 2),     # the generic engine (too few tiles for the direct kernels)
    ("c4a_down3x3", 16),  # stride-2 forward, phase-form dX, stride-2 dW
    ("c4b_down1x1", 4),   # 1x1 kernels (no padding)
    ("c5_stem", 9),       # stem forward, dW and rolling-row dX
    ("c1_example", 1),    # few-channel kernels
]


@pytest.mark.parametrize("name,batch", CASES)
def test_nonfinite_inputs_match_oracle(name, batch, dev):
    c = dict(synth.CONV_CONFIGS[name])
    c["x"] = (batch,) + c["x"][1:]
    x, w, g = _plant(c)
    st, p = c["stride"], c["pad"]
    k, ci, r, s = w.shape
    n, _, oh, ow = g.shape
    print(f"\n{name} N={batch}: x{x.shape} w{w.shape} s{st} p{p}", flush=True)
    (y, dx, dw, dx1, dw1, dxa, dwa), init_x, init_w = _run_all(x, w, g, st, p, dev)
    y_ref = O.conv2d_forward(x, w, st, p)
    dx_ref, dw_ref = O.conv2d_backward(x, w, g, st, p)
    ys = O.conv2d_forward(_finite0(x), _finite0(w), st, p)
    dxs, dws = O.conv2d_backward(_finite0(x), _finite0(w), _finite0(g), st, p)
    # The planted values reach borders and interiors of every output.
    for ref in (y_ref, dx_ref, dw_ref):
        assert np.isnan(ref).any() or np.isinf(ref).any()
        assert np.isfinite(ref).any()
    _check(y, y_ref, ys, ci * r * s, f"{name} fwd")
    _check(dx, dx_ref, dxs, k * r * s, f"{name} dX")
    _check(dw, dw_ref, dws, n * oh * ow, f"{name} dW")
    _check(dx1, dx_ref, dxs, k * r * s, f"{name} one-call dX")
    _check(dw1, dw_ref, dws, n * oh * ow, f"{name} one-call dW")
    # beta = 1: one more rounding of the pending value (S grows by |init|).
    _check(dxa, (init_x + dx_ref).astype(np.float32), dxs + np.abs(init_x), k * r * s + 1,
           f"{name} one-call dX beta=1")
    _check(dwa, (init_w + dw_ref).astype(np.float32), dws + np.abs(init_w), n * oh * ow + 1,
           f"{name} one-call dW beta=1")


def test_nonfinite_host_entry_points(dev):
    """The drop-in host-pointer entry points on a config-3 layer with planted
    non-finite values (direct kernels, N = 9)."""
    from katsu_amd import host
    c = dict(synth.CONV_CONFIGS["c3_resnet"])
    c["x"] = (9,) + c["x"][1:]
    x, w, g = _plant(c)
    y = host.conv2d_forward(x, w, 1, 1)
    dx, dw = host.conv2d_backward(x, w, g, 1, 1)
    y_ref = O.conv2d_forward(x, w, 1, 1)
    dx_ref, dw_ref = O.conv2d_backward(x, w, g, 1, 1)
    ys = O.conv2d_forward(_finite0(x), _finite0(w), 1, 1)
    dxs, dws = O.conv2d_backward(_finite0(x), _finite0(w), _finite0(g), 1, 1)
    _check(y, y_ref, ys, 64 * 9, "host fwd")
    _check(dx, dx_ref, dxs, 64 * 9, "host dX")
    _check(dw, dw_ref, dws, 9 * 56 * 56, "host dW")


@pytest.mark.parametrize("plant", [False, True])
def test_forward_two_fragment_counts(plant, dev):
    """Config 3's forward at N = 16, the smallest batch that takes the tiles
    of two fragment counts (each image's first tiles 13 fragments, the rest
    12): every output against the oracle, on finite data and with Inf and NaN
    planted in x and w (the classes exactly, finite values within the f32
    bound)."""
    import torch

    from katsu_amd import ops
    c = dict(synth.CONV_CONFIGS["c3_resnet"])
    c["x"] = (16,) + c["x"][1:]
    if plant:
        x, w, _ = _plant(c)
    else:
        x, w = synth.conv_inputs(c)
    st, p = c["stride"], c["pad"]
    print(f"\nc3_resnet N=16 forward plant={plant}", flush=True)
    y = ops.conv2d_forward(torch.from_numpy(x).to(dev), torch.from_numpy(w).to(dev), st, p)
    torch.cuda.synchronize()
    y_ref = O.conv2d_forward(x, w, st, p)
    ys = O.conv2d_forward(_finite0(x), _finite0(w), st, p)
    if plant:
        assert np.isfinite(y_ref).any() and not np.isfinite(y_ref).all()
    _check(y.cpu().numpy(), y_ref, ys, w.shape[1] * w.shape[2] * w.shape[3], "fwd N=16")


@pytest.mark.parametrize("plant", [False, True])
def test_dx_two_fragment_counts(plant, dev):
    """The separate data-gradient call at config 3's shapes and N = 16, which
    takes the same tiles of two fragment counts as the forward (the stride-1
    dX is the forward's kernel on G with the flipped filter): every element
    of dX against the oracle, on finite data and with Inf and NaN planted in
    w and G."""
    import torch

    from katsu_amd import ops
    c = dict(synth.CONV_CONFIGS["c3_resnet"])
    c["x"] = (16,) + c["x"][1:]
    if plant:
        x, w, g = _plant(c)
    else:
        x, w = synth.conv_inputs(c)
        g = synth.normal(synth.SEED_G, synth.out_shape(c))
    st, p = c["stride"], c["pad"]
    print(f"\nc3_resnet N=16 dX plant={plant}", flush=True)
    dx = ops.conv2d_backward_data(torch.from_numpy(g).to(dev), torch.from_numpy(w).to(dev),
                                  x.shape, st, p)
    torch.cuda.synchronize()
    dx_ref, _ = O.conv2d_backward(x, w, g, st, p)
    dxs, _ = O.conv2d_backward(_finite0(x), _finite0(w), _finite0(g), st, p)
    if plant:
        assert np.isfinite(dx_ref).any() and not np.isfinite(dx_ref).all()
    _check(dx.cpu().numpy(), dx_ref, dxs, w.shape[0] * w.shape[2] * w.shape[3], "dX N=16")
