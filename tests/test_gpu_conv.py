"""GPU parity of the convolution passes against the CPU oracle.

Every call goes through the C ABI (libkatsu_hip.so).  Known-answer tests
from the reference are compared exactly; everything else within the f32
dot-product bound (tests/parity.py)."""
import numpy as np
import pytest

from katsu_amd import synth
from oracle import oracle as O
from tests.parity import (assert_within, edge_samples, max_rel_mixed, random_samples,
                          sample_dw, sample_dx, sample_fwd)

pytestmark = pytest.mark.gpu


def _run(x, w, g, st, p, dev):
    import torch

    from katsu_amd import ops
    xd = torch.from_numpy(np.ascontiguousarray(x)).to(dev)
    wd = torch.from_numpy(np.ascontiguousarray(w)).to(dev)
    gd = torch.from_numpy(np.ascontiguousarray(g)).to(dev)
    y = ops.conv2d_forward(xd, wd, st, p)
    dx = ops.conv2d_backward_data(gd, wd, x.shape, st, p)
    dw = ops.conv2d_backward_filter(xd, gd, w.shape, st, p)
    torch.cuda.synchronize()
    return y.cpu().numpy(), dx.cpu().numpy(), dw.cpu().numpy()


def _check_full(x, w, g, st, p, dev, what):
    y, dx, dw = _run(x, w, g, st, p, dev)
    k, c, r, s = w.shape
    n, _, oh, ow = g.shape
    y_ref = O.conv2d_forward(x, w, st, p)
    dx_ref, dw_ref = O.conv2d_backward(x, w, g, st, p)
    ys = O.conv2d_forward(np.abs(x), np.abs(w), st, p)
    dxs, dws = O.conv2d_backward(np.abs(x), np.abs(w), np.abs(g), st, p)
    assert_within(y, y_ref, ys, c * r * s, f"{what} fwd")
    assert_within(dx, dx_ref, dxs, k * r * s, f"{what} dX")
    assert_within(dw, dw_ref, dws, max(1, n * oh * ow), f"{what} dW")
    return y, dx, dw


# (x shape, w shape, stride, padding): tile edges, every stride phase
# pattern, rectangular kernels, tiny and >128 channel counts.
CASES = [
    ((2, 2, 3, 4), (2, 2, 2, 3), 1, 0),   # the shapes of tests/conv2d.rs:46-87
    ((2, 2, 3, 4), (2, 2, 2, 3), 1, 1),
    ((2, 2, 3, 4), (2, 2, 2, 3), 2, 1),
    ((3, 5, 17, 13), (7, 5, 3, 3), 1, 1),
    ((2, 3, 20, 21), (70, 3, 5, 5), 2, 2),
    ((1, 130, 9, 9), (20, 130, 3, 3), 1, 1),
    ((2, 16, 15, 15), (130, 16, 1, 1), 2, 0),   # 1x1 stride 2: phases without taps
    ((1, 4, 11, 11), (3, 4, 7, 7), 3, 3),       # 9 phases
    ((2, 8, 8, 8), (16, 8, 3, 3), 1, 0),
    ((1, 2, 5, 5), (4, 2, 5, 5), 1, 0),         # kernel covers the whole input
    ((1, 3, 6, 7), (2, 3, 2, 2), 4, 1),         # 16 phases, some empty
    ((1, 2, 20, 20), (3, 2, 3, 3), 5, 2),       # 25 phases: more than one launch
    ((2, 33, 10, 12), (65, 33, 1, 3), 1, 1),    # rectangular kernel, odd channels
    ((1, 1, 1, 1), (1, 1, 1, 1), 1, 0),
]


@pytest.mark.parametrize("xs,ws,st,p", CASES)
def test_conv_parity_small(xs, ws, st, p, dev):
    x = synth.uniform(101, xs)
    w = synth.uniform(102, ws)
    oh = (xs[2] + 2 * p - ws[2]) // st + 1
    ow = (xs[3] + 2 * p - ws[3]) // st + 1
    g = synth.uniform(103, (xs[0], ws[0], oh, ow))
    _check_full(x, w, g, st, p, dev, f"{xs}*{ws} s{st} p{p}")


def test_known_answers_exact(dev):
    """tests/conv2d.rs:16-43 and 172-179, bit-exact on the GPU."""
    x = np.arange(1, 10, dtype=np.float32).reshape(1, 1, 3, 3)
    w = np.array([1, 2, 3, 4], np.float32).reshape(1, 1, 2, 2)
    y, dx, dw = _run(x, w, np.ones((1, 1, 2, 2), np.float32), 1, 0, dev)
    assert y.ravel().tolist() == [37, 47, 67, 77]
    assert dx.ravel().tolist() == [1, 3, 2, 4, 10, 6, 3, 7, 4]
    assert dw.ravel().tolist() == [12, 16, 24, 28]
    y2, _, _ = _run(x, w, np.ones((1, 1, 2, 2), np.float32), 2, 1, dev)
    assert y2.ravel().tolist() == [4, 18, 36, 77]


def test_reference_finite_difference_cases(dev):
    """The exact inputs of tests/conv2d.rs:46-87; the reference's own metric at 1e-6."""
    for st, p in [(1, 0), (1, 1), (2, 1)]:
        xs, ws = (2, 2, 3, 4), (2, 2, 2, 3)
        x = ((np.arange(48) % 11) * np.float32(0.07) - np.float32(0.3)).astype(np.float32)
        w = ((np.arange(24) % 7) * np.float32(0.09) - np.float32(0.2)).astype(np.float32)
        x, w = x.reshape(xs), w.reshape(ws)
        oh = (3 + 2 * p - 2) // st + 1
        ow = (4 + 2 * p - 3) // st + 1
        g = ((np.arange(2 * 2 * oh * ow) % 5) * np.float32(0.13)
             - np.float32(0.2)).astype(np.float32).reshape(2, 2, oh, ow)
        y, dx, dw = _check_full(x, w, g, st, p, dev, f"fd s{st} p{p}")
        dx_ref, dw_ref = O.conv2d_backward(x, w, g, st, p)
        assert max_rel_mixed(dx, dx_ref) <= 1e-6
        assert max_rel_mixed(dw, dw_ref) <= 1e-6


def test_empty_batch(dev):
    """tests/conv2d.rs:156-167: N=0 gives an empty output and dW of zeros."""
    import torch

    from katsu_amd import ops
    x = torch.zeros((0, 3, 4, 5), device=dev)
    w = torch.from_numpy(synth.uniform(5, (2, 3, 3, 3))).to(dev)
    y = ops.conv2d_forward(x, w, 1, 1)
    assert tuple(y.shape) == (0, 2, 4, 5)
    dw = torch.full((2, 3, 3, 3), 7.0, device=dev)
    ops.conv2d_backward_filter(x, y, (2, 3, 3, 3), 1, 1, out=dw)
    assert torch.all(dw == 0).item()
    dx = ops.conv2d_backward_data(y, w, (0, 3, 4, 5), 1, 1)
    assert dx.numel() == 0


def test_beta_accumulates_exactly(dev):
    """beta=1 adds the fresh result to the pending buffer: fl(init + fresh)."""
    import torch

    from katsu_amd import ops
    xs, ws, st, p = (2, 6, 12, 10), (9, 6, 3, 3), 2, 1
    x = torch.from_numpy(synth.uniform(21, xs)).to(dev)
    w = torch.from_numpy(synth.uniform(22, ws)).to(dev)
    g = torch.from_numpy(synth.uniform(23, (2, 9, 6, 5))).to(dev)
    dx0 = ops.conv2d_backward_data(g, w, xs, st, p)
    dw0 = ops.conv2d_backward_filter(x, g, ws, st, p)
    init_x = torch.from_numpy(synth.uniform(24, xs)).to(dev)
    init_w = torch.from_numpy(synth.uniform(25, ws)).to(dev)
    dx1 = ops.conv2d_backward_data(g, w, xs, st, p, out=init_x.clone(), beta=1.0)
    dw1 = ops.conv2d_backward_filter(x, g, ws, st, p, out=init_w.clone(), beta=1.0)
    torch.cuda.synchronize()
    assert torch.equal(dx1, init_x + dx0)
    assert torch.equal(dw1, init_w + dw0)


def test_filter_gradient_is_deterministic(dev):
    """Split-K partials are reduced in a fixed order: identical bits every run."""
    import torch

    from katsu_amd import ops
    c = synth.CONV_CONFIGS["c3_resnet"]
    xs = (4,) + c["x"][1:]
    x = torch.from_numpy(synth.uniform(31, xs)).to(dev)
    g = torch.from_numpy(synth.uniform(32, (4, 64, 56, 56))).to(dev)
    a = ops.conv2d_backward_filter(x, g, c["w"], 1, 1)
    b = ops.conv2d_backward_filter(x, g, c["w"], 1, 1)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


@pytest.mark.parametrize("name,batch", [("c1_example", 1), ("c3_resnet", 2),
                                        ("c4a_down3x3", 2), ("c4b_down1x1", 2),
                                        ("c5_stem", 1)])
def test_baseline_layers_small_batch(name, batch, dev):
    """The BASELINE layers' channel and kernel shapes at a batch of 1 or 2,
    full oracle comparison with a random upstream gradient (all-ones would
    hide a flipped kernel).  At these batches configs 3 and 4a take the
    generic engine (too few tiles for the direct kernels); the production
    kernels are the next test's."""
    c = dict(synth.CONV_CONFIGS[name])
    c["x"] = (batch,) + c["x"][1:]
    x, w = synth.conv_inputs(c)
    g = synth.normal(synth.SEED_G, synth.out_shape(c))
    _check_full(x, w, g, c["stride"], c["pad"], dev, name)


# A stride-1 3x3 layer with 40-pixel rows: like config 3's 56, 8 (mod 16), so
# the direct kernels stage its halo rows 8 floats longer; 40 rows take the
# plain (one tile size) forward tiles where config 3 takes two sizes.
_ROWS40 = dict(x=(32, 64, 40, 40), w=(64, 64, 3, 3), stride=1, pad=1, law="u11")


@pytest.mark.parametrize("name,batch", [("c3_resnet", 9), ("c4a_down3x3", 16),
                                        ("c5_stem", 9), ("c4b_down1x1", 32),
                                        ("rows40", 32)])
def test_production_kernels_full_parity(name, batch, dev):
    """The kernels the BASELINE configurations run (the direct 3x3 kernels of
    configs 3 and 4a and their one-launch backward, the stem's kernels, the
    1x1 kernels) at the smallest batch where the planner picks them: every
    element of y, dX and dW, from the separate calls and from the one-call
    backward, against the oracle on finite random data."""
    import torch

    from katsu_amd import ops
    c = dict(_ROWS40 if name == "rows40" else synth.CONV_CONFIGS[name])
    c["x"] = (batch,) + c["x"][1:]
    x, w = synth.conv_inputs(c)
    g = synth.normal(synth.SEED_G, synth.out_shape(c))
    st, p = c["stride"], c["pad"]
    print(f"\n{name} N={batch}", flush=True)
    y, dx, dw = _run(x, w, g, st, p, dev)
    xd, wd, gd = (torch.from_numpy(a).to(dev) for a in (x, w, g))
    dx1, dw1 = ops.conv2d_backward(xd, wd, gd, st, p)
    torch.cuda.synchronize()
    k, ci, r, s = w.shape
    n, _, oh, ow = g.shape
    y_ref = O.conv2d_forward(x, w, st, p)
    dx_ref, dw_ref = O.conv2d_backward(x, w, g, st, p)
    ys = O.conv2d_forward(np.abs(x), np.abs(w), st, p)
    dxs, dws = O.conv2d_backward(np.abs(x), np.abs(w), np.abs(g), st, p)
    assert_within(y, y_ref, ys, ci * r * s, f"{name} fwd")
    for what, got_dx, got_dw in (("separate", dx, dw),
                                 ("one-call", dx1.cpu().numpy(), dw1.cpu().numpy())):
        assert_within(got_dx, dx_ref, dxs, k * r * s, f"{name} {what} dX")
        assert_within(got_dw, dw_ref, dws, n * oh * ow, f"{name} {what} dW")


def test_repo_example_config1(dev):
    """examples/conv2d/main.rs:5-9: X=(i%256)/255, new_seeded(3,8,(3,3),1,1,123),
    loss sum(Y*Y) so G = 2Y exactly (tensor.rs:392-409)."""
    x = ((np.arange(3 * 224 * 224) % 256).astype(np.float32) / np.float32(255.0)
         ).reshape(1, 3, 224, 224)
    w = O.seeded_weights(3, 8, (3, 3), 123)
    y_ref = O.conv2d_forward(x, w, 1, 1)
    g = (y_ref + y_ref).astype(np.float32)  # the two Mul edges into a zero pending buffer
    _check_full(x, w, g, 1, 1, dev, "repo example")


@pytest.mark.parametrize("name", ["c3_resnet", "c4a_down3x3", "c4b_down1x1", "c5_stem"])
def test_baseline_configs_full_size_sampled(name, dev):
    """Full BASELINE sizes: sampled outputs against exact f64 dot products
    (edges and corners included), within the f32 bound."""
    c = synth.CONV_CONFIGS[name]
    x, w = synth.conv_inputs(c)
    st, p = c["stride"], c["pad"]
    yshape = synth.out_shape(c)
    g = synth.normal(synth.SEED_G, yshape)
    y, dx, dw = _run(x, w, g, st, p, dev)
    k, cin, r, s = w.shape
    ys = random_samples(yshape, 300, 1) + edge_samples(yshape)
    ref, sab = sample_fwd(x, w, st, p, ys)
    assert_within(np.array([y[t] for t in ys]), ref, sab, cin * r * s, f"{name} fwd")
    xs = random_samples(x.shape, 300, 2) + edge_samples(x.shape)
    ref, sab = sample_dx(g, w, x.shape, st, p, xs)
    assert_within(np.array([dx[t] for t in xs]), ref, sab, k * r * s, f"{name} dX")
    ws = random_samples(w.shape, 64, 3) + [(0, 0, 0, 0), (k - 1, cin - 1, r - 1, s - 1)]
    ref, sab = sample_dw(x, g, w.shape, st, p, ws)
    kred = yshape[0] * yshape[2] * yshape[3]
    assert_within(np.array([dw[t] for t in ws]), ref, sab, kred, f"{name} dW")


def test_batch_linearity_of_filter_gradient(dev):
    """dW over a batch equals the sum of dW over its halves (up to rounding):
    a size-independent property at the config-3 shape."""
    import torch

    from katsu_amd import ops
    c = synth.CONV_CONFIGS["c3_resnet"]
    x, w = synth.conv_inputs(c)
    g = synth.normal(synth.SEED_G, synth.out_shape(c))
    xd, gd = torch.from_numpy(x).to(dev), torch.from_numpy(g).to(dev)
    full = ops.conv2d_backward_filter(xd, gd, w.shape, 1, 1)
    h = x.shape[0] // 2
    a = ops.conv2d_backward_filter(xd[:h].contiguous(), gd[:h].contiguous(), w.shape, 1, 1)
    b = ops.conv2d_backward_filter(xd[h:].contiguous(), gd[h:].contiguous(), w.shape, 1, 1)
    torch.cuda.synchronize()
    xs = np.abs(x).astype(np.float64)
    gs = np.abs(g).astype(np.float64)
    # S for every dw element via the sampled helper would be slow; bound by the
    # global maximum instead: S <= sum over n,oy,ox of max|x| * |g[:, oc]|.
    s_oc = xs.max() * gs.sum(axis=(0, 2, 3))
    s = np.broadcast_to(s_oc[:, None, None, None], w.shape)
    assert_within((a + b).cpu().numpy(), full.cpu().numpy(), s, 32 * 56 * 56, "linearity")


@pytest.mark.parametrize("xs", [(4, 3, 224, 224), (8, 3, 150, 130), (3, 2, 101, 99)])
def test_stem_forward_direct(xs, dev):
    """7x7 stride-2 forward with few input channels (stem-like layers at
    sizes between the small cases and the full config-5 sampled test), full
    output against the oracle; (3,2,101,99) has two channels and odd
    sizes."""
    import torch

    from katsu_amd import ops
    ws = (64, xs[1], 7, 7)
    x = synth.uniform(301, xs)
    w = synth.normal(302, ws)
    y = ops.conv2d_forward(torch.from_numpy(x).to(dev), torch.from_numpy(w).to(dev), 2, 3)
    torch.cuda.synchronize()
    y_ref = O.conv2d_forward(x, w, 2, 3)
    ys = O.conv2d_forward(np.abs(x), np.abs(w), 2, 3)
    assert_within(y.cpu().numpy(), y_ref, ys, xs[1] * 49, f"stem fwd {xs}")


@pytest.mark.parametrize("xs,k,st", [((2, 3, 224, 224), 64, 2),   # the stem at batch 2
                                     ((3, 3, 129, 130), 70, 2),   # 65-pixel rows; 70 outputs
                                     ((2, 3, 100, 111), 64, 1),   # stride 1: 111-pixel rows
                                     ((1, 3, 40, 64), 16, 1)])    # 64-pixel rows, 16 outputs
def test_stem_forward(xs, k, st, dev):
    """Forward of 3-channel 7x7 layers with padding 3 (the stem kernel:
    k = (c, r, s) in the filter's order, 37 k-steps, each lane's tap offset
    in a register) against the oracle: rows shorter than the 112 pixels the
    waves cover (the lanes past the end are computed and not stored), an
    output-channel block of 6, both strides."""
    import torch

    from katsu_amd import ops
    ws = (k, 3, 7, 7)
    x = synth.uniform(341, xs)
    w = synth.normal(342, ws)
    y = ops.conv2d_forward(torch.from_numpy(x).to(dev), torch.from_numpy(w).to(dev), st, 3)
    torch.cuda.synchronize()
    ref = O.conv2d_forward(x, w, st, 3)
    sab = O.conv2d_forward(np.abs(x), np.abs(w), st, 3)
    assert_within(y.cpu().numpy(), ref, sab, 147, f"stem fwd {xs} k{k} s{st}")


@pytest.mark.parametrize("xs", [(4, 3, 224, 224), (5, 3, 61, 150), (1, 3, 20, 300)])
def test_stem_filter_gradient(xs, dev):
    """7x7 stride-2 filter gradient of a 3-channel layer (the stem kernel:
    56-pixel half-row tiles, two row groups per block, one partial per block)
    against the oracle.  (5,3,61,150) has 75-pixel rows, so its second tile
    of each row is partly empty; (1,3,20,300) has 150-pixel rows (three
    tiles, the last partial) and few tiles per block."""
    import torch

    from katsu_amd import ops
    ws = (64, 3, 7, 7)
    x = synth.uniform(311, xs)
    oh, ow = (xs[2] + 6 - 7) // 2 + 1, (xs[3] + 6 - 7) // 2 + 1
    g = synth.normal(313, (xs[0], 64, oh, ow))
    dw = ops.conv2d_backward_filter(torch.from_numpy(x).to(dev), torch.from_numpy(g).to(dev),
                                    ws, 2, 3)
    torch.cuda.synchronize()
    _, dw_ref = O.conv2d_backward(x, np.zeros(ws, np.float32), g, 2, 3)
    _, dws = O.conv2d_backward(np.abs(x), np.zeros(ws, np.float32), np.abs(g), 2, 3)
    assert_within(dw.cpu().numpy(), dw_ref, dws, xs[0] * oh * ow, f"stem dW {xs}")


@pytest.mark.parametrize("xs,ws,st,p", [
    ((1, 3, 224, 224), (8, 3, 3, 3), 1, 1),   # config 1 (the repo example's shape)
    ((2, 2, 9, 11), (5, 2, 3, 2), 2, 1),      # stride 2, rectangular filter
    ((3, 4, 7, 6), (16, 4, 2, 2), 1, 2),      # padding wider than the filter overhang
    ((1, 1, 5, 5), (3, 1, 5, 5), 3, 2),
    ((1, 3, 224, 224), (8, 3, 3, 3), 2, 1),   # 3x3 register forms: stride 2
    ((2, 4, 17, 13), (16, 4, 3, 3), 2, 1),    # 16 outputs, 4 channels, odd sizes
    ((3, 1, 30, 70), (4, 1, 3, 3), 1, 0),     # 4 outputs, 1 channel, no padding
    ((2, 2, 20, 19), (7, 2, 3, 3), 1, 2),     # padding past the filter overhang
    ((600, 1, 8, 8), (2, 1, 3, 3), 1, 1),     # more dW tiles than dW blocks
])
def test_few_channel_bit_exact(xs, ws, st, p, dev):
    """Layers with at most 4 input and 16 output channels run on the vector
    ALUs in the reference's own summation order with separate multiply and
    add roundings: the forward and dX equal the oracle (the reference's
    loops) bit for bit; dW is a parallel sum, within the f32 bound.  beta = 1
    adds dX into an existing buffer with one more rounding, as the engine's
    pending += does."""
    import torch

    from katsu_amd import ops
    x = synth.uniform(321, xs)
    w = synth.normal(322, ws)
    oh = (xs[2] + 2 * p - ws[2]) // st + 1
    ow = (xs[3] + 2 * p - ws[3]) // st + 1
    g = synth.normal(323, (xs[0], ws[0], oh, ow))
    xd, wd, gd = (torch.from_numpy(a).to(dev) for a in (x, w, g))
    y = ops.conv2d_forward(xd, wd, st, p)
    dx = ops.conv2d_backward_data(gd, wd, xs, st, p)
    dw = ops.conv2d_backward_filter(xd, gd, ws, st, p)
    dx0 = synth.uniform(324, xs)
    dxa = torch.from_numpy(dx0.copy()).to(dev)
    ops.conv2d_backward_data(gd, wd, xs, st, p, out=dxa, beta=1.0)
    torch.cuda.synchronize()
    y_ref = O.conv2d_forward(x, w, st, p)
    dx_ref, dw_ref = O.conv2d_backward(x, w, g, st, p)
    assert np.array_equal(y.cpu().numpy(), y_ref), "forward not bit-exact"
    assert np.array_equal(dx.cpu().numpy(), dx_ref), "dX not bit-exact"
    assert np.array_equal(dxa.cpu().numpy(), (dx0 + dx_ref).astype(np.float32)), "dX beta=1"
    _, dws = O.conv2d_backward(np.abs(x), np.abs(w), np.abs(g), st, p)
    assert_within(dw.cpu().numpy(), dw_ref, dws, xs[0] * oh * ow, "few-channel dW")
    # The dW blocks sum their own partials in a fixed tree (the 3x3 forms):
    # the same bits on every call, and beta = 1 adds one more rounding.
    for _ in range(3):
        again = ops.conv2d_backward_filter(xd, gd, ws, st, p)
        torch.cuda.synchronize()
        assert torch.equal(again, dw), "dW differs between calls"
    dw0 = synth.uniform(325, ws)
    dwa = torch.from_numpy(dw0.copy()).to(dev)
    ops.conv2d_backward_filter(xd, gd, ws, st, p, out=dwa, beta=1.0)
    torch.cuda.synchronize()
    assert np.array_equal(dwa.cpu().numpy(), (dw0 + dw.cpu().numpy()).astype(np.float32)), \
        "dW beta=1"


def test_stem_kernels_two_channel_blocks(dev):
    """3-channel 7x7 stride-2 layers with 96 output channels: the stem
    forward and filter-gradient kernels split them into two 64-channel
    blocks (the second half empty past 96)."""
    import torch

    from katsu_amd import ops
    xs, ws = (2, 3, 160, 200), (96, 3, 7, 7)
    x = synth.uniform(331, xs)
    w = synth.normal(332, ws)
    oh, ow = (xs[2] + 6 - 7) // 2 + 1, (xs[3] + 6 - 7) // 2 + 1
    g = synth.normal(333, (xs[0], ws[0], oh, ow))
    xd, wd, gd = (torch.from_numpy(a).to(dev) for a in (x, w, g))
    y = ops.conv2d_forward(xd, wd, 2, 3)
    dw = ops.conv2d_backward_filter(xd, gd, ws, 2, 3)
    torch.cuda.synchronize()
    y_ref = O.conv2d_forward(x, w, 2, 3)
    ys = O.conv2d_forward(np.abs(x), np.abs(w), 2, 3)
    assert_within(y.cpu().numpy(), y_ref, ys, 3 * 49, "stem fwd, 96 channels")
    _, dw_ref = O.conv2d_backward(x, w, g, 2, 3)
    _, dws = O.conv2d_backward(np.abs(x), np.abs(w), np.abs(g), 2, 3)
    assert_within(dw.cpu().numpy(), dw_ref, dws, xs[0] * oh * ow, "stem dW, 96 channels")
