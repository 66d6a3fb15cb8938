"""The one-call backward (katsu_hip_conv2d_bwd_f32[_dev]) against the two
separate passes.  Where dX and dW share one launch, dX comes from the same
kernel and summation order as the separate call and must be identical bit for
bit; dW splits its pixel reduction into half as many partials there, so it
must agree with the separate call within the bound of two fp32 sums of the
same products.  The shared launch takes 3x3 layers at stride 1 (stride-1 dX
blocks) and stride 2 (phase-form dX blocks) with enough blocks to fill the
GPU.  Unpadded 1x1 layers share one launch with the separate passes' own
plans; they and the other shapes (few blocks, small channel counts, other
filter sizes) must match the separate passes bit for bit.  beta = 1
accumulates into both outputs."""
import numpy as np
import pytest

from katsu_amd import synth
from oracle import oracle as O
from tests.parity import assert_within, gamma

pytestmark = pytest.mark.gpu

# (x shape, w shape, stride, pad, whether dX and dW share one launch)
CASES = [
    ((32, 64, 56, 56), (64, 64, 3, 3), 1, 1, True),    # config 3
    ((32, 64, 30, 30), (64, 64, 3, 3), 1, 1, True),    # rows not a multiple of 4 (masked dW)
    ((32, 80, 28, 28), (96, 80, 3, 3), 1, 1, True),    # channel counts off the tiles
    ((2, 80, 17, 9), (96, 80, 3, 3), 1, 0, False),     # too few blocks to fuse
    ((4, 128, 28, 28), (256, 128, 3, 3), 2, 1, False),  # stride 2, too few blocks to fuse
    ((32, 128, 28, 28), (256, 128, 3, 3), 2, 1, True),  # config 4a: phase-form dX + stride-2 dW
    ((32, 64, 27, 27), (128, 64, 3, 3), 2, 1, True),    # odd sizes
    ((2, 3, 40, 40), (64, 3, 7, 7), 2, 3, False),      # stem-like, too small for its kernels
    ((16, 3, 224, 224), (64, 3, 7, 7), 2, 3, False),   # the stem's kernels, as two launches
    ((2, 16, 12, 12), (8, 16, 1, 1), 1, 0, False),     # 1x1
    ((32, 128, 28, 28), (256, 128, 1, 1), 2, 0, False),  # config 4b: one pw_bwd_kernel launch
    ((6, 40, 15, 17), (24, 40, 1, 1), 2, 0, False),    # 1x1 stride 2, odd sizes
    ((16, 40, 30, 32), (64, 40, 1, 1), 1, 0, False),   # 1x1 stride 1, 240 dW slices
    ((1, 3, 224, 224), (8, 3, 3, 3), 1, 1, False),     # config 1: few-channel register forms
    ((2, 4, 17, 13), (16, 4, 3, 3), 2, 1, False),      # few channels, stride 2
    ((600, 1, 8, 8), (2, 1, 3, 3), 1, 1, False),       # more dW tiles than dW blocks
]


def _tensors(xs, ws, st, p, dev):
    import torch
    c = {"x": xs, "w": ws, "stride": st, "pad": p}
    x = synth.uniform(synth.SEED_X, xs, -1.0, 1.0)
    w = synth.normal(synth.SEED_W, ws)
    g = synth.normal(synth.SEED_G, synth.out_shape(c))
    return [torch.from_numpy(a).to(dev) for a in (x, w, g)]


@pytest.mark.parametrize("xs,ws,st,p,fused", CASES)
def test_fused_matches_separate(xs, ws, st, p, fused, dev):
    import torch

    from katsu_amd import ops
    x, w, g = _tensors(xs, ws, st, p, dev)
    # Both dW sums lie within 2*gamma(K)*S of the exact one, S the same sum
    # over |x|*|G| (computed here in fp32, hence the 1e-5 margin), so they lie
    # within twice that of each other; with beta = 1 each result adds one more
    # rounding of its own magnitude.
    oshape = synth.out_shape({"x": xs, "w": ws, "stride": st, "pad": p})
    kred = xs[0] * oshape[2] * oshape[3]
    s_abs = ops.conv2d_backward_filter(x.abs(), g.abs(), w.shape, st, p).double()
    lim = 4.0 * gamma(kred) * s_abs * (1 + 1e-5)
    for beta in (0.0, 1.0):
        dx0 = torch.randn(x.shape, device=dev) if beta else None
        dw0 = torch.randn(w.shape, device=dev) if beta else None
        dx_s = ops.conv2d_backward_data(g, w, x.shape, st, p,
                                        out=None if dx0 is None else dx0.clone(), beta=beta)
        dw_s = ops.conv2d_backward_filter(x, g, w.shape, st, p,
                                          out=None if dw0 is None else dw0.clone(), beta=beta)
        dx_f, dw_f = ops.conv2d_backward(x, w, g, st, p,
                                         dx=None if dx0 is None else dx0.clone(),
                                         dw=None if dw0 is None else dw0.clone(), beta=beta)
        torch.cuda.synchronize()
        assert torch.equal(dx_f, dx_s), f"dX beta={beta}"
        if not fused:
            assert torch.equal(dw_f, dw_s), f"dW beta={beta}"
            continue
        err = (dw_f.double() - dw_s.double()).abs()
        lim_b = lim + 2.0 ** -24 * (dw_f.double().abs() + dw_s.double().abs())
        assert bool((err <= lim_b).all()), \
            f"dW beta={beta}: worst excess {(err - lim_b).max().item():.3e}"


@pytest.mark.parametrize("xs,ws,st,p", [((32, 64, 56, 56), (64, 64, 3, 3), 1, 1),
                                        ((32, 128, 28, 28), (256, 128, 3, 3), 2, 1)])
def test_fused_matches_separate_nonfinite(xs, ws, st, p, dev):
    """Inf, -Inf and NaN planted in G and w (border and interior): the shared
    launch's dX blocks (at config 3 the two-size tiles of the shared launch,
    at config 4a the phase form) take the recompute of non-finite outputs as
    the separate dX call does, so the two dX tensors hold the same bits,
    NaNs included; dW's non-finite classes agree too."""
    import torch

    from katsu_amd import ops
    x, w, g = _tensors(xs, ws, st, p, dev)
    n, k, oh, ow = g.shape
    g[0, 0, 0, 0] = float("inf")
    g[n // 2, k // 3, oh // 2, ow - 1] = float("-inf")
    g[n - 1, k - 1, oh - 1, ow // 3] = float("nan")
    w[1, 2, 0, 1] = float("inf")
    dx_s = ops.conv2d_backward_data(g, w, x.shape, st, p)
    dw_s = ops.conv2d_backward_filter(x, g, w.shape, st, p)
    dx_f, dw_f = ops.conv2d_backward(x, w, g, st, p)
    torch.cuda.synchronize()
    assert not torch.isfinite(dx_s).all(), "the planted values must reach dX"
    assert torch.equal(dx_f.view(torch.int32), dx_s.view(torch.int32)), "dX bits"
    for f in (torch.isnan, torch.isposinf, torch.isneginf):
        assert torch.equal(f(dw_f), f(dw_s)), f"dW {f.__name__}"


def test_fused_caller_workspace_and_graph_replay(dev):
    import torch

    from katsu_amd import ops
    xs, ws, st, p = (8, 64, 56, 56), (64, 64, 3, 3), 1, 1
    x, w, g = _tensors(xs, ws, st, p, dev)
    nbytes = ops.bwd_filter_workspace_bytes(xs, ws, st, p)
    work = torch.empty(max(1, nbytes), device=dev, dtype=torch.uint8)
    dx = torch.empty_like(x)
    dw = torch.empty_like(w)
    ops.conv2d_backward(x, w, g, st, p, dx=dx, dw=dw, workspace=work)
    torch.cuda.synchronize()
    ref = (dx.clone(), dw.clone())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        ops.conv2d_backward(x, w, g, st, p, dx=dx, dw=dw, workspace=work)
    for _ in range(3):
        dx.fill_(float("nan"))
        dw.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(dx, ref[0]) and torch.equal(dw, ref[1])


def test_fused_host_entry_against_oracle():
    """The host-pointer form (what katsu-core's backward_buffers would call)
    against the CPU oracle, at a size that takes the shared launch (256 dX
    blocks; 384 dW row tiles, 128 partials there against 192 in the separate
    dW call)."""
    from katsu_amd import host
    xs, ws, st, p = (16, 64, 24, 24), (64, 64, 3, 3), 1, 1
    c = {"x": xs, "w": ws, "stride": st, "pad": p}
    x = synth.uniform(synth.SEED_X, xs, -1.0, 1.0)
    w = synth.normal(synth.SEED_W, ws)
    g = synth.normal(synth.SEED_G, synth.out_shape(c))
    dx, dw = host.conv2d_backward(x, w, g, st, p)
    dx_ref, dw_ref = O.conv2d_backward(x, w, g, st, p)
    dxs, dws = O.conv2d_backward(np.abs(x), np.abs(w), np.abs(g), st, p)
    assert_within(dx, dx_ref, dxs, 64 * 9, "fused host dX")
    assert_within(dw, dw_ref, dws, 16 * 24 * 24, "fused host dW")


@pytest.mark.parametrize("name", ["c3_resnet", "c4a_down3x3"])
def test_fused_full_size_sampled_exact(name, dev):
    """The one-call backward the bench times, at the full BASELINE shape
    (config 3: one direct_bwd_kernel launch of stride-1 dX and dW blocks;
    config 4a: phase-form dX with stride-2 dW blocks), against exact f64 dot
    products on sampled elements (corners and edges included).  The bound
    2*gamma(K)*S takes S from the same f64 evaluation (tests/parity.py), not
    from the GPU.  With the bench's all-ones G (config 3) and a random G."""
    import torch

    from katsu_amd import ops
    from tests.parity import edge_samples, random_samples, sample_dw, sample_dx
    c = synth.CONV_CONFIGS[name]
    x, w = synth.conv_inputs(c)
    st, p = c["stride"], c["pad"]
    yshape = synth.out_shape(c)
    k, cin, r, s = w.shape
    kred_w = yshape[0] * yshape[2] * yshape[3]
    grads = [synth.normal(synth.SEED_G, yshape)]
    if name == "c3_resnet":
        grads.append(np.ones(yshape, np.float32))
    for g in grads:
        xd, wd, gd = (torch.from_numpy(a).to(dev) for a in (x, w, g))
        dx, dw = ops.conv2d_backward(xd, wd, gd, st, p)
        torch.cuda.synchronize()
        dx, dw = dx.cpu().numpy(), dw.cpu().numpy()
        xs = random_samples(x.shape, 400, 5) + edge_samples(x.shape)
        ref, sab = sample_dx(g, w, x.shape, st, p, xs)
        assert_within(np.array([dx[t] for t in xs]), ref, sab, k * r * s, f"{name} dX")
        ws = random_samples(w.shape, 96, 6) + [(0, 0, 0, 0), (k - 1, cin - 1, r - 1, s - 1),
                                              (0, cin - 1, 0, s - 1), (k - 1, 0, r - 1, 0)]
        ref, sab = sample_dw(x, g, w.shape, st, p, ws)
        assert_within(np.array([dw[t] for t in ws]), ref, sab, kred_w, f"{name} dW")
