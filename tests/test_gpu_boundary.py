"""The C ABI's edges on the GPU: the host-pointer matmul at shapes whose
GEMM splits K (its library scratch), scratch that a captured graph keeps
using after the library needed a larger buffer, and the one-call backward
with dx and dw the same buffer (an engine's pending buffer when input and
weights are one node, tensor.rs:374-391)."""
import ctypes

import numpy as np
import pytest

from katsu_amd import host, synth
from oracle import oracle as O
from tests.parity import assert_within

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("m,k,n", [(64, 1000, 64), (128, 512, 128), (64, 64, 1000)])
def test_host_matmul_and_vjp_split_k(m, k, n):
    """Tensor::matmul and its VJP through the host-pointer seams (S1, S2) at
    shapes whose dedicated GEMM splits K (the config-5 head's dA is
    64 x 1000 . 1000 x 64), against the oracle."""
    a = synth.uniform(71, (m, k))
    b = synth.uniform(72, (k, n))
    g = synth.uniform(73, (m, n))
    c = host.matmul(a, b)
    assert_within(c, O.matmul(a, b), np.abs(a) @ np.abs(b), k, "C")
    da0 = synth.uniform(74, (m, k))
    db0 = synth.uniform(75, (k, n))
    da, db = host.matmul_vjp(a, b, g, da0.copy(), db0.copy())
    da_ref, db_ref = O.matmul_vjp(a, b, g, da0.copy(), db0.copy())
    assert_within(da, da_ref, np.abs(g) @ np.abs(b).T + np.abs(da0), n + 1, "dA")
    assert_within(db, db_ref, np.abs(a).T @ np.abs(g) + np.abs(db0), m + 1, "dB")


def test_graph_keeps_scratch_after_growth(dev):
    """A captured split-K GEMM keeps its partials buffer: a later, larger
    split-K GEMM on the same stream makes the library take a bigger buffer,
    and the graph's replays must still give the eager result, each time."""
    import torch

    from katsu_amd import ops
    a = torch.from_numpy(synth.uniform(81, (64, 512))).to(dev)
    b = torch.from_numpy(synth.uniform(82, (512, 64))).to(dev)
    big_a = torch.from_numpy(synth.uniform(83, (128, 2048))).to(dev)
    big_b = torch.from_numpy(synth.uniform(84, (2048, 128))).to(dev)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        eager = ops.matmul(a, b)  # warm-up: plans, scratch and kernel attributes
        torch.cuda.synchronize()
        out = torch.empty_like(eager)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=s):
            ops.gemm(a, b, 64, 64, 512, out=out)
        big = ops.matmul(big_a, big_b)  # grows this stream's GEMM scratch
        torch.cuda.synchronize()
        big_ref = big.clone()
        for _ in range(3):
            out.fill_(float("nan"))
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, eager)
            again = ops.matmul(big_a, big_b)
            torch.cuda.synchronize()
            assert torch.equal(again, big_ref)


def _backward_aliased_expect(x, w, g, init, st, p, dev):
    """(init + dX) + dW from the separate device calls, the order the
    reference's two += make."""
    import torch

    from katsu_amd import ops
    xd, wd, gd = (torch.from_numpy(a).to(dev) for a in (x, w, g))
    dx = ops.conv2d_backward_data(gd, wd, x.shape, st, p)
    dw = ops.conv2d_backward_filter(xd, gd, w.shape, st, p)
    torch.cuda.synchronize()
    return (init + dx.cpu().numpy()) + dw.cpu().numpy().reshape(init.shape)


@pytest.mark.parametrize("shape,st,p", [((4, 3, 3, 3), 1, 1), ((8, 5, 3, 3), 2, 1)])
def test_backward_same_buffer(shape, st, p, dev):
    """dx and dw the same buffer (input and weights one node, so the shapes
    are equal): the host entry point and the device one both give
    (pending + dX) + dW, dX first, with beta = 1; with beta = 0,
    dX + dW."""
    import torch

    from katsu_amd import ops
    x = synth.uniform(91, shape)
    w = x.copy()
    n, c, h, wd = shape
    oh, ow = (h + 2 * p - 3) // st + 1, (wd + 2 * p - 3) // st + 1
    g = synth.normal(92, (n, n, oh, ow))
    init = synth.uniform(93, shape)
    want = _backward_aliased_expect(x, w, g, init, st, p, dev)
    # Host pointers: one numpy buffer for both outputs.
    buf = init.copy()
    geo = host.geometry(*shape, n, 3, 3, st, p)
    L = host.lib()
    ptr = ctypes.c_void_p(buf.ctypes.data)
    rc = L.katsu_hip_conv2d_bwd_f32(ctypes.c_void_p(x.ctypes.data),
                                    ctypes.c_void_p(w.ctypes.data),
                                    ctypes.c_void_p(g.ctypes.data), ptr, ptr,
                                    ctypes.byref(geo), 1.0)
    assert rc == 0
    assert np.array_equal(buf, want)
    # Device pointers, beta 1 and beta 0.
    xd, wd, gd = (torch.from_numpy(a).to(dev) for a in (x, w, g))
    pend = torch.from_numpy(init.copy()).to(dev)
    ops.conv2d_backward(xd, wd, gd, st, p, dx=pend, dw=pend, beta=1.0)
    torch.cuda.synchronize()
    assert np.array_equal(pend.cpu().numpy(), want)
    fresh = torch.full(shape, 7.0, device=dev)
    ops.conv2d_backward(xd, wd, gd, st, p, dx=fresh, dw=fresh, beta=0.0)
    torch.cuda.synchronize()
    zero = np.zeros(shape, np.float32)
    assert np.array_equal(fresh.cpu().numpy(),
                          _backward_aliased_expect(x, w, g, zero, st, p, dev))
    # Against the oracle, within the bound of the two passes.
    dx_ref, dw_ref = O.conv2d_backward(x, w, g, st, p)
    dxs, dws = O.conv2d_backward(np.abs(x), np.abs(w), np.abs(g), st, p)
    kred = max(n * 9, n * oh * ow) + 2
    assert_within(buf, (init + dx_ref) + dw_ref, np.abs(init) + dxs + dws, kred, "aliased")


# Bytes per operand against the host copies' pinned ring (8 MiB chunks, four
# slots, copies under 1 MiB passed straight to HIP): below the ring, half a
# chunk, one chunk exactly, one row past it, and four chunks plus a partial
# one (the ring wraps, in both directions).
@pytest.mark.parametrize("m,n", [(256, 256), (1024, 1024), (2048, 1024), (2049, 1024),
                                 (3072, 3072)])
def test_host_copies_through_pinned_ring(m, n, dev):
    """The host-pointer GEMM with beta = 1 (C goes in and comes back) gives
    the same bits as the device entry point on the same operands."""
    import torch

    from katsu_amd import ops
    k = 64
    a = synth.uniform(91, (m, k))
    b = synth.uniform(92, (k, n))
    c0 = synth.uniform(93, (m, n))
    c = host.gemm(a, b, c0.copy(), m, n, k, beta=1.0)
    cd = torch.from_numpy(c0).to(dev)
    ops.gemm(torch.from_numpy(a).to(dev), torch.from_numpy(b).to(dev), m, n, k, out=cd,
             beta=1.0)
    torch.cuda.synchronize()
    assert np.array_equal(c, cd.cpu().numpy())
