"""Pins for the CPU oracle (oracle/katsu_oracle.c), CPU only.

Each oracle function is checked against (1) the reference's own known-answer
and finite-difference tests (crates/katsu-core/tests/*.rs), (2) independent
f64 evaluations (torch CPU conv/grad routines and numpy slicing), (3) exact
small-integer cases, and (4) published SplitMix64 outputs.  test_mutants
shows that planted mistakes in the oracle fail these pins."""
import numpy as np
import pytest

from katsu_amd import synth
from oracle import oracle as O
from tests.parity import (assert_within, max_rel_mixed, random_samples, sample_dw, sample_dx,
                          sample_fwd)

X9 = np.arange(1, 10, dtype=np.float32).reshape(1, 1, 3, 3)
W4 = np.array([1, 2, 3, 4], np.float32).reshape(1, 1, 2, 2)


# ---- known answers (exact) -------------------------------------------------

def test_known_forward_and_overlap_gradients():
    """tests/conv2d.rs:16-43."""
    y = O.conv2d_forward(X9, W4, 1, 0)
    assert y.shape == (1, 1, 2, 2)
    assert y.ravel().tolist() == [37, 47, 67, 77]
    dx, dw = O.conv2d_backward(X9, W4, np.ones((1, 1, 2, 2), np.float32), 1, 0)
    assert dx.ravel().tolist() == [1, 3, 2, 4, 10, 6, 3, 7, 4]
    assert dw.ravel().tolist() == [12, 16, 24, 28]


def test_known_stride_and_padding():
    """tests/conv2d.rs:172-179."""
    assert O.conv2d_forward(X9, W4, 2, 1).ravel().tolist() == [4, 18, 36, 77]


def test_reused_layer_gradients():
    """tests/conv2d.rs:90-106: w=2 applied to a=3 and b=5; loss ya+yb."""
    w = np.array([[[[2.0]]]], np.float32)
    a = np.array([[[[3.0]]]], np.float32)
    b = np.array([[[[5.0]]]], np.float32)
    one = np.ones((1, 1, 1, 1), np.float32)
    da, dwa = O.conv2d_backward(a, w, one, 1, 0)
    db, dwb = O.conv2d_backward(b, w, one, 1, 0)
    assert (dwa + dwb).ravel().tolist() == [8.0]
    assert da.ravel().tolist() == [2.0] and db.ravel().tolist() == [2.0]
    assert dwb.ravel().tolist() == [5.0]
    assert O.conv2d_forward(b, w, 1, 0).ravel().tolist() == [10.0]


def test_shared_operand_chain():
    """tests/conv2d.rs:109-116: weights are the input; y = x*x, z = y*x,
    d sum(z)/dx = 12 at x = 2, composed from the local VJPs."""
    x = np.array([[[[2.0]]]], np.float32)
    y = O.conv2d_forward(x, x, 1, 0)
    one = np.ones((1, 1, 1, 1), np.float32)
    dy, dx_w2 = O.conv2d_backward(y, x, one, 1, 0)       # z = conv(y, w=x)
    dx_in, dx_w1 = O.conv2d_backward(x, x, dy, 1, 0)     # y = conv(x, w=x)
    assert float((dx_w2 + dx_in + dx_w1).ravel()[0]) == 12.0


def test_rectangular_matmul():
    """tests/tensor.rs:41-48 (also examples/basic.rs:7)."""
    a = np.arange(1, 7, dtype=np.float32).reshape(2, 3)
    b = np.arange(7, 13, dtype=np.float32).reshape(3, 2)
    assert O.matmul(a, b).ravel().tolist() == [58, 64, 139, 154]


def test_same_parent_accumulates_both_edges():
    """tests/autograd.rs:98-103: a@a with one pending buffer for both edges."""
    a = np.array([[1, 2], [3, 4]], np.float32)
    pend = np.zeros((2, 2), np.float32)
    O.matmul_vjp(a, a, np.ones((2, 2), np.float32), pend, pend)
    assert pend.ravel().tolist() == [7, 11, 9, 13]


def test_empty_matmul_and_vjp():
    """tests/tensor.rs:65-74 and autograd.rs:106-111."""
    c = O.matmul(np.zeros((2, 0), np.float32), np.zeros((0, 3), np.float32))
    assert c.ravel().tolist() == [0.0] * 6
    da, db = O.matmul_vjp(np.zeros((2, 0), np.float32), np.zeros((0, 3), np.float32),
                          np.ones((2, 3), np.float32))
    assert da.size == 0 and db.size == 0


def test_empty_batch():
    """tests/conv2d.rs:156-167."""
    w = O.seeded_weights(3, 2, (3, 3), 7)
    x = np.zeros((0, 3, 4, 5), np.float32)
    y = O.conv2d_forward(x, w, 1, 1)
    assert y.shape == (0, 2, 4, 5)
    dx, dw = O.conv2d_backward(x, w, y, 1, 1)
    assert dx.size == 0 and np.all(dw == 0)


# ---- finite differences (the reference's own tests) -------------------------

@pytest.mark.parametrize("st,p", [(1, 0), (1, 1), (2, 1)])
def test_conv_finite_differences(st, p):
    """tests/conv2d.rs:46-87, same inputs, eps and tolerance."""
    xs, ws = (2, 2, 3, 4), (2, 2, 2, 3)
    xv = ((np.arange(48) % 11) * np.float32(0.07) - np.float32(0.3)).astype(np.float32)
    wv = ((np.arange(24) % 7) * np.float32(0.09) - np.float32(0.2)).astype(np.float32)
    y = O.conv2d_forward(xv.reshape(xs), wv.reshape(ws), st, p)
    seed = ((np.arange(y.size) % 5) * np.float32(0.13) - np.float32(0.2)).astype(np.float32)
    dx, dw = O.conv2d_backward(xv.reshape(xs), wv.reshape(ws), seed.reshape(y.shape), st, p)

    def ev(xa, wa):
        out = O.conv2d_forward(xa.reshape(xs), wa.reshape(ws), st, p).ravel()
        return O.fsum((out * seed).astype(np.float32))

    eps = np.float32(0.001)
    for side, grad in ((0, dx.ravel()), (1, dw.ravel())):
        for i, expected in enumerate(grad):
            xp, xm, wp, wm = xv.copy(), xv.copy(), wv.copy(), wv.copy()
            if side == 0:
                xp[i] += eps
                xm[i] -= eps
            else:
                wp[i] += eps
                wm[i] -= eps
            num = (ev(xp, wp) - ev(xm, wm)) / (2 * 0.001)
            assert max_rel_mixed([expected], [num]) <= 3e-4, (side, i, expected, num)


def test_matmul_finite_differences():
    """tests/autograd.rs:63-95: loss sum(y*y) so G = 2y; eps 1e-3, abs tol 1e-3."""
    av = np.array([0.2, -0.4, 0.7, 0.3, 0.8, -0.1], np.float32)
    bv = np.array([0.1, 0.5, -0.3, 0.6, 0.9, -0.2], np.float32)
    y = O.matmul(av.reshape(2, 3), bv.reshape(3, 2))
    da, db = O.matmul_vjp(av.reshape(2, 3), bv.reshape(3, 2), (y + y).astype(np.float32))

    def ev(a, b):
        yy = O.matmul(a.reshape(2, 3), b.reshape(3, 2))
        return O.fsum((yy * yy).astype(np.float32))

    for side, grad in ((0, da.ravel()), (1, db.ravel())):
        for i in range(6):
            ap, am, bp, bm = av.copy(), av.copy(), bv.copy(), bv.copy()
            if side == 0:
                ap[i] += np.float32(0.001)
                am[i] -= np.float32(0.001)
            else:
                bp[i] += np.float32(0.001)
                bm[i] -= np.float32(0.001)
            num = (ev(ap, bp) - ev(am, bm)) / 0.002
            assert abs(grad[i] - num) < 1e-3, (side, i)


# ---- independent f64 evaluations -------------------------------------------

CONV_CASES = [((2, 3, 7, 9), (4, 3, 3, 3), 1, 1), ((1, 2, 9, 8), (3, 2, 2, 3), 2, 1),
              ((2, 4, 11, 10), (5, 4, 5, 5), 3, 2), ((1, 5, 6, 6), (2, 5, 1, 1), 2, 0),
              ((1, 3, 16, 16), (6, 3, 7, 7), 2, 3)]


@pytest.mark.parametrize("xs,ws,st,p", CONV_CASES)
def test_conv_against_torch_f64(xs, ws, st, p):
    """torch.nn.functional.conv2d and torch.nn.grad.conv2d_input/_weight (CPU,
    float64) are a library restatement of the same cross-correlation."""
    import torch
    x = synth.uniform(41, xs)
    w = synth.uniform(42, ws)
    y = O.conv2d_forward(x, w, st, p)
    g = synth.uniform(43, y.shape)
    dx, dw = O.conv2d_backward(x, w, g, st, p)
    xt, wt, gt = (torch.from_numpy(a.astype(np.float64)) for a in (x, w, g))
    y64 = torch.nn.functional.conv2d(xt, wt, stride=st, padding=p).numpy()
    dx64 = torch.nn.grad.conv2d_input(xt.shape, wt, gt, stride=st, padding=p).numpy()
    dw64 = torch.nn.grad.conv2d_weight(xt, wt.shape, gt, stride=st, padding=p).numpy()
    ax, aw, ag = (torch.from_numpy(np.abs(a).astype(np.float64)) for a in (x, w, g))
    ys = torch.nn.functional.conv2d(ax, aw, stride=st, padding=p).numpy()
    dxs = torch.nn.grad.conv2d_input(ax.shape, aw, ag, stride=st, padding=p).numpy()
    dws = torch.nn.grad.conv2d_weight(ax, aw.shape, ag, stride=st, padding=p).numpy()
    k, c, r, s = ws
    # One-sided: the oracle's own error against exact is <= gamma(K) S; use 2x.
    assert_within(y, y64, ys, c * r * s, "fwd")
    assert_within(dx, dx64, dxs, k * r * s, "dX")
    assert_within(dw, dw64, dws, xs[0] * y.shape[2] * y.shape[3], "dW")


@pytest.mark.parametrize("xs,ws,st,p", CONV_CASES)
def test_conv_against_sampled_f64(xs, ws, st, p):
    x = synth.normal(51, xs)
    w = synth.normal(52, ws)
    y = O.conv2d_forward(x, w, st, p)
    g = synth.normal(53, y.shape)
    dx, dw = O.conv2d_backward(x, w, g, st, p)
    k, c, r, s = ws
    ys = random_samples(y.shape, 40, 1)
    ref, sab = sample_fwd(x, w, st, p, ys)
    assert_within([y[t] for t in ys], ref, sab, c * r * s, "fwd")
    xsamp = random_samples(x.shape, 40, 2)
    ref, sab = sample_dx(g, w, x.shape, st, p, xsamp)
    assert_within([dx[t] for t in xsamp], ref, sab, k * r * s, "dX")
    wsamp = random_samples(w.shape, 20, 3)
    ref, sab = sample_dw(x, g, w.shape, st, p, wsamp)
    assert_within([dw[t] for t in wsamp], ref, sab, xs[0] * y.shape[2] * y.shape[3], "dW")


def test_small_integers_are_exact():
    """Integer data whose partial sums stay below 2^24 are exact in f32 in any
    order, so the oracle must equal the f64 result bit for bit."""
    import torch
    rng = np.random.default_rng(0)
    x = rng.integers(-4, 5, (2, 3, 8, 7)).astype(np.float32)
    w = rng.integers(-3, 4, (5, 3, 3, 3)).astype(np.float32)
    y = O.conv2d_forward(x, w, 2, 1)
    g = rng.integers(-2, 3, y.shape).astype(np.float32)
    dx, dw = O.conv2d_backward(x, w, g, 2, 1)
    xt, wt, gt = (torch.from_numpy(a.astype(np.float64)) for a in (x, w, g))
    assert np.array_equal(y, torch.nn.functional.conv2d(xt, wt, stride=2, padding=1).numpy())
    assert np.array_equal(dx, torch.nn.grad.conv2d_input(xt.shape, wt, gt, stride=2,
                                                          padding=1).numpy())
    assert np.array_equal(dw, torch.nn.grad.conv2d_weight(xt, wt.shape, gt, stride=2,
                                                           padding=1).numpy())
    a = rng.integers(-5, 6, (13, 17)).astype(np.float32)
    b = rng.integers(-5, 6, (17, 11)).astype(np.float32)
    gm = rng.integers(-2, 3, (13, 11)).astype(np.float32)
    assert np.array_equal(O.matmul(a, b), a.astype(np.float64) @ b)
    da, db = O.matmul_vjp(a, b, gm)
    assert np.array_equal(da, gm.astype(np.float64) @ b.T.astype(np.float64))
    assert np.array_equal(db, a.T.astype(np.float64) @ gm.astype(np.float64))


def test_matmul_against_f64_and_closed_forms():
    a = synth.uniform(61, (37, 53))
    b = synth.uniform(62, (53, 29))
    aa, ab = np.abs(a).astype(np.float64), np.abs(b).astype(np.float64)
    assert_within(O.matmul(a, b), a.astype(np.float64) @ b, aa @ ab, 53, "C")
    # loss = sum(C): G = 1, so every row of dA equals the row sums of B and
    # every column of dB equals the column sums of A (tensor.rs:424-444).
    da, db = O.matmul_vjp(a, b, np.ones((37, 29), np.float32))
    assert np.all(da == da[0:1, :])
    assert np.all(db == db[:, 0:1])
    assert_within(da[0], b.astype(np.float64).sum(axis=1), ab.sum(axis=1), 29, "dA rows")
    assert_within(db[:, 0], a.astype(np.float64).sum(axis=0), aa.sum(axis=0), 37, "dB cols")


def test_sum_is_sequential():
    """tensor.rs:242-247: a left-to-right f32 fold (1e8 + 1 + ... stays 1e8)."""
    assert O.fsum(np.array([1e8] + [1.0] * 16, np.float32)) == 1e8
    assert O.fsum(np.array([1.0] * 16 + [1e8], np.float32)) == np.float32(1e8 + 16)
    assert O.fsum(np.zeros(0, np.float32)) == 0.0


# ---- SplitMix64 init --------------------------------------------------------

def test_splitmix_published_outputs():
    """SplitMix64 from state 0 (Vigna's reference splitmix64.c): the first three
    outputs are e220a8397b1dcdaf, 6e789e6aa1b965f4, 06c45d188009454f."""
    assert O.splitmix_outputs(0, 3) == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4,
                                        0x06C45D188009454F]
    # the vectorised generator of the synthetic inputs is the same stream
    assert synth.splitmix64(0, 3).tolist() == O.splitmix_outputs(0, 3)
    assert synth.splitmix64(123, 50).tolist() == O.splitmix_outputs(123, 50)


def test_seeded_initialization():
    """tests/conv2d.rs:145-155 and the mapping of conv2d.rs:57-58."""
    a = O.seeded_weights(3, 2, (3, 3), 7)
    b = O.seeded_weights(3, 2, (3, 3), 7)
    c = O.seeded_weights(3, 2, (3, 3), 8)
    assert np.array_equal(a, b) and not np.array_equal(a, c)
    assert np.all(np.abs(a) <= np.float32(1.0) / np.sqrt(np.float32(27.0)))
    z = np.array(O.splitmix_outputs(7, a.size), dtype=np.uint64)
    u = (z >> np.uint64(40)).astype(np.float32) / np.float32(16777216.0)
    bound = np.float32(1.0) / np.sqrt(np.float32(27.0))
    assert np.array_equal(a.ravel(), ((np.float32(2.0) * u - np.float32(1.0)) * bound))


# ---- geometry and element counts -------------------------------------------

U64MAX = 2 ** 64 - 1


def test_element_count():
    """tests/tensor.rs:4-25."""
    assert O.element_count([2, 3]) == 6
    assert O.element_count([]) == 1
    assert O.element_count([U64MAX, 0]) == 0
    with pytest.raises(O.OracleError):
        O.element_count([U64MAX, 2])
    with pytest.raises(O.OracleError):
        O.element_count([2 ** 63 - 1])


def test_geometry_errors():
    """tests/conv2d.rs:119-142 and the Geometry::new order of checks."""
    g = O.conv_geometry([1, 1, 3, 3], [1, 1, 2, 2], 1, 0)
    assert (g["oh"], g["ow"]) == (2, 2)
    bad = [([1, 1, 3, 3], [1, 0, 3, 3], 1, 0),   # zero weight dim
           ([1, 1, 3, 3], [1, 1, 1, 1], 0, 0),   # stride 0
           ([1, 1, 3], [1, 1, 1, 1], 1, 0),      # rank 3 input
           ([1, 2, 3, 3], [1, 1, 3, 3], 1, 0),   # channel mismatch
           ([1, 1, 2, 2], [1, 1, 3, 3], 1, 0),   # kernel exceeds padded input
           ([1, 1, 0, 2], [1, 1, 3, 3], 1, 0)]   # H = 0
    for xs, ws, st, p in bad:
        with pytest.raises(O.OracleError) as e:
            O.conv_geometry(xs, ws, st, p)
        assert e.value.code == O.INVALID_CONV
    with pytest.raises(O.OracleError) as e:
        O.conv_geometry([0, 1, 2, 2], [1, 1, 1, 1], 1, U64MAX // 2)
    assert e.value.code == O.SHAPE_OVERFLOW
    g = O.conv_geometry([0, 3, 4, 5], [2, 3, 3, 3], 1, 1)
    assert (g["batch"], g["oh"], g["ow"]) == (0, 4, 5)


# ---- planted mistakes must fail the pins -----------------------------------

MUTANTS = {
    1: "forward uses the flipped kernel (convolution instead of correlation)",
    2: "dX accumulates g*x instead of g*w (wrong operand)",
    3: "dA reads B transposed",
    4: "padded taps wrap to the opposite edge instead of being skipped",
}


@pytest.fixture(scope="module")
def mutant_libs(tmp_path_factory):
    import ctypes
    import os
    import subprocess
    d = tmp_path_factory.mktemp("mutants")
    src = os.path.join(os.path.dirname(O.__file__), "katsu_oracle.c")
    libs = {}
    for m in MUTANTS:
        out = str(d / f"libmut{m}.so")
        subprocess.run(["gcc", "-O1", "-ffp-contract=off", "-fPIC", "-shared",
                        f"-DKO_MUTANT={m}", src, "-o", out, "-lm"], check=True)
        libs[m] = ctypes.CDLL(out)
    return libs


def _with_lib(lib, fn, *a):
    saved = O._lib
    try:
        O._lib = lib
        O._lib.ko_conv2d_forward.argtypes = saved.ko_conv2d_forward.argtypes
        for name in ("ko_conv2d_backward", "ko_matmul_vjp", "ko_conv_geometry", "ko_matmul"):
            getattr(O._lib, name).argtypes = getattr(saved, name).argtypes
        return fn(*a)
    finally:
        O._lib = saved


def _pins_pass():
    """The cheap pins above, as one boolean."""
    try:
        test_known_forward_and_overlap_gradients()
        test_known_stride_and_padding()
        test_same_parent_accumulates_both_edges()
        test_rectangular_matmul()
        for case in CONV_CASES[:2]:
            test_conv_against_torch_f64(*case)
        test_matmul_against_f64_and_closed_forms()
        return True
    except AssertionError:
        return False


@pytest.mark.parametrize("m", sorted(MUTANTS))
def test_mutants_are_caught(m, mutant_libs):
    assert _pins_pass(), "the pins must pass on the real oracle"
    assert not _with_lib(mutant_libs[m], _pins_pass), f"mutant {m} not caught: {MUTANTS[m]}"
