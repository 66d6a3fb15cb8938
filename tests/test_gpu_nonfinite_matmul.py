"""Non-finite inputs: the GPU matmul, its VJP and the sum against the CPU oracle.

The reference multiplies every product of a matmul and of both VJP products
(crates/katsu-core/src/tensor.rs:264-273, 424-444): no term is skipped, so
NaN and Inf follow f32 arithmetic over all of them (docs/api.md:34).  The
GPU kernels must give the same NaN, +Inf and -Inf masks exactly, and every
finite value within the f32 dot-product bound.  Zero-filled tile edges, split-K
partial sums, the register-direct kernel, the one-launch VJP, the aliased
a@a VJP and beta = 1 over a finite pending buffer each see the planted values.

Inf, -Inf and NaN are planted in A, B and G at tile corners, at the last row
and column (partial-tile edges where the shape is not a tile multiple) and in
the interior; with U[-1,1) data and these depths nothing overflows, so the
class of each sum does not depend on its order.  The outputs are filled with
NaN before every beta = 0 call: beta = 0 must not read them."""
import numpy as np
import pytest

from katsu_amd import synth
from oracle import oracle as O
from tests.parity import assert_within

pytestmark = pytest.mark.gpu

INF = np.float32(np.inf)
NAN = np.float32(np.nan)


def _t(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dev)


def _plant3(a, where):
    """+Inf, -Inf and NaN at three positions of the 2-D array `a`."""
    r, c = a.shape
    (i0, j0), (i1, j1), (i2, j2) = where(r, c)
    a[i0, j0] = INF
    a[i1, j1] = -INF
    a[i2, j2] = NAN
    return a


def _finite0(a):
    return np.where(np.isfinite(a), np.abs(a), 0).astype(np.float64)


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
    assert fin.any() and (~fin).any(), f"{what}: the planted values must reach some outputs only"
    assert_within(got[fin], ref[fin], s[fin], kred, what)


def _operands(m, k, n):
    a = _plant3(synth.uniform(21, (m, k)),
                lambda r, c: ((0, 0), (r - 1, c - 1), (r // 2, c // 3)))
    b = _plant3(synth.uniform(22, (k, n)),
                lambda r, c: ((0, c - 1), (r - 1, 0), (r // 2, c // 2)))
    g = _plant3(synth.uniform(23, (m, n)),
                lambda r, c: ((0, 0), (r - 1, c - 1), (r // 3, c // 2)))
    return a, b, g


# (m, k, n) and the kernels they take:
#   37 x 41 x 29       the generic engine (dimensions not multiples of 4)
#   512^3              32 x 32 tiles; the VJP's dA and dB blocks in one launch
#   64 x 1000 x 64     64-tiles with K split six ways + the fixed-order reduce;
#                      one-launch VJP on 64-tiles
#   1024 x 100 x 1024  64-tiles; the VJP's two products split K eight ways
#   1024^3             the register-direct kernels (forward and one-launch VJP)
#   2048 x 64 x 2048   128 x 128 tiles with edge tiles in K; split VJP
SHAPES = [(37, 41, 29), (512, 512, 512), (64, 1000, 64), (1024, 100, 1024),
          (1024, 1024, 1024), (2048, 64, 2048)]


@pytest.mark.parametrize("m,k,n", SHAPES)
def test_matmul_and_vjp_nonfinite(m, k, n, dev):
    import torch

    from katsu_amd import ops
    print(f"\nmatmul nonfinite m={m} k={k} n={n}", flush=True)
    a, b, g = _operands(m, k, n)
    ad, bd, gd = _t(a, dev), _t(b, dev), _t(g, dev)
    c = torch.full((m, n), float("nan"), device=dev)
    ops.gemm(ad, bd, m, n, k, out=c)
    # beta = 1 into finite pending buffers (tensor.rs:427-443 add into them).
    da0 = synth.uniform(24, (m, k))
    db0 = synth.uniform(25, (k, n))
    da, db = _t(da0, dev), _t(db0, dev)
    ops.matmul_vjp(ad, bd, gd, da, db)
    torch.cuda.synchronize()
    da_ref, db_ref = O.matmul_vjp(a, b, g, da0.copy(), db0.copy())
    fa, fb, fg = _finite0(a), _finite0(b), _finite0(g)
    _check(c.cpu().numpy(), O.matmul(a, b), fa @ fb, k, "C")
    _check(da.cpu().numpy(), da_ref, fg @ fb.T + np.abs(da0), n + 1, "dA")
    _check(db.cpu().numpy(), db_ref, fa.T @ fg + np.abs(db0), m + 1, "dB")


@pytest.mark.parametrize("m,k,n", [(37, 41, 29), (2048, 64, 2048), (1024, 100, 1024)])
@pytest.mark.parametrize("ta,tb", [(0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("beta", [0.0, 1.0])
def test_gemm_transposes_nonfinite(m, k, n, ta, tb, beta, dev):
    """The GEMM entry point with transposed operands (the seams of dA = G.B^T
    and dB = A^T.G) on every tile size; beta = 1 over a finite buffer, beta = 0
    over NaN.  Checked against the oracle's matmul of the materialised
    transposes: the same products, so the same classes."""
    import torch

    from katsu_amd import ops
    print(f"\ngemm nonfinite m={m} k={k} n={n} ta={ta} tb={tb} beta={beta}", flush=True)
    opa = _plant3(synth.uniform(31, (m, k)),
                  lambda r, c: ((0, c - 1), (r - 1, 0), (r // 2, c // 2)))
    opb = _plant3(synth.uniform(32, (k, n)),
                  lambda r, c: ((r - 1, c - 1), (0, 0), (r // 3, c // 2)))
    a = np.ascontiguousarray(opa.T) if ta else opa
    b = np.ascontiguousarray(opb.T) if tb else opb
    c0 = synth.uniform(33, (m, n))
    c = _t(c0, dev) if beta else torch.full((m, n), float("nan"), device=dev)
    ops.gemm(_t(a, dev), _t(b, dev), m, n, k, bool(ta), bool(tb), out=c, beta=beta)
    torch.cuda.synchronize()
    ref = O.matmul(opa, opb)
    s = _finite0(opa) @ _finite0(opb)
    if beta:
        ref = (c0 + ref).astype(np.float32)
        s = s + np.abs(c0)
    _check(c.cpu().numpy(), ref, s, k + 1, f"ta={ta} tb={tb} beta={beta}")


@pytest.mark.parametrize("n", [2, 64, 512])
def test_aliased_vjp_nonfinite(n, dev):
    """a@a with A and B the same node: dA and dB accumulate into one pending
    buffer, dA first (tensor.rs:418-445; tests/autograd.rs:98-103)."""
    import torch

    from katsu_amd import ops
    a = synth.uniform(41, (n, n))
    a[0, 0] = INF
    a[n - 1, n - 1] = -INF
    if n > 2:
        a[n // 2, n // 3] = NAN
    g = synth.uniform(42, (n, n))
    g[n - 1, 0] = NAN if n > 2 else INF
    p0 = synth.uniform(43, (n, n))
    ad = _t(a, dev)
    pend = _t(p0, dev)
    ops.matmul_vjp(ad, ad, _t(g, dev), pend, pend)
    torch.cuda.synchronize()
    ref = p0.copy()
    O.matmul_vjp(a, a, g, ref, ref)
    fa, fg = _finite0(a), _finite0(g)
    s = fg @ fa.T + fa.T @ fg + np.abs(p0)
    got = pend.cpu().numpy()
    for name, mask in (("NaN", np.isnan), ("+Inf", np.isposinf), ("-Inf", np.isneginf)):
        assert np.array_equal(mask(got), mask(ref)), f"aliased VJP n={n}: {name} mask"
    fin = np.isfinite(ref)
    assert_within(got[fin], ref[fin], s[fin], 2 * n + 1, f"aliased VJP n={n}")


@pytest.mark.parametrize("size", [7, 1000, 1 << 20])
@pytest.mark.parametrize("plant", ["+inf", "-inf", "both", "nan", "none"])
def test_sum_nonfinite(size, plant, dev):
    """Tensor::sum (tensor.rs:242-247) on the GPU's fixed tree: the class of
    the result is the oracle's sequential sum's; a finite result is within
    the f32 bound."""
    import torch

    from katsu_amd import ops
    x = synth.uniform(51, (size,))
    if plant in ("+inf", "both"):
        x[size // 3] = INF
    if plant in ("-inf", "both"):
        x[size - 1] = -INF
    if plant == "nan":
        x[0] = NAN
    got = float(ops.sum(_t(x, dev)).cpu().numpy()[0])
    torch.cuda.synchronize()
    ref = O.fsum(x)
    for f in (np.isnan, np.isposinf, np.isneginf):
        assert bool(f(got)) == bool(f(ref)), (plant, size, got, ref)
    if np.isfinite(ref):
        assert_within(np.array([got]), np.array([ref]), np.array([np.abs(x).sum()]), size,
                      "sum")
