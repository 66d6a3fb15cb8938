"""Parity helpers shared by the tests.

Error bound: an f32 dot product of length K evaluated in any order is within
gamma(K) * sum|a_i b_i| of the exact value, gamma(K) = K u / (1 - K u),
u = 2^-24 (Higham, Accuracy and Stability of Numerical Algorithms, 3.1).
The CPU oracle and the GPU both obey it, so they differ by at most
2 gamma(K) sum|a b| per element; that is the parity bar for every
floating-point comparison here.  Integer-valued known-answer tests are exact
in f32 and are compared with ==.

The sampled references below are an independent f64 formulation (numpy
slicing over a zero-padded copy, not the reference's visit loop); they pin
both the oracle and the GPU at sizes where a full CPU pass is too slow.
"""
import numpy as np

U = 2.0 ** -24


def gamma(k):
    k = float(k)
    return k * U / (1.0 - k * U)


def assert_within(got, ref, s, kred, what=""):
    """|got - ref| <= 2 gamma(kred) s elementwise."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    s = np.asarray(s, np.float64)
    assert got.shape == ref.shape, (what, got.shape, ref.shape)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    lim = 2.0 * gamma(kred) * s
    err = np.abs(got - ref)
    bad = err > lim
    if bad.any():
        idx = np.unravel_index(np.argmax(np.where(bad, err - lim, -np.inf)), err.shape)
        raise AssertionError(
            f"{what}: {int(bad.sum())}/{bad.size} elements beyond 2*gamma({kred})*S; "
            f"worst at {idx}: got {got[idx]!r} ref {ref[idx]!r} err {err[idx]:.3e} "
            f"bound {lim[idx]:.3e}")


def max_rel_mixed(a, b):
    """The reference's mixed metric (tests/conv2d.rs:5-13): the smallest tol
    with |x - y| <= tol * (1 + max(|x|, |y|)) for every element."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    if a.size == 0:
        return 0.0
    return float(np.max(np.abs(a - b) / (1.0 + np.maximum(np.abs(a), np.abs(b)))))


def out_hw(h, w, r, s, st, p):
    return (h + 2 * p - r) // st + 1, (w + 2 * p - s) // st + 1


def _pad(x, p):
    return np.pad(x.astype(np.float64), ((0, 0), (0, 0), (p, p), (p, p)))


def sample_fwd(x, w, st, p, samples):
    """Exact-f64 y[n,oc,oy,ox] and S = sum|x||w| at the sampled outputs."""
    xp = _pad(x, p)
    w64 = w.astype(np.float64)
    _, _, r, s = w.shape
    vals, sabs = [], []
    for n, oc, oy, ox in samples:
        patch = xp[n, :, oy * st:oy * st + r, ox * st:ox * st + s]
        vals.append(float(np.sum(patch * w64[oc])))
        sabs.append(float(np.sum(np.abs(patch) * np.abs(w64[oc]))))
    return np.array(vals), np.array(sabs)


def sample_dx(g, w, xshape, st, p, samples):
    """Exact-f64 dx[n,c,iy,ix] and S at the sampled inputs."""
    k, c_, r, s = w.shape
    _, _, oh, ow = g.shape
    g64 = g.astype(np.float64)
    w64 = w.astype(np.float64)
    vals, sabs = [], []
    for n, c, iy, ix in samples:
        acc = 0.0
        sa = 0.0
        for ky in range(r):
            ty = iy + p - ky
            if ty < 0 or ty % st or ty // st >= oh:
                continue
            oy = ty // st
            for kx in range(s):
                tx = ix + p - kx
                if tx < 0 or tx % st or tx // st >= ow:
                    continue
                ox = tx // st
                gv = g64[n, :, oy, ox]
                wv = w64[:, c, ky, kx]
                acc += float(np.dot(gv, wv))
                sa += float(np.dot(np.abs(gv), np.abs(wv)))
        vals.append(acc)
        sabs.append(sa)
    return np.array(vals), np.array(sabs)


def sample_dw(x, g, wshape, st, p, samples):
    """Exact-f64 dw[oc,c,ky,kx] and S at the sampled weights."""
    xp = _pad(x, p)
    g64 = g.astype(np.float64)
    _, _, oh, ow = g.shape
    vals, sabs = [], []
    for oc, c, ky, kx in samples:
        xs = xp[:, c, ky:ky + st * (oh - 1) + 1:st, kx:kx + st * (ow - 1) + 1:st]
        gv = g64[:, oc]
        vals.append(float(np.sum(xs * gv)))
        sabs.append(float(np.sum(np.abs(xs) * np.abs(gv))))
    return np.array(vals), np.array(sabs)


def random_samples(shape, count, seed):
    rng = np.random.default_rng(seed)
    return [tuple(int(rng.integers(0, d)) for d in shape) for _ in range(count)]


def edge_samples(shape):
    """Corners and edges of the spatial plane for the first/last batch and channel."""
    n, c, h, w = shape
    out = []
    for nn in {0, n - 1}:
        for cc in {0, c - 1}:
            for yy in {0, 1, h // 2, h - 2, h - 1}:
                for xx in {0, 1, w // 2, w - 2, w - 1}:
                    if 0 <= yy < h and 0 <= xx < w:
                        out.append((nn, cc, yy, xx))
    return out
