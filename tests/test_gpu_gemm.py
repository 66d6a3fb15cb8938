"""GPU parity of matmul and its VJPs against the CPU oracle (through the C ABI)."""
import numpy as np
import pytest

from katsu_amd import synth
from oracle import oracle as O
from tests.parity import assert_within

pytestmark = pytest.mark.gpu


def _t(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dev)


def test_rectangular_kat_exact(dev):
    """tests/tensor.rs:41-48."""
    from katsu_amd import ops
    a = _t([[1, 2, 3], [4, 5, 6]], dev)
    b = _t([[7, 8], [9, 10], [11, 12]], dev)
    assert ops.matmul(a, b).cpu().numpy().ravel().tolist() == [58, 64, 139, 154]


def test_same_parent_accumulates_both_edges_exact(dev):
    """tests/autograd.rs:98-103: a@a, loss sum -> grad [7, 11, 9, 13]; dA and dB
    accumulate into one pending buffer, dA first."""
    import torch

    from katsu_amd import ops
    a = _t([[1, 2], [3, 4]], dev)
    pend = torch.zeros_like(a)
    ops.matmul_vjp(a, a, torch.ones((2, 2), device=dev), pend, pend)
    assert pend.cpu().numpy().ravel().tolist() == [7, 11, 9, 13]


SHAPES = [(1, 1, 1), (2, 3, 2), (17, 5, 33), (33, 257, 31), (130, 70, 129), (128, 128, 128),
          (129, 16, 300), (64, 1000, 64), (3, 200, 7), (256, 37, 384)]


@pytest.mark.parametrize("m,k,n", SHAPES)
def test_matmul_and_vjp_parity(m, k, n, dev):
    import torch

    from katsu_amd import ops
    a = synth.uniform(1, (m, k))
    b = synth.uniform(2, (k, n))
    g = synth.uniform(3, (m, n))
    c = ops.matmul(_t(a, dev), _t(b, dev))
    da0 = synth.uniform(4, (m, k))  # non-zero pending values: the VJP accumulates
    db0 = synth.uniform(5, (k, n))
    da = _t(da0, dev)
    db = _t(db0, dev)
    ops.matmul_vjp(_t(a, dev), _t(b, dev), _t(g, dev), da, db)
    torch.cuda.synchronize()
    aa, ab, ag = np.abs(a).astype(np.float64), np.abs(b).astype(np.float64), np.abs(g)
    assert_within(c.cpu().numpy(), O.matmul(a, b), aa @ ab, k, "C")
    da_ref, db_ref = O.matmul_vjp(a, b, g, da0.copy(), db0.copy())
    # pending + sum: one more rounding of the pending add on both sides.
    assert_within(da.cpu().numpy(), da_ref, ag @ ab.T + np.abs(da0), n + 1, "dA")
    assert_within(db.cpu().numpy(), db_ref, aa.T @ ag + np.abs(db0), m + 1, "dB")


# (m, n, k): unaligned (the generic engine), then multiples of 4 (the
# dedicated GEMM: 64-tiles with split-K, a long split-K reduction, 128-tiles
# with edge tiles, 32-tiles at 512 deep), then the register-direct GEMM
# (64-tiles, K = 1024 in four wave quarters; tiles in patches of four tile
# rows, or in column order when the tile rows are not a multiple of four).
@pytest.mark.parametrize("m,n,k", [(70, 45, 131), (72, 44, 132), (128, 96, 2048),
                                   (516, 260, 68), (1024, 512, 1024), (512, 512, 512),
                                   (256, 640, 512), (192, 2752, 1024)])
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_all_transposes_beta(ta, tb, m, n, k, dev):
    import torch

    from katsu_amd import ops
    a = synth.uniform(7, (k, m) if ta else (m, k))
    b = synth.uniform(8, (n, k) if tb else (k, n))
    c0 = synth.uniform(9, (m, n))
    opa = a.T if ta else a
    opb = b.T if tb else b
    for beta in (0.0, 1.0):
        c = _t(c0, dev)
        ops.gemm(_t(a, dev), _t(b, dev), m, n, k, bool(ta), bool(tb), out=c, beta=beta)
        torch.cuda.synchronize()
        ref = opa.astype(np.float64) @ opb.astype(np.float64) + beta * c0
        s = np.abs(opa).astype(np.float64) @ np.abs(opb) + beta * np.abs(c0)
        assert_within(c.cpu().numpy(), ref, s, k + 1, f"ta={ta} tb={tb} beta={beta}")


def test_empty_and_k_zero(dev):
    """tests/tensor.rs:65-86 and autograd.rs:106-116: [2,0]@[0,3] gives six
    zeros; m == 0 gives an empty result; empty VJPs leave grads untouched."""
    import torch

    from katsu_amd import ops
    c = ops.gemm(torch.zeros((2, 0), device=dev), torch.zeros((0, 3), device=dev), 2, 3, 0,
                 out=torch.full((2, 3), 5.0, device=dev))
    assert c.cpu().numpy().ravel().tolist() == [0.0] * 6
    c1 = ops.gemm(torch.zeros((2, 0), device=dev), torch.zeros((0, 3), device=dev), 2, 3, 0,
                  out=torch.full((2, 3), 5.0, device=dev), beta=1.0)
    assert c1.cpu().numpy().ravel().tolist() == [5.0] * 6
    e = ops.matmul(torch.zeros((0, 2), device=dev), torch.zeros((2, 3), device=dev))
    assert tuple(e.shape) == (0, 3)


@pytest.mark.parametrize("n", [512, 1024])
def test_config2_full_parity(n, dev):
    """Config 2 at 512 and 1024: full oracle comparison of C, dA, dB with
    loss = sum(C) (G = 1) and with a random G."""
    import torch

    from katsu_amd import ops
    a = synth.uniform(synth.SEED_X, (n, n))
    b = synth.uniform(synth.SEED_W, (n, n))
    ad, bd = _t(a, dev), _t(b, dev)
    c = ops.matmul(ad, bd).cpu().numpy()
    aa, ab = np.abs(a).astype(np.float64), np.abs(b).astype(np.float64)
    assert_within(c, O.matmul(a, b), aa @ ab, n, "C")
    for g in (np.ones((n, n), np.float32), synth.uniform(synth.SEED_G, (n, n))):
        da = torch.zeros_like(ad)
        db = torch.zeros_like(bd)
        ops.matmul_vjp(ad, bd, _t(g, dev), da, db)
        torch.cuda.synchronize()
        da_ref, db_ref = O.matmul_vjp(a, b, g)
        ag = np.abs(g).astype(np.float64)
        assert_within(da.cpu().numpy(), da_ref, ag @ ab.T, n, "dA")
        assert_within(db.cpu().numpy(), db_ref, aa.T @ ag, n, "dB")


def test_config2_4096_sampled_rows(dev):
    """Config 2 at 4096: every output row of C and dA (and row p of dB) is an
    independent unit, so sampled rows are compared to the oracle on those rows."""
    import torch

    from katsu_amd import ops
    n = 4096
    a = synth.uniform(synth.SEED_X, (n, n))
    b = synth.uniform(synth.SEED_W, (n, n))
    g = np.ones((n, n), np.float32)
    ad, bd = _t(a, dev), _t(b, dev)
    c = ops.matmul(ad, bd)
    da = torch.zeros_like(ad)
    db = torch.zeros_like(bd)
    ops.matmul_vjp(ad, bd, _t(g, dev), da, db)
    torch.cuda.synchronize()
    c, da, db = c.cpu().numpy(), da.cpu().numpy(), db.cpu().numpy()
    rows = [0, 1, 2047, 4094, 4095]
    aa, ab = np.abs(a).astype(np.float64), np.abs(b).astype(np.float64)
    assert_within(c[rows], O.matmul(a[rows], b), aa[rows] @ ab, n, "C rows")
    da_ref, _ = O.matmul_vjp(a[rows], b, g[rows])
    assert_within(da[rows], da_ref, np.ones((len(rows), n)) @ ab.T, n, "dA rows")
    # dB row p = sum_i A[i,p] G[i,:]; with G = 1 every column of a row is equal
    # (the closed form of tensor.rs:437-443 under loss = sum(C)).
    col = np.abs(a).astype(np.float64).sum(axis=0)
    ref = a.astype(np.float64).sum(axis=0)
    for p in rows:
        assert_within(db[p], np.full(n, ref[p]), np.full(n, col[p]), n, f"dB row {p}")


@pytest.mark.parametrize("m,k,n", [(512, 512, 512), (1024, 1024, 1024), (256, 512, 768),
                                   (64, 128, 96), (1000, 36, 52)])
@pytest.mark.parametrize("beta", [0.0, 1.0])
def test_vjp_entry_matches_two_gemms(m, k, n, beta, dev):
    """katsu_hip_matmul_vjp_f32_dev (dA and dB as one launch when both tile
    plans agree, else two) agrees with the two GEMM calls within the f32
    dot-product bound (its k-sums may be grouped differently), and gives the
    same bits when called again."""
    import torch

    from katsu_amd import ops
    from katsu_amd._abi import lib
    a = _t(synth.uniform(61, (m, k)), dev)
    b = _t(synth.uniform(62, (k, n)), dev)
    g = _t(synth.uniform(63, (m, n)), dev)
    da0 = _t(synth.uniform(64, (m, k)), dev)
    db0 = _t(synth.uniform(65, (k, n)), dev)
    da, db = da0.clone(), db0.clone()
    rc = lib().katsu_hip_matmul_vjp_f32_dev(a.data_ptr(), b.data_ptr(), g.data_ptr(),
                                            da.data_ptr(), db.data_ptr(), m, k, n, beta, beta,
                                            ops._stream())
    assert rc == 0
    da2, db2 = da0.clone(), db0.clone()
    assert lib().katsu_hip_matmul_vjp_f32_dev(a.data_ptr(), b.data_ptr(), g.data_ptr(),
                                              da2.data_ptr(), db2.data_ptr(), m, k, n, beta,
                                              beta, ops._stream()) == 0
    ra, rb = da0.clone(), db0.clone()
    ops.gemm(g, b, m, k, n, trans_b=True, out=ra, beta=beta)
    ops.gemm(a, g, k, n, m, trans_a=True, out=rb, beta=beta)
    torch.cuda.synchronize()
    assert torch.equal(da, da2) and torch.equal(db, db2)
    ab, bb, gb = (t.abs() for t in (a, b, g))
    sa = ops.gemm(gb, bb, m, k, n, trans_b=True) + beta * da0.abs()
    sb = ops.gemm(ab, gb, k, n, m, trans_a=True) + beta * db0.abs()
    torch.cuda.synchronize()
    # Two f32 evaluations of the same sum: each within the bound of the exact
    # value, so within twice the bound of each other.
    assert_within(da.cpu().numpy(), ra.cpu().numpy().astype(np.float64),
                  2 * sa.cpu().numpy().astype(np.float64), n + 1, "dA")
    assert_within(db.cpu().numpy(), rb.cpu().numpy().astype(np.float64),
                  2 * sb.cpu().numpy().astype(np.float64), m + 1, "dB")


def test_vjp_entry_null_output(dev):
    """A NULL dA or dB skips that product and leaves the other as the GEMM."""
    import torch

    from katsu_amd import ops
    from katsu_amd._abi import lib
    m = k = n = 512
    a, b, g = (_t(synth.uniform(71 + i, (512, 512)), dev) for i in range(3))
    for which in (0, 1):
        out = torch.zeros((512, 512), device=dev)
        ptrs = (out.data_ptr(), None) if which == 0 else (None, out.data_ptr())
        assert lib().katsu_hip_matmul_vjp_f32_dev(a.data_ptr(), b.data_ptr(), g.data_ptr(),
                                                  *ptrs, m, k, n, 0.0, 0.0, ops._stream()) == 0
        ref = ops.gemm(g, b, m, k, n, trans_b=True) if which == 0 else \
            ops.gemm(a, g, k, n, m, trans_a=True)
        torch.cuda.synchronize()
        assert torch.equal(out, ref)
