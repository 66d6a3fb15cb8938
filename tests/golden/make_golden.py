"""Writes the golden fixtures of tests/golden (run from the repository root:
``python tests/golden/make_golden.py``).

Every fixture is data: seeded inputs, the CPU oracle's outputs (oracle/, the
C restatement of the reference's loops, built with -ffp-contract=off), and
the largest deviation of those outputs from an independent float64
evaluation (torch CPU conv/grad routines, numpy matmul), stated relative to
the f32 dot-product bound 2*gamma(K)*sum|a*b| (which must stay <= 1).

  reference_kats.json  the reference's known-answer tests as input/expected
                       pairs, each with the test file:line it comes from
  conv_*.npz           one seeded Conv2D case per (filter, stride, padding)
                       of the BASELINE configs, at small spatial sizes:
                       x, w, g -> y, dx, dw
  matmul_*.npz         Tensor::matmul and its VJP (random G and G = 1):
                       a, b, g -> c, da, db
  example_1b.json      the repository example (examples/conv2d/main.rs:5-20):
                       its loss, first dX values, dW, and SHA-256 digests of
                       the full y and dX bit patterns
  MANIFEST.json        SHA-256 of every fixture file

The reference itself is not run (no Rust toolchain here); the oracle is
pinned against the reference's own tests in tests/test_oracle.py, and these
fixtures freeze its outputs so both the oracle and the HIP path are checked
against the same bytes.
"""
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from katsu_amd import synth  # noqa: E402
from oracle import oracle as O  # noqa: E402

U = 2.0 ** -24


def gamma(k):
    return k * U / (1.0 - k * U)


def rel_to_bound(got, ref64, s64, kred):
    lim = 2.0 * gamma(max(kred, 1)) * s64
    err = np.abs(got.astype(np.float64) - ref64)
    with np.errstate(divide="ignore", invalid="ignore"):
        r = np.where(lim > 0, err / lim, np.where(err > 0, np.inf, 0.0))
    return float(r.max()) if r.size else 0.0


# (name, x shape, w shape, stride, pad, x law, G law, BASELINE config it stands for)
CONV_CASES = [
    ("conv_c1_3x3_s1p1", (1, 3, 12, 13), (8, 3, 3, 3), 1, 1, "u11", "2y", "config 1"),
    ("conv_c3_3x3_s1p1", (2, 16, 8, 9), (16, 16, 3, 3), 1, 1, "u11", "n01", "config 3"),
    ("conv_c4a_3x3_s2p1", (2, 12, 9, 10), (20, 12, 3, 3), 2, 1, "n01", "n01", "config 4a"),
    ("conv_c4b_1x1_s2p0", (2, 12, 9, 10), (20, 12, 1, 1), 2, 0, "n01", "n01", "config 4b"),
    ("conv_c5_7x7_s2p3", (2, 3, 20, 17), (8, 3, 7, 7), 2, 3, "u01", "n01", "config 5"),
    ("conv_rect_2x3_s1p1", (2, 5, 7, 9), (6, 5, 2, 3), 1, 1, "u11", "n01", "tests/conv2d.rs:46-87 shapes"),
]

# (name, m, k, n, G law)
MM_CASES = [
    ("matmul_37x29x41_randg", 37, 29, 41, "n01"),
    ("matmul_48x40x56_ones", 48, 40, 56, "ones"),
]


def x_of(law, seed, shape):
    if law == "u11":
        return synth.uniform(seed, shape)
    if law == "u01":
        return synth.uniform(seed, shape, 0.0, 1.0)
    return synth.normal(seed, shape)


def conv_case(name, xs, ws, st, p, xlaw, glaw, stands_for):
    import torch
    x = x_of(xlaw, synth.SEED_X, xs)
    w = synth.he_normal(synth.SEED_W, ws)
    y = O.conv2d_forward(x, w, st, p)
    if glaw == "2y":
        g = (y + y).astype(np.float32)  # sum(Y*Y): two +=1*Y edges into zero
    else:
        g = synth.normal(synth.SEED_G, y.shape)
    dx, dw = O.conv2d_backward(x, w, g, st, p)
    # independent f64 evaluation
    xt, wt, gt = (torch.from_numpy(a).double() for a in (x, w, g))
    y64 = torch.nn.functional.conv2d(xt, wt, stride=st, padding=p).numpy()
    dx64 = torch.nn.grad.conv2d_input(xt.shape, wt, gt, stride=st, padding=p).numpy()
    dw64 = torch.nn.grad.conv2d_weight(xt, wt.shape, gt, stride=st, padding=p).numpy()
    ax, aw, ag = (torch.from_numpy(np.abs(a)).double() for a in (x, w, g))
    ys = torch.nn.functional.conv2d(ax, aw, stride=st, padding=p).numpy()
    dxs = torch.nn.grad.conv2d_input(ax.shape, aw, ag, stride=st, padding=p).numpy()
    dws = torch.nn.grad.conv2d_weight(ax, aw.shape, ag, stride=st, padding=p).numpy()
    k, c, r, s = ws
    n, _, oh, ow = y.shape
    checks = {
        "y": rel_to_bound(y, y64, ys, c * r * s),
        "dx": rel_to_bound(dx, dx64, dxs, k * r * s),
        "dw": rel_to_bound(dw, dw64, dws, n * oh * ow),
    }
    assert all(v <= 1.0 for v in checks.values()), (name, checks)
    np.savez(os.path.join(HERE, name + ".npz"), x=x, w=w, g=g, y=y, dx=dx, dw=dw,
             stride=np.int64(st), pad=np.int64(p))
    return {"file": name + ".npz", "stands_for": stands_for, "x_law": xlaw,
            "g": "2*y (loss sum(y*y))" if glaw == "2y" else "N(0,1) seed 3",
            "w": "He-normal seed 2", "stride": st, "pad": p,
            "oracle_vs_f64_over_bound": checks}


def mm_case(name, m, k, n, glaw):
    a = synth.uniform(synth.SEED_X, (m, k))
    b = synth.uniform(synth.SEED_W, (k, n))
    g = np.ones((m, n), np.float32) if glaw == "ones" else synth.normal(synth.SEED_G, (m, n))
    c = O.matmul(a, b)
    da, db = O.matmul_vjp(a, b, g)
    a64, b64, g64 = (v.astype(np.float64) for v in (a, b, g))
    checks = {
        "c": rel_to_bound(c, a64 @ b64, np.abs(a64) @ np.abs(b64), k),
        "da": rel_to_bound(da, g64 @ b64.T, np.abs(g64) @ np.abs(b64).T, n),
        "db": rel_to_bound(db, a64.T @ g64, np.abs(a64).T @ np.abs(g64), m),
    }
    assert all(v <= 1.0 for v in checks.values()), (name, checks)
    np.savez(os.path.join(HERE, name + ".npz"), a=a, b=b, g=g, c=c, da=da, db=db)
    return {"file": name + ".npz", "m": m, "k": k, "n": n,
            "g": "ones (loss sum(C))" if glaw == "ones" else "N(0,1) seed 3",
            "oracle_vs_f64_over_bound": checks}


def example_1b():
    """examples/conv2d/main.rs:5-20: pixels (i % 256)/255, Conv2D::new_seeded(3, 8,
    (3, 3), 1, 1, 123), loss = sum(y*y), G = 2y."""
    x = (np.arange(3 * 224 * 224) % 256).astype(np.float32) / np.float32(255.0)
    x = x.reshape(1, 3, 224, 224)
    w = O.seeded_weights(3, 8, (3, 3), 123)
    y = O.conv2d_forward(x, w, 1, 1)
    loss = O.fsum((y * y).astype(np.float32))
    g = (y + y).astype(np.float32)
    dx, dw = O.conv2d_backward(x, w, g, 1, 1)
    sha = lambda a: hashlib.sha256(np.ascontiguousarray(a, np.float32).tobytes()).hexdigest()
    return {
        "source": "examples/conv2d/main.rs:5-20 (prints these values, asserts none)",
        "x": "(i % 256) / 255 over [1,3,224,224]",
        "w": "Conv2D::new_seeded(3, 8, (3, 3), 1, 1, 123), conv2d.rs:35-61",
        "loss_sum_y_sq": loss,
        "dx_first5": [float(v) for v in dx.ravel()[:5]],
        "y_first5": [float(v) for v in y.ravel()[:5]],
        "w": w.ravel().tolist(),
        "dw": dw.ravel().tolist(),
        "sha256_y_f32": sha(y),
        "sha256_dx_f32": sha(dx),
        "y_shape": list(y.shape),
    }


def reference_kats():
    """The reference's known answers, as data (file:line of each)."""
    return [
        {"src": "tests/conv2d.rs:16-43", "op": "conv2d",
         "x": {"shape": [1, 1, 3, 3], "data": list(range(1, 10))},
         "w": {"shape": [1, 1, 2, 2], "data": [1, 2, 3, 4]}, "stride": 1, "pad": 0,
         "g": "ones", "y": [37, 47, 67, 77], "dx": [1, 3, 2, 4, 10, 6, 3, 7, 4],
         "dw": [12, 16, 24, 28]},
        {"src": "tests/conv2d.rs:172-179", "op": "conv2d",
         "x": {"shape": [1, 1, 3, 3], "data": list(range(1, 10))},
         "w": {"shape": [1, 1, 2, 2], "data": [1, 2, 3, 4]}, "stride": 2, "pad": 1,
         "y": [4, 18, 36, 77]},
        {"src": "tests/conv2d.rs:90-106", "op": "conv2d",
         "x": {"shape": [1, 1, 1, 1], "data": [5]}, "w": {"shape": [1, 1, 1, 1], "data": [2]},
         "stride": 1, "pad": 0, "g": "ones", "y": [10], "dx": [2], "dw": [5]},
        {"src": "tests/tensor.rs:41-48", "op": "matmul",
         "a": {"shape": [2, 3], "data": [1, 2, 3, 4, 5, 6]},
         "b": {"shape": [3, 2], "data": [7, 8, 9, 10, 11, 12]}, "c": [58, 64, 139, 154]},
        {"src": "tests/autograd.rs:98-103", "op": "matmul_vjp_aliased",
         "a": {"shape": [2, 2], "data": [1, 2, 3, 4]}, "g": "ones",
         "pending_after": [7, 11, 9, 13]},
    ]


def main():
    meta = {"conv": [], "matmul": []}
    for case in CONV_CASES:
        meta["conv"].append(conv_case(*case))
    for case in MM_CASES:
        meta["matmul"].append(mm_case(*case))
    with open(os.path.join(HERE, "example_1b.json"), "w") as f:
        json.dump(example_1b(), f, indent=1)
    with open(os.path.join(HERE, "reference_kats.json"), "w") as f:
        json.dump(reference_kats(), f, indent=1)
    files = sorted(fn for fn in os.listdir(HERE)
                   if fn.endswith((".npz", ".json")) and fn != "MANIFEST.json")
    meta["sha256"] = {fn: hashlib.sha256(open(os.path.join(HERE, fn), "rb").read()).hexdigest()
                      for fn in files}
    with open(os.path.join(HERE, "MANIFEST.json"), "w") as f:
        json.dump(meta, f, indent=1)
    print(json.dumps({k: len(v) for k, v in meta.items()}))


if __name__ == "__main__":
    main()
