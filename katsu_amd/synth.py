"""Seeded synthetic inputs shared by the bench and the parity tests.

One SplitMix64 stream per tensor (the generator of the reference's
Conv2D::new_seeded, conv2d.rs:51-57), vectorised: the i-th output mixes
state seed + (i+1)*gamma.
  U[0,1):  u = (z >> 40) / 2^24            (exact in f32, conv2d.rs:57)
  U[-1,1): 2u - 1                          (exact)
  N(0,1):  Box-Muller in f64 on u1 = 1 - u(z_2i) in (0,1], u2 = u(z_2i+1)
  He-normal: N(0,1) * sqrt(2 / fan_in), rounded to f32.
Seeds used by the workloads: X=1, W=2, G=3, head=4.
"""
import numpy as np

GAMMA = np.uint64(0x9E3779B97F4A7C15)
M1 = np.uint64(0xBF58476D1CE4E5B9)
M2 = np.uint64(0x94D049BB133111EB)

SEED_X, SEED_W, SEED_G, SEED_HEAD = 1, 2, 3, 4


def splitmix64(seed, count):
    """First `count` outputs of SplitMix64 started from state `seed`."""
    with np.errstate(over="ignore"):
        idx = np.arange(1, count + 1, dtype=np.uint64)
        z = np.uint64(seed) + idx * GAMMA
        z = (z ^ (z >> np.uint64(30))) * M1
        z = (z ^ (z >> np.uint64(27))) * M2
        z = z ^ (z >> np.uint64(31))
    return z


def unit_uniform(seed, count):
    z = splitmix64(seed, count)
    return (z >> np.uint64(40)).astype(np.float32) / np.float32(16777216.0)


def uniform(seed, shape, lo=-1.0, hi=1.0):
    n = int(np.prod(shape))
    u = unit_uniform(seed, n)
    if (lo, hi) == (-1.0, 1.0):
        out = np.float32(2.0) * u - np.float32(1.0)
    elif (lo, hi) == (0.0, 1.0):
        out = u
    else:
        out = (lo + (hi - lo) * u.astype(np.float64)).astype(np.float32)
    return out.reshape(shape)


def normal(seed, shape, scale=1.0):
    n = int(np.prod(shape))
    z = splitmix64(seed, 2 * n)
    u = (z >> np.uint64(40)).astype(np.float64) / 16777216.0
    u1 = 1.0 - u[0::2]
    u2 = u[1::2]
    v = np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)
    return (v * scale).astype(np.float32).reshape(shape)


def he_normal(seed, shape):
    fan_in = int(np.prod(shape[1:]))
    return normal(seed, shape, np.sqrt(2.0 / fan_in))


# The BASELINE workloads.  Each entry: input shape, weight shape, stride,
# padding, input law.
CONV_CONFIGS = {
    "c1_example": dict(x=(1, 3, 224, 224), w=(8, 3, 3, 3), stride=1, pad=1, law="u11"),
    "c3_resnet": dict(x=(32, 64, 56, 56), w=(64, 64, 3, 3), stride=1, pad=1, law="u11"),
    "c4a_down3x3": dict(x=(32, 128, 28, 28), w=(256, 128, 3, 3), stride=2, pad=1, law="n01"),
    "c4b_down1x1": dict(x=(32, 128, 28, 28), w=(256, 128, 1, 1), stride=2, pad=0, law="n01"),
    "c5_stem": dict(x=(64, 3, 224, 224), w=(64, 3, 7, 7), stride=2, pad=3, law="u01"),
}


def conv_inputs(cfg):
    """(x, w) for one of CONV_CONFIGS (or a dict of the same form)."""
    c = CONV_CONFIGS[cfg] if isinstance(cfg, str) else cfg
    law = c["law"]
    if law == "u11":
        x = uniform(SEED_X, c["x"])
    elif law == "u01":
        x = uniform(SEED_X, c["x"], 0.0, 1.0)
    else:
        x = normal(SEED_X, c["x"])
    w = he_normal(SEED_W, c["w"])
    return x, w


def out_shape(c):
    n, _, h, w = c["x"]
    k, _, r, s = c["w"]
    st, p = c["stride"], c["pad"]
    return (n, k, (h + 2 * p - r) // st + 1, (w + 2 * p - s) // st + 1)


def conv_flops(c):
    """Algorithmic FLOP of one pass (dense taps, padding counted)."""
    n, k, oh, ow = out_shape(c)
    _, cin, r, s = c["w"]
    return 2 * n * k * oh * ow * cin * r * s
