"""Host-buffer ("drop-in") entry points over the C ABI.

These are the calls a Rust binding of katsu-core would make with its
``&[f32]`` slices: inputs are copied to the device, the gfx950 kernels run,
outputs are copied back before the call returns.
"""
import ctypes

import numpy as np

from ._abi import check, geometry, lib


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _p(a):
    return ctypes.c_void_p(a.ctypes.data) if a.size else ctypes.c_void_p(0)


def conv2d_forward(x, w, stride, pad):
    x, w = _f32(x), _f32(w)
    g = geometry(*x.shape, w.shape[0], w.shape[2], w.shape[3], stride, pad)
    if w.shape[1] != x.shape[1]:
        raise ValueError("input channels must match weights")
    y = np.empty((g.n, g.k, g.oh, g.ow), np.float32)
    check(lib().katsu_hip_conv2d_fwd_f32(_p(x), _p(w), _p(y), ctypes.byref(g)), "conv2d_fwd")
    return y


def conv2d_backward(x, w, gy, stride, pad):
    """(dx, dw) as fresh buffers: backward_buffers (conv2d.rs:269-292)."""
    x, w, gy = _f32(x), _f32(w), _f32(gy)
    g = geometry(*x.shape, w.shape[0], w.shape[2], w.shape[3], stride, pad)
    if gy.shape != (g.n, g.k, g.oh, g.ow):
        raise ValueError("grad length must match the output")
    dx = np.zeros(x.shape, np.float32)
    dw = np.zeros(w.shape, np.float32)
    check(lib().katsu_hip_conv2d_bwd_f32(_p(x), _p(w), _p(gy), _p(dx), _p(dw), ctypes.byref(g),
                                         0.0), "conv2d_bwd")
    return dx, dw


def gemm(a, b, c, m, n, k, trans_a=False, trans_b=False, beta=0.0):
    """c = beta*c + op(a) op(b), in place on the numpy array c."""
    a, b = _f32(a), _f32(b)
    assert c.dtype == np.float32 and c.flags.c_contiguous
    check(lib().katsu_hip_gemm_f32(_p(a), _p(b), _p(c), m, n, k, int(trans_a), int(trans_b),
                                   float(beta)), "gemm")
    return c


def matmul(a, b):
    a, b = _f32(a), _f32(b)
    m, k = a.shape
    n = b.shape[1]
    c = np.zeros((m, n), np.float32)
    return gemm(a, b, c, m, n, k)


def matmul_vjp(a, b, g, da, db):
    a, b, g = _f32(a), _f32(b), _f32(g)
    m, k = a.shape
    n = b.shape[1]
    if m * n == 0 or k == 0:
        return da, db
    gemm(g, b, da, m, k, n, trans_b=True, beta=1.0)
    gemm(a, g, db, k, n, m, trans_a=True, beta=1.0)
    return da, db
