"""ctypes view of the CPU oracle (test infrastructure only).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline
leg import this module, and only as the checker.  Each wrapper names the
reference function it restates; the restatement itself is
``oracle/katsu_oracle.c``.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "libkatsu_oracle.so")

OK, SHAPE_OVERFLOW, INVALID_CONV = 0, 1, 2
GEO_FIELDS = ("batch", "cin", "cout", "h", "w", "kh", "kw", "oh", "ow", "stride", "padding")

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"oracle not built: {LIB_PATH} (run oracle/build.py)")
        L = ctypes.CDLL(LIB_PATH)
        u64p = ctypes.POINTER(ctypes.c_uint64)
        fp = ctypes.c_void_p
        L.ko_element_count.argtypes = [u64p, ctypes.c_size_t, u64p]
        L.ko_conv_geometry.argtypes = [u64p, ctypes.c_size_t, u64p, ctypes.c_size_t,
                                       ctypes.c_uint64, ctypes.c_uint64, u64p]
        L.ko_conv2d_forward.argtypes = [fp, fp, fp, u64p]
        L.ko_conv2d_backward.argtypes = [fp, fp, fp, fp, fp, u64p]
        L.ko_conv2d_backward_data.argtypes = [fp, fp, fp, u64p]
        L.ko_conv2d_backward_filter.argtypes = [fp, fp, fp, u64p]
        L.ko_matmul.argtypes = [fp, fp, fp, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_uint64]
        L.ko_matmul_vjp.argtypes = [fp, fp, fp, fp, fp,
                                    ctypes.c_uint64, ctypes.c_uint64, ctypes.c_uint64]
        L.ko_sum.argtypes = [fp, ctypes.c_uint64]
        L.ko_sum.restype = ctypes.c_float
        L.ko_splitmix_next.argtypes = [u64p]
        L.ko_splitmix_next.restype = ctypes.c_uint64
        L.ko_splitmix_fill.argtypes = [ctypes.c_uint64, ctypes.c_uint64, fp, ctypes.c_uint64]
        _lib = L
    return _lib


def _u64(values):
    arr = (ctypes.c_uint64 * max(1, len(values)))(*[int(v) for v in values])
    return arr


def _f32(a):
    a = np.ascontiguousarray(a, dtype=np.float32)
    return a


def _ptr(a):
    return ctypes.c_void_p(a.ctypes.data) if a.size else ctypes.c_void_p(0)


class OracleError(Exception):
    def __init__(self, code):
        super().__init__({SHAPE_OVERFLOW: "ShapeOverflow", INVALID_CONV: "InvalidConv"}.get(code, code))
        self.code = code


def element_count(shape):
    """tensor.rs:127-138."""
    out = ctypes.c_uint64(0)
    st = lib().ko_element_count(_u64(shape), len(shape), ctypes.byref(out))
    if st:
        raise OracleError(st)
    return out.value


def conv_geometry(xshape, wshape, stride, padding):
    """Geometry::new (conv2d.rs:183-224) -> dict of the Geometry fields."""
    geo = (ctypes.c_uint64 * 11)()
    st = lib().ko_conv_geometry(_u64(xshape), len(xshape), _u64(wshape), len(wshape),
                                ctypes.c_uint64(stride), ctypes.c_uint64(padding), geo)
    if st:
        raise OracleError(st)
    return dict(zip(GEO_FIELDS, list(geo)))


def _geo_arr(geo):
    return _u64([geo[f] for f in GEO_FIELDS])


def conv2d_forward(x, w, stride, padding):
    """Conv2D::forward (conv2d.rs:95-115) -> y, NCHW."""
    x, w = _f32(x), _f32(w)
    geo = conv_geometry(x.shape, w.shape, stride, padding)
    y = np.empty((geo["batch"], geo["cout"], geo["oh"], geo["ow"]), np.float32)
    lib().ko_conv2d_forward(_ptr(x), _ptr(w), _ptr(y), _geo_arr(geo))
    return y


def conv2d_backward(x, w, g, stride, padding):
    """backward_buffers (conv2d.rs:269-292) -> (dx, dw), fresh buffers."""
    x, w, g = _f32(x), _f32(w), _f32(g)
    geo = conv_geometry(x.shape, w.shape, stride, padding)
    assert g.shape == (geo["batch"], geo["cout"], geo["oh"], geo["ow"])
    dx = np.empty(x.shape, np.float32)
    dw = np.empty(w.shape, np.float32)
    lib().ko_conv2d_backward(_ptr(x), _ptr(w), _ptr(g), _ptr(dx), _ptr(dw), _geo_arr(geo))
    return dx, dw


def conv2d_backward_data(xshape, w, g, stride, padding):
    """dX half of backward_buffers (conv2d.rs:288), bit-identical to it."""
    w, g = _f32(w), _f32(g)
    geo = conv_geometry(xshape, w.shape, stride, padding)
    dx = np.empty(tuple(xshape), np.float32)
    lib().ko_conv2d_backward_data(_ptr(w), _ptr(g), _ptr(dx), _geo_arr(geo))
    return dx


def conv2d_backward_filter(x, wshape, g, stride, padding):
    """dW half of backward_buffers (conv2d.rs:289), bit-identical to it."""
    x, g = _f32(x), _f32(g)
    geo = conv_geometry(x.shape, wshape, stride, padding)
    dw = np.empty(tuple(wshape), np.float32)
    lib().ko_conv2d_backward_filter(_ptr(x), _ptr(g), _ptr(dw), _geo_arr(geo))
    return dw


def matmul(a, b):
    """Tensor::matmul kernel (tensor.rs:264-273)."""
    a, b = _f32(a), _f32(b)
    m, k = a.shape
    k2, n = b.shape
    assert k == k2
    c = np.empty((m, n), np.float32)
    lib().ko_matmul(_ptr(a), _ptr(b), _ptr(c), m, k, n)
    return c


def matmul_vjp(a, b, g, da=None, db=None):
    """Matmul VJP (tensor.rs:418-445), accumulating into da/db in place.

    Pass the same array for da and db to reproduce aliased parents (A is B).
    Returns (da, db)."""
    a, b, g = _f32(a), _f32(b), _f32(g)
    m, k = a.shape
    n = b.shape[1]
    if da is None:
        da = np.zeros((m, k), np.float32)
    if db is None:
        db = np.zeros((k, n), np.float32)
    assert da.dtype == np.float32 and da.flags.c_contiguous
    assert db.dtype == np.float32 and db.flags.c_contiguous
    lib().ko_matmul_vjp(_ptr(a), _ptr(b), _ptr(g), _ptr(da), _ptr(db), m, k, n)
    return da, db


def fsum(x):
    """Tensor::sum (tensor.rs:242-247), sequential f32."""
    x = _f32(x).ravel()
    return float(lib().ko_sum(_ptr(x), x.size))


def splitmix_outputs(seed, count):
    """Raw SplitMix64 outputs (conv2d.rs:52-56)."""
    state = ctypes.c_uint64(seed)
    return [lib().ko_splitmix_next(ctypes.byref(state)) for _ in range(count)]


def seeded_weights(in_channels, out_channels, kernel_size, seed):
    """Conv2D::new_seeded weight values (conv2d.rs:35-61), OIHW."""
    shape = (out_channels, in_channels, kernel_size[0], kernel_size[1])
    fan_in = in_channels * kernel_size[0] * kernel_size[1]
    out = np.empty(shape, np.float32)
    lib().ko_splitmix_fill(seed, fan_in, _ptr(out), out.size)
    return out
