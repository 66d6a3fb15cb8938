"""Device-tensor entry points over the C ABI (the ``*_dev`` functions).

torch is plumbing here: it owns device memory and the stream.  Every call
launches the gfx950 kernels of libkatsu_hip.so on torch's current stream;
nothing is computed by torch.  Host (numpy) entry points live in
``katsu_amd.host``.
"""
import ctypes

import torch

from ._abi import check, geometry, lib


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _p(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None and t.numel() else ctypes.c_void_p(0)


def _dev_f32(*ts):
    for t in ts:
        if t is None:
            continue
        if not t.is_cuda or t.dtype != torch.float32 or not t.is_contiguous():
            raise ValueError("katsu_amd.ops expects contiguous float32 device tensors")


def conv_geom(xshape, wshape, stride, pad):
    n, c, h, w = xshape
    k, c2, r, s = wshape
    if c != c2:
        raise ValueError("input channels must match weights")
    return geometry(n, c, h, w, k, r, s, stride, pad)


def conv2d_forward(x, w, stride, pad, out=None):
    """y = conv(x, w): Conv2D::forward (conv2d.rs:95-115)."""
    _dev_f32(x, w, out)
    g = conv_geom(x.shape, w.shape, stride, pad)
    if out is None:
        out = torch.empty((g.n, g.k, g.oh, g.ow), device=x.device, dtype=torch.float32)
    check(lib().katsu_hip_conv2d_fwd_f32_dev(_p(x), _p(w), _p(out), ctypes.byref(g), _stream()),
          "conv2d_fwd")
    return out


def conv2d_backward_data(gy, w, xshape, stride, pad, out=None, beta=0.0):
    """dx (conv2d.rs:288); beta=1 accumulates into `out`."""
    _dev_f32(gy, w, out)
    g = conv_geom(xshape, w.shape, stride, pad)
    if out is None:
        out = torch.empty(tuple(xshape), device=gy.device, dtype=torch.float32)
    check(lib().katsu_hip_conv2d_bwd_data_f32_dev(_p(gy), _p(w), _p(out), ctypes.byref(g),
                                                   float(beta), _stream()), "conv2d_bwd_data")
    return out


def bwd_filter_workspace_bytes(xshape, wshape, stride, pad):
    g = conv_geom(xshape, wshape, stride, pad)
    nbytes = ctypes.c_size_t(0)
    check(lib().katsu_hip_conv2d_bwd_filter_workspace(ctypes.byref(g), ctypes.byref(nbytes)),
          "bwd_filter_workspace")
    return nbytes.value


def conv2d_backward_filter(x, gy, wshape, stride, pad, out=None, beta=0.0, workspace=None):
    """dw (conv2d.rs:289); beta=1 accumulates into `out`.

    `workspace` is an optional uint8/float device tensor of at least
    bwd_filter_workspace_bytes(); without it the library's own buffer is used."""
    _dev_f32(x, gy, out)
    g = conv_geom(x.shape, wshape, stride, pad)
    if out is None:
        out = torch.empty(tuple(wshape), device=x.device, dtype=torch.float32)
    ws = ctypes.c_void_p(workspace.data_ptr()) if workspace is not None else ctypes.c_void_p(0)
    wsb = workspace.numel() * workspace.element_size() if workspace is not None else 0
    check(lib().katsu_hip_conv2d_bwd_filter_f32_dev(_p(x), _p(gy), _p(out), ctypes.byref(g),
                                                     float(beta), ws, wsb, _stream()),
          "conv2d_bwd_filter")
    return out


def conv2d_backward(x, w, gy, stride, pad, dx=None, dw=None, beta=0.0, workspace=None):
    """(dx, dw) of backward_buffers (conv2d.rs:265-292) in one call; beta=1
    accumulates into `dx` and `dw`.  When both passes take the direct gfx950
    kernels they run as a single launch.  `workspace` as for
    conv2d_backward_filter."""
    _dev_f32(x, w, gy, dx, dw)
    g = conv_geom(x.shape, w.shape, stride, pad)
    if dx is None:
        dx = torch.empty(tuple(x.shape), device=x.device, dtype=torch.float32)
    if dw is None:
        dw = torch.empty(tuple(w.shape), device=x.device, dtype=torch.float32)
    ws = ctypes.c_void_p(workspace.data_ptr()) if workspace is not None else ctypes.c_void_p(0)
    wsb = workspace.numel() * workspace.element_size() if workspace is not None else 0
    check(lib().katsu_hip_conv2d_bwd_f32_dev(_p(x), _p(w), _p(gy), _p(dx), _p(dw),
                                              ctypes.byref(g), float(beta), ws, wsb, _stream()),
          "conv2d_bwd")
    return dx, dw


def gemm(a, b, m, n, k, trans_a=False, trans_b=False, out=None, beta=0.0):
    """out[m,n] = beta*out + op(a) op(b) (tensor.rs:264-273, 424-444)."""
    _dev_f32(a, b, out)
    if out is None:
        out = torch.empty((m, n), device=a.device, dtype=torch.float32)
    check(lib().katsu_hip_gemm_f32_dev(_p(a), _p(b), _p(out), m, n, k, int(trans_a),
                                       int(trans_b), float(beta), _stream()), "gemm")
    return out


def matmul(a, b):
    """Tensor::matmul forward: [m,k] @ [k,n] (tensor.rs:249-280)."""
    m, k = a.shape
    k2, n = b.shape
    if k != k2:
        raise ValueError("matmul inner dimensions differ")
    return gemm(a, b, m, n, k)


def matmul_vjp(a, b, g, da, db):
    """Matmul VJP (tensor.rs:418-445): da += g b^T, then db += a^T g.

    One call of katsu_hip_matmul_vjp_f32_dev: the two products run as one
    launch when da and db are separate buffers, and in the reference's order
    when they are the same tensor (A and B the same node)."""
    m, k = a.shape
    n = b.shape[1]
    if m * n == 0 or k == 0:
        return da, db
    _dev_f32(a, b, g, da, db)
    check(lib().katsu_hip_matmul_vjp_f32_dev(_p(a), _p(b), _p(g), _p(da), _p(db), m, k, n,
                                             1.0, 1.0, _stream()), "matmul_vjp")
    return da, db


# ---- the device engine's elementwise work (f32, n elements, device tensors) ----

def add(a, b, out=None, beta=0.0):
    """out = beta*out + (a + b): Tensor::add (tensor.rs:217-240), bit-exact."""
    _dev_f32(a, b, out)
    if a.shape != b.shape:
        raise ValueError("identical shapes required")
    out = torch.empty_like(a) if out is None else out
    check(lib().katsu_hip_add_f32_dev(_p(a), _p(b), _p(out), a.numel(), float(beta), _stream()),
          "add")
    return out


def mul(a, b, out=None, beta=0.0):
    """out = beta*out + a*b: Tensor::mul, or Mul's VJP with beta = 1."""
    _dev_f32(a, b, out)
    if a.shape != b.shape:
        raise ValueError("identical shapes required")
    out = torch.empty_like(a) if out is None else out
    check(lib().katsu_hip_mul_f32_dev(_p(a), _p(b), _p(out), a.numel(), float(beta), _stream()),
          "mul")
    return out


def accumulate(x, y, beta=1.0):
    """y = beta*y + x (an adjoint into a pending buffer)."""
    _dev_f32(x, y)
    check(lib().katsu_hip_accumulate_f32_dev(_p(x), _p(y), x.numel(), float(beta), _stream()),
          "accumulate")
    return y


def fill(x, value):
    _dev_f32(x)
    check(lib().katsu_hip_fill_f32_dev(_p(x), x.numel(), float(value), _stream()), "fill")
    return x


def add_scalar(s, y, beta=1.0):
    """y = beta*y + s[0] (Sum's VJP)."""
    _dev_f32(s, y)
    check(lib().katsu_hip_add_scalar_f32_dev(_p(s), _p(y), y.numel(), float(beta), _stream()),
          "add_scalar")
    return y


def sum(x, out=None, beta=0.0):
    """out[0] = beta*out[0] + sum(x): Tensor::sum (tensor.rs:242-247), fixed tree."""
    _dev_f32(x, out)
    out = torch.empty(1, device=x.device, dtype=torch.float32) if out is None else out
    check(lib().katsu_hip_sum_f32_dev(_p(x), x.numel(), _p(out), float(beta), _stream()), "sum")
    return out


def mean_rows(y, rows, cols, out=None):
    """out[r] = sum_c y[r][c] / cols (the stem chain's global average pool)."""
    _dev_f32(y, out)
    out = torch.empty(rows, device=y.device, dtype=torch.float32) if out is None else out
    check(lib().katsu_hip_mean_rows_f32_dev(_p(y), rows, cols, _p(out), _stream()), "mean_rows")
    return out


def broadcast_rows(g, rows, cols, scale, dy=None, beta=0.0):
    """dy[r][c] = beta*dy[r][c] + scale*g[r] (the mean pool's VJP)."""
    _dev_f32(g, dy)
    dy = torch.empty(rows * cols, device=g.device, dtype=torch.float32) if dy is None else dy
    check(lib().katsu_hip_broadcast_rows_f32_dev(_p(g), rows, cols, float(scale), _p(dy),
                                                  float(beta), _stream()), "broadcast_rows")
    return dy


def grad_cam(act, grad, size=None):
    """Grad-CAM of an NCHW activation map and its gradient: [N, H, W] maps,
    ReLU of the channel sum weighted by the gradient's spatial means, each
    divided by its maximum; with size=(OH, OW), each map then resized to the
    original image by resize_bilinear."""
    _dev_f32(act, grad)
    if act.shape != grad.shape or act.dim() != 4:
        raise ValueError("activation and gradient must be the same NCHW shape")
    n, c, h, w = act.shape
    cam = torch.empty((n, h, w), device=act.device, dtype=torch.float32)
    check(lib().katsu_hip_gradcam_f32_dev(_p(act), _p(grad), n, c, h * w, _p(cam), _stream()),
          "grad_cam")
    return cam if size is None else resize_bilinear(cam, size)


def resize_bilinear(maps, size):
    """[N, H, W] maps resized to [N, OH, OW]: bilinear, half-pixel centres."""
    _dev_f32(maps)
    if maps.dim() != 3:
        raise ValueError("maps must be [N, H, W]")
    n, h, w = maps.shape
    oh, ow = (int(v) for v in size)
    out = torch.empty((n, oh, ow), device=maps.device, dtype=torch.float32)
    check(lib().katsu_hip_resize_bilinear_f32_dev(_p(maps), n, h, w, oh, ow, _p(out),
                                                   _stream()), "resize_bilinear")
    return out
