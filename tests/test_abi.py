"""The C ABI without a GPU: libkatsu_hip.so loads, exports every function
include/katsu_hip.h declares, and its host-side entry points (geometry
validation, status texts, argument checks, empty problems) behave as the
reference's Geometry::new and seams do.  No kernel is launched here."""
import ctypes
import os
import re

import numpy as np
import pytest

import katsu_amd
from katsu_amd import _abi, host
from oracle import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "katsu_hip.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(katsu_hip_\w+)\s*\(", text)))


def test_header_and_exports_agree():
    declared = _declared()
    assert declared, "no declarations found"
    assert sorted(katsu_amd.EXPORTS) == declared
    lib = katsu_amd.lib()
    for name in declared:
        assert hasattr(lib, name), name


def test_library_is_gfx950_build():
    assert "gfx950" in katsu_amd.version()


def test_strerror_texts():
    assert katsu_amd.strerror(0) == "ok"
    for code in (1, 2, 3, 4, 5):
        assert katsu_amd.strerror(code) != "unknown katsu status"
    assert katsu_amd.strerror(99) == "unknown katsu status"


GEOMETRY_CASES = [
    ((1, 1, 3, 3), (1, 1, 2, 2), 1, 0),
    ((2, 3, 7, 9), (4, 3, 3, 3), 2, 1),
    ((1, 2, 5, 5), (4, 2, 5, 5), 1, 0),
    ((0, 3, 4, 5), (2, 3, 3, 3), 1, 1),
    ((32, 64, 56, 56), (64, 64, 3, 3), 1, 1),
    ((64, 3, 224, 224), (64, 3, 7, 7), 2, 3),
    ((32, 128, 28, 28), (256, 128, 1, 1), 2, 0),
]


@pytest.mark.parametrize("xs,ws,st,p", GEOMETRY_CASES)
def test_geometry_matches_reference(xs, ws, st, p):
    """katsu_hip_conv2d_geometry against the oracle's Geometry::new."""
    g = katsu_amd.geometry(xs[0], xs[1], xs[2], xs[3], ws[0], ws[2], ws[3], st, p)
    ref = O.conv_geometry(xs, ws, st, p)
    assert (g.oh, g.ow) == (ref["oh"], ref["ow"])


@pytest.mark.parametrize("args", [
    (1, 0, 3, 3, 1, 3, 3, 1, 0),      # zero channels
    (1, 1, 3, 3, 1, 0, 3, 1, 0),      # zero kernel height
    (1, 1, 3, 3, 1, 1, 1, 0, 0),      # stride 0
    (1, 1, 2, 2, 1, 3, 3, 1, 0),      # kernel exceeds padded input
    (1, 1, 0, 2, 1, 1, 1, 1, 0),      # H = 0
    (0, 1, 2, 2, 1, 1, 1, 1, 2 ** 63),  # 2*pad overflows
    # element_count (tensor.rs:129-140) of C*H*W, K*OH*OW, N*K*OH*OW
    # (conv2d.rs:196, 214-215): overflow, or above isize::MAX / 4
    (1, 2 ** 40, 2 ** 20, 2 ** 10, 1, 1, 1, 1, 0),
    (1, 2 ** 31, 2 ** 30, 1, 1, 1, 1, 1, 0),
    (1, 1, 1, 1, 2 ** 62, 1, 1, 1, 0),
    (2 ** 31, 1, 1, 1, 2 ** 31, 1, 1, 1, 0),
])
def test_geometry_rejects(args):
    with pytest.raises(katsu_amd.KatsuError) as e:
        katsu_amd.geometry(*args)
    assert e.value.status == _abi.E_INVALID


def test_invalid_arguments_are_rejected_before_any_launch():
    L = katsu_amd.lib()
    buf = (ctypes.c_float * 4)()
    p = ctypes.cast(buf, ctypes.c_void_p)
    # beta must be 0 or 1; transposes 0 or 1
    assert L.katsu_hip_gemm_f32(p, p, p, 2, 2, 1, 0, 0, 0.5) == _abi.E_INVALID
    assert L.katsu_hip_gemm_f32(p, p, p, 2, 2, 1, 2, 0, 0.0) == _abi.E_INVALID
    # null output
    assert L.katsu_hip_gemm_f32(p, p, None, 2, 2, 1, 0, 0, 0.0) == _abi.E_INVALID
    # the VJP entry: either beta outside {0, 1}; sizes past the 32-bit index range
    assert L.katsu_hip_matmul_vjp_f32_dev(p, p, p, p, p, 2, 2, 2, 0.5, 1.0, None) == _abi.E_INVALID
    assert L.katsu_hip_matmul_vjp_f32_dev(p, p, p, p, p, 2, 2, 2, 1.0, 2.0, None) == _abi.E_INVALID
    assert L.katsu_hip_matmul_vjp_f32_dev(p, p, p, p, p, 1 << 32, 2, 2, 1.0, 1.0,
                                          None) == _abi.E_INVALID
    # oh/ow inconsistent with the geometry
    g = _abi.ConvGeom(1, 1, 3, 3, 1, 2, 2, 1, 0, 5, 5)
    assert L.katsu_hip_conv2d_fwd_f32(p, p, p, ctypes.byref(g)) == _abi.E_INVALID


def test_resize_bilinear_rejects_before_any_launch():
    """Grad-CAM's resize: null buffers and per-image sizes past the 32-bit
    index range are refused; empty outputs need no device."""
    L = katsu_amd.lib()
    buf = (ctypes.c_float * 4)()
    p = ctypes.cast(buf, ctypes.c_void_p)
    assert L.katsu_hip_resize_bilinear_f32_dev(None, 1, 4, 4, 8, 8, p, None) == _abi.E_INVALID
    assert L.katsu_hip_resize_bilinear_f32_dev(p, 1, 0, 4, 8, 8, p, None) == _abi.E_INVALID
    assert L.katsu_hip_resize_bilinear_f32_dev(p, 1, 4, 4, 1 << 16, 1 << 16, p,
                                               None) == _abi.E_INVALID
    assert L.katsu_hip_resize_bilinear_f32_dev(None, 0, 4, 4, 8, 8, None, None) == _abi.OK
    assert L.katsu_hip_resize_bilinear_f32_dev(None, 2, 4, 4, 0, 8, None, None) == _abi.OK


def test_empty_problems_need_no_device():
    """tests/tensor.rs:65-86 at the ABI: [2,0]@[0,3] gives six zeros (beta 0) or
    leaves C alone (beta 1); N = 0 leaves dW = beta*dW (tests/conv2d.rs:156-167).
    None of these touch a device."""
    c = np.full((2, 3), 5.0, np.float32)
    host.gemm(np.zeros((2, 0), np.float32), np.zeros((0, 3), np.float32), c, 2, 3, 0)
    assert c.ravel().tolist() == [0.0] * 6
    c[:] = 5.0
    host.gemm(np.zeros((2, 0), np.float32), np.zeros((0, 3), np.float32), c, 2, 3, 0, beta=1.0)
    assert c.ravel().tolist() == [5.0] * 6
    x = np.zeros((0, 3, 4, 5), np.float32)
    w = np.ones((2, 3, 3, 3), np.float32)
    dx, dw = host.conv2d_backward(x, w, np.zeros((0, 2, 4, 5), np.float32), 1, 1)
    assert dx.size == 0 and np.all(dw == 0)


def test_geometry_accepts_counts_at_the_limit():
    """Products up to isize::MAX / 4 pass Geometry::new's checks (the 32-bit
    kernel limits are the launchers' concern); batch 0 skips N*K*OH*OW."""
    g = katsu_amd.geometry(1, 2 ** 30, 2 ** 29, 2, 1, 1, 1, 1, 0)  # C*H*W = 2^60
    assert (g.oh, g.ow) == (2 ** 29, 2)
    g = katsu_amd.geometry(0, 1, 1, 1, 2 ** 61 - 1, 1, 1, 1, 0)    # K*OH*OW = isize::MAX/4
    assert (g.oh, g.ow) == (1, 1)
    with pytest.raises(katsu_amd.KatsuError):
        katsu_amd.geometry(0, 1, 1, 1, 2 ** 61, 1, 1, 1, 0)


def test_empty_problems_before_size_limits():
    """An empty matmul returns OK whatever its other dimensions, before the
    32-bit limits (tests/tensor.rs:65-86 accepts [usize::MAX, 0] . [0, 0]),
    on the host and device entry points and the VJP, with no device."""
    L = katsu_amd.lib()
    buf = (ctypes.c_float * 4)()
    p = ctypes.cast(buf, ctypes.c_void_p)
    big = 2 ** 64 - 1
    assert L.katsu_hip_gemm_f32(p, p, p, big, 0, 0, 0, 0, 0.0) == _abi.OK
    assert L.katsu_hip_gemm_f32_dev(p, p, p, big, 0, 0, 0, 0, 0.0, None) == _abi.OK
    assert L.katsu_hip_gemm_f32_dev(p, p, p, 0, 2 ** 40, 7, 0, 0, 1.0, None) == _abi.OK
    assert L.katsu_hip_matmul_vjp_f32_dev(p, p, p, p, p, big, 0, 0, 1.0, 1.0, None) == _abi.OK
    assert L.katsu_hip_matmul_vjp_f32_dev(p, p, p, p, p, 0, 5, 2 ** 40, 1.0, 1.0,
                                          None) == _abi.OK
    # Non-empty problems past the 32-bit limits are still refused.
    assert L.katsu_hip_gemm_f32_dev(p, p, p, 2 ** 31, 4, 4, 0, 0, 0.0, None) == _abi.E_INVALID


def test_overlapping_backward_outputs_are_rejected():
    """dx and dw either apart or the same buffer: a partial overlap is
    refused before anything is copied or launched (host and device forms)."""
    L = katsu_amd.lib()
    buf = np.zeros(200, np.float32)
    base = buf.ctypes.data
    g = katsu_amd.geometry(4, 3, 3, 3, 4, 3, 3, 1, 1)
    x = ctypes.c_void_p(base)
    # dx = buf[0:108], dw = buf[40:148]: they overlap without being equal.
    dx, dw = ctypes.c_void_p(base), ctypes.c_void_p(base + 40 * 4)
    assert L.katsu_hip_conv2d_bwd_f32(x, x, x, dx, dw, ctypes.byref(g), 1.0) == _abi.E_INVALID
    assert L.katsu_hip_conv2d_bwd_f32_dev(x, x, x, dx, dw, ctypes.byref(g), 1.0, None, 0,
                                          None) == _abi.E_INVALID
    # The same buffer with different sizes cannot be one node's pending buffer.
    g2 = katsu_amd.geometry(2, 3, 5, 5, 4, 3, 3, 1, 1)
    assert L.katsu_hip_conv2d_bwd_f32(x, x, x, dx, dx, ctypes.byref(g2), 1.0) == _abi.E_INVALID


def test_noalloc_scratch_covers_every_plan():
    """Every BASELINE layer's dW workspace fits the static scratch of the
    allocation-free backward (host-side plans only; no GPU)."""
    from katsu_amd import synth
    lim = _abi.lib().katsu_hip_noalloc_scratch_bytes()
    assert lim == 40 << 20
    for name, c in synth.CONV_CONFIGS.items():
        g = katsu_amd.geometry(*c["x"], c["w"][0], c["w"][2], c["w"][3], c["stride"], c["pad"])
        need = ctypes.c_size_t(0)
        assert _abi.lib().katsu_hip_conv2d_bwd_filter_workspace(ctypes.byref(g),
                                                                  ctypes.byref(need)) == 0
        assert 0 <= need.value <= lim, (name, need.value)
