"""ctypes bindings of ``include/katsu_hip.h`` (libkatsu_hip.so).

The library is required: importing a compute entry point without the built
.so raises immediately, and there is no CPU fallback anywhere in the package.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libkatsu_hip.so")

OK, E_INVALID, E_NODEVICE, E_OOM, E_LAUNCH, E_SCRATCH = 0, 1, 2, 3, 4, 5

# Every symbol include/katsu_hip.h declares.
EXPORTS = (
    "katsu_hip_version", "katsu_hip_strerror", "katsu_hip_init", "katsu_hip_shutdown",
    "katsu_hip_conv2d_geometry",
    "katsu_hip_gemm_f32", "katsu_hip_gemm_f32_dev", "katsu_hip_matmul_vjp_f32_dev",
    "katsu_hip_conv2d_fwd_f32", "katsu_hip_conv2d_fwd_f32_dev",
    "katsu_hip_conv2d_bwd_data_f32", "katsu_hip_conv2d_bwd_data_f32_dev",
    "katsu_hip_conv2d_bwd_filter_workspace",
    "katsu_hip_conv2d_bwd_filter_f32", "katsu_hip_conv2d_bwd_filter_f32_dev",
    "katsu_hip_conv2d_bwd_f32", "katsu_hip_conv2d_bwd_f32_dev",
    "katsu_hip_conv2d_bwd_f32_dev_noalloc", "katsu_hip_noalloc_scratch_bytes",
    "katsu_hip_device_allocations",
    "katsu_hip_stream", "katsu_hip_malloc", "katsu_hip_free", "katsu_hip_upload",
    "katsu_hip_download", "katsu_hip_sync",
    "katsu_hip_add_f32_dev", "katsu_hip_mul_f32_dev", "katsu_hip_accumulate_f32_dev",
    "katsu_hip_fill_f32_dev", "katsu_hip_add_scalar_f32_dev", "katsu_hip_sum_f32_dev",
    "katsu_hip_mean_rows_f32_dev", "katsu_hip_broadcast_rows_f32_dev",
    "katsu_hip_gradcam_f32_dev", "katsu_hip_resize_bilinear_f32_dev",
)


class KatsuError(RuntimeError):
    def __init__(self, status, where=""):
        self.status = status
        text = strerror(status) if _lib is not None else str(status)
        super().__init__(f"{where}: katsu status {status} ({text})" if where else text)


class ConvGeom(ctypes.Structure):
    """katsu_conv_geom: the fields of the reference's Geometry (conv2d.rs:168-180)."""
    _fields_ = [(f, ctypes.c_uint64) for f in
                ("n", "c", "h", "w", "k", "r", "s", "stride", "pad", "oh", "ow")]


_lib = None


def lib():
    """Load libkatsu_hip.so (once).  Raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"katsu_amd: {LIB_PATH} is missing; run __graft_entry__.build() "
                "(there is no CPU fallback)")
        L = ctypes.CDLL(LIB_PATH)
        vp, sz, fp, i = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_float, ctypes.c_int
        gp = ctypes.POINTER(ConvGeom)
        L.katsu_hip_version.restype = ctypes.c_char_p
        L.katsu_hip_strerror.restype = ctypes.c_char_p
        L.katsu_hip_strerror.argtypes = [i]
        L.katsu_hip_init.restype = i
        L.katsu_hip_shutdown.restype = None
        L.katsu_hip_conv2d_geometry.argtypes = [gp]
        L.katsu_hip_gemm_f32.argtypes = [vp, vp, vp, sz, sz, sz, i, i, fp]
        L.katsu_hip_gemm_f32_dev.argtypes = [vp, vp, vp, sz, sz, sz, i, i, fp, vp]
        L.katsu_hip_matmul_vjp_f32_dev.argtypes = [vp, vp, vp, vp, vp, sz, sz, sz, fp, fp, vp]
        L.katsu_hip_conv2d_fwd_f32.argtypes = [vp, vp, vp, gp]
        L.katsu_hip_conv2d_fwd_f32_dev.argtypes = [vp, vp, vp, gp, vp]
        L.katsu_hip_conv2d_bwd_data_f32.argtypes = [vp, vp, vp, gp, fp]
        L.katsu_hip_conv2d_bwd_data_f32_dev.argtypes = [vp, vp, vp, gp, fp, vp]
        L.katsu_hip_conv2d_bwd_filter_workspace.argtypes = [gp, ctypes.POINTER(sz)]
        L.katsu_hip_conv2d_bwd_filter_f32.argtypes = [vp, vp, vp, gp, fp]
        L.katsu_hip_conv2d_bwd_filter_f32_dev.argtypes = [vp, vp, vp, gp, fp, vp, sz, vp]
        L.katsu_hip_conv2d_bwd_f32.argtypes = [vp, vp, vp, vp, vp, gp, fp]
        L.katsu_hip_conv2d_bwd_f32_dev.argtypes = [vp, vp, vp, vp, vp, gp, fp, vp, sz, vp]
        L.katsu_hip_conv2d_bwd_f32_dev_noalloc.argtypes = [vp, vp, vp, vp, vp, gp, fp, vp]
        L.katsu_hip_noalloc_scratch_bytes.argtypes = []
        L.katsu_hip_stream.restype = vp
        L.katsu_hip_stream.argtypes = []
        L.katsu_hip_malloc.argtypes = [ctypes.POINTER(vp), sz]
        L.katsu_hip_free.argtypes = [vp]
        L.katsu_hip_upload.argtypes = [vp, vp, sz, vp]
        L.katsu_hip_download.argtypes = [vp, vp, sz, vp]
        L.katsu_hip_sync.argtypes = [vp]
        L.katsu_hip_add_f32_dev.argtypes = [vp, vp, vp, sz, fp, vp]
        L.katsu_hip_mul_f32_dev.argtypes = [vp, vp, vp, sz, fp, vp]
        L.katsu_hip_accumulate_f32_dev.argtypes = [vp, vp, sz, fp, vp]
        L.katsu_hip_fill_f32_dev.argtypes = [vp, sz, fp, vp]
        L.katsu_hip_add_scalar_f32_dev.argtypes = [vp, vp, sz, fp, vp]
        L.katsu_hip_sum_f32_dev.argtypes = [vp, sz, vp, fp, vp]
        L.katsu_hip_mean_rows_f32_dev.argtypes = [vp, sz, sz, vp, vp]
        L.katsu_hip_broadcast_rows_f32_dev.argtypes = [vp, sz, sz, fp, vp, fp, vp]
        L.katsu_hip_gradcam_f32_dev.argtypes = [vp, vp, sz, sz, sz, vp, vp]
        L.katsu_hip_resize_bilinear_f32_dev.argtypes = [vp, sz, sz, sz, sz, sz, vp, vp]
        for name in EXPORTS:
            if name not in ("katsu_hip_version", "katsu_hip_strerror", "katsu_hip_shutdown",
                            "katsu_hip_noalloc_scratch_bytes",
                            "katsu_hip_device_allocations"):
                getattr(L, name).restype = i
        L.katsu_hip_noalloc_scratch_bytes.restype = sz
        L.katsu_hip_device_allocations.argtypes = []
        L.katsu_hip_device_allocations.restype = ctypes.c_uint64
        _lib = L
    return _lib


def strerror(status):
    return lib().katsu_hip_strerror(int(status)).decode()


def check(status, where=""):
    if status != OK:
        raise KatsuError(status, where)


def version():
    return lib().katsu_hip_version().decode()


def geometry(n, c, h, w, k, r, s, stride, pad):
    """katsu_hip_conv2d_geometry: validated geometry with oh/ow filled in."""
    g = ConvGeom(n, c, h, w, k, r, s, stride, pad, 0, 0)
    check(lib().katsu_hip_conv2d_geometry(ctypes.byref(g)), "conv2d_geometry")
    return g
