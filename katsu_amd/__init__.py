"""katsu_amd -- MI355X-native dense-contraction path of Katsu.

Conv2D forward / dX / dW and matmul with its VJPs run as hand-written
fp32-MFMA HIP kernels for gfx950 behind the C ABI in include/katsu_hip.h
(libkatsu_hip.so).  Submodules:
  katsu_amd.ops    device-tensor entry points (torch owns memory and stream)
  katsu_amd.host   host-buffer drop-in entry points
  katsu_amd.synth  seeded synthetic inputs of the benchmark workloads
"""
from ._abi import (EXPORTS, LIB_PATH, ConvGeom, KatsuError, check, geometry, lib,  # noqa: F401
                   strerror, version)

__all__ = ["EXPORTS", "LIB_PATH", "ConvGeom", "KatsuError", "check", "geometry", "lib",
           "strerror", "version"]
