"""Builds the native libraries in-tree:

  katsu_amd/lib/libkatsu_hip.so   the gfx950 kernels behind the C ABI (hipcc)
  katsu_amd/lib/libkatsu.so       the C++ front end (Tensor/Conv2D mirror of
                                  katsu-core) over that ABI (g++)
  katsu_amd/lib/frontend_bench    end-to-end steps through the front end

hipcc cross-compiles for gfx950 without a GPU, so this runs in the CPU
container; the resulting .so files travel with the tree to the GPU box.
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIB_DIR = os.path.join(HERE, "lib")
LIB = os.path.join(LIB_DIR, "libkatsu_hip.so")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

# -packed-fp32-ops: never emit v_pk_{add,mul,fma}_f32 (hipcc's host pass
# warns that it does not know the feature; that is harmless).
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-shared",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-ffp-contract=fast-honor-pragmas", "-Wall", "-Wno-unused-function",
]

SOURCES = [os.path.join(CSRC, "katsu_hip.hip")]
FRONTEND_SRC = os.path.join(HERE, "cpp", "katsu.cpp")
FRONTEND_LIB = os.path.join(LIB_DIR, "libkatsu.so")
CXX_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", "-Wextra"]


def build_frontend(verbose: bool = False) -> str:
    """The C++ front end, linked against libkatsu_hip.so (found next to it)."""
    tmp = FRONTEND_LIB + ".tmp"
    cmd = ["g++", *CXX_FLAGS, FRONTEND_SRC, "-o", tmp, "-L", LIB_DIR, "-lkatsu_hip",
           "-Wl,-rpath,$ORIGIN"]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"g++ failed ({proc.returncode}):\n{proc.stderr}")
    os.replace(tmp, FRONTEND_LIB)
    return FRONTEND_LIB


BENCH_SRC = os.path.join(HERE, "cpp", "frontend_bench.cpp")
BENCH_BIN = os.path.join(LIB_DIR, "frontend_bench")


def build_frontend_bench(verbose: bool = False) -> str:
    """The front end's end-to-end benchmark (run by bench.py)."""
    tmp = BENCH_BIN + ".tmp"
    cmd = ["g++", "-O2", "-std=c++17", "-Wall", BENCH_SRC, "-o", tmp, "-L", LIB_DIR, "-lkatsu",
           "-lkatsu_hip", "-Wl,-rpath,$ORIGIN"]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"g++ failed ({proc.returncode}):\n{proc.stderr}")
    os.replace(tmp, BENCH_BIN)
    return BENCH_BIN


def build(verbose: bool = False) -> str:
    os.makedirs(LIB_DIR, exist_ok=True)
    tmp = LIB + ".tmp"
    cmd = [HIPCC, *HIP_FLAGS, "-I", os.path.join(ROOT, "include"), *SOURCES, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # Drop the known-harmless feature warning; surface everything else.
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in proc.stderr.splitlines() if noise not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{err}")
    if err.strip() and verbose:
        print(err, file=sys.stderr)
    os.replace(tmp, LIB)
    build_frontend(verbose)
    build_frontend_bench(verbose)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
