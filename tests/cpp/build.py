"""Builds the C++ front-end test driver tests/cpp/_build/test_frontend
(test infrastructure).  The front end (katsu_amd/cpp/katsu.cpp) is compiled
into the driver with KATSU_TESTING, which adds the publication fault hook
that the production libkatsu.so leaves out; the kernels come from
katsu_amd/lib/libkatsu_hip.so."""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
LIB_DIR = os.path.join(ROOT, "katsu_amd", "lib")
OUT = os.path.join(HERE, "_build", "test_frontend")


def build(verbose: bool = False) -> str:
    os.makedirs(os.path.dirname(OUT), exist_ok=True)
    tmp = OUT + ".tmp"
    rpath = "-Wl,-rpath,$ORIGIN/../../../katsu_amd/lib"
    cmd = ["g++", "-O2", "-std=c++17", "-Wall", "-Wextra", "-DKATSU_TESTING",
           os.path.join(HERE, "test_frontend.cpp"),
           os.path.join(ROOT, "katsu_amd", "cpp", "katsu.cpp"),
           "-o", tmp, "-L", LIB_DIR, "-lkatsu_hip", rpath]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
