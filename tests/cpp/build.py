"""Builds the C++ front-end test driver tests/cpp/_build/test_frontend
(test infrastructure; links katsu_amd/lib/libkatsu.so)."""
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
    cmd = ["g++", "-O2", "-std=c++17", "-Wall", "-Wextra", os.path.join(HERE, "test_frontend.cpp"),
           "-o", tmp, "-L", LIB_DIR, "-lkatsu", "-lkatsu_hip", rpath]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
