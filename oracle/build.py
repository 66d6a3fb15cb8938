"""Build recipe for the CPU oracle (test infrastructure only).

Compiles ``oracle/katsu_oracle.c`` into ``oracle/_build/libkatsu_oracle.so``
with the flags that make it bit-identical to the reference's Rust arithmetic:
``-O3 -ffp-contract=off``, no ``-ffast-math``, default ``-march=x86-64``
(SSE2 only, so no FMA instructions exist to contract into).

The reference itself (Rust, crates/katsu-core) cannot be built here: the
image has no ``rustc``/``cargo``, so there is no ``oracle/_ref`` build.
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "katsu_oracle.c")
OUT_DIR = os.path.join(HERE, "_build")
LIB = os.path.join(OUT_DIR, "libkatsu_oracle.so")

CFLAGS = ["-O3", "-ffp-contract=off", "-fno-fast-math", "-march=x86-64",
          "-std=c11", "-Wall", "-Wextra", "-fPIC", "-shared"]


def build(verbose: bool = False) -> str:
    os.makedirs(OUT_DIR, exist_ok=True)
    tmp = LIB + ".tmp"
    cmd = ["gcc", *CFLAGS, SRC, "-o", tmp, "-lm"]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
