"""Build recipe for the C restatement oracle (test infrastructure only).

Compiles oracle/afa_contract.c into oracle/_build/liboracle_afa.so with gcc.
The reference itself (JAX/Python, no C sources on this path) has nothing to build,
so there is no oracle/_ref/ artefact.
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
OUT_DIR = os.path.join(HERE, "_build")
LIB = os.path.join(OUT_DIR, "liboracle_afa.so")

# x86-64-v3 (AVX2/FMA ISA level) instead of -march=native: the library is built here and
# run on the GPU box's host CPU.  -ffp-contract=off keeps every multiply and add rounded
# separately, as the reference's elementwise ops are.
CFLAGS = ["-O3", "-march=x86-64-v3", "-fopenmp", "-ffp-contract=off", "-fno-math-errno",
          "-fPIC", "-shared", "-std=c11", "-Wall", "-Wextra", "-Wno-unused-parameter"]


def build(verbose: bool = False) -> str:
    os.makedirs(OUT_DIR, exist_ok=True)
    cmd = ["gcc", *CFLAGS, os.path.join(HERE, "afa_contract.c"), "-o", LIB + ".tmp", "-lm"]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(LIB + ".tmp", LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
