"""Build recipe for the CPU oracle (test infrastructure): hn_oracle.c -> oracle/liboracle.so.

The reference (PedroMarinhoDev/ComfyUI-Hy-Nomas) has no C/C++ sources on this path (its kernels are
Triton JIT functions), so there is nothing to compile into oracle/_ref/; the oracle is this restatement.
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))


def build(verbose=False):
    src = os.path.join(HERE, "hn_oracle.c")
    out = os.path.join(HERE, "liboracle.so")
    tmp = out + ".tmp"
    cmd = ["gcc", "-O2", "-std=c11", "-fPIC", "-shared", "-fopenmp", "-ffp-contract=off", "-fno-fast-math",
           src, "-o", tmp, "-lm"]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
