"""Build recipe for the oracle (test infrastructure): oracle/*.c -> oracle/liboracle.so.

The reference (sammcj/purebee) is JavaScript with runtime-generated WASM;
there is no C/C++ reference source to compile, so there is no oracle/_ref.
"""
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "liboracle.so")


def build(verbose=False):
    srcs = sorted(os.path.join(HERE, f) for f in os.listdir(HERE) if f.endswith(".c"))
    tmp = OUT + ".tmp"
    # -ffp-contract=off: the restated f32 kernels multiply and add separately,
    # as the reference's WebAssembly does.
    cmd = ["gcc", "-O2", "-g", "-fPIC", "-shared", "-std=c11", "-ffp-contract=off", "-mssse3",
           "-pthread", "-fopenmp", "-Wall", *srcs, "-o", tmp, "-lm"]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{r.stdout}")
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))
