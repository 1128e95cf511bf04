"""Build the CPU oracle (test infrastructure only) into oracle/libmlrs_oracle.so
and oracle/libmlrs_oracle_v4.so.

The flags are part of the oracle's definition:
  -ffp-contract=off   every multiply and add rounds on its own; fused
                      multiply-adds appear only where ref_cpu.c calls fma()
  -fopenmp            query blocks spread over the host cores (bench.py's CPU
                      baseline); results do not depend on the thread count
and the instruction set is not: the build runs in the CPU container and ships
the .so files to the GPU box, whose CPU model is only known there, so two
builds are made -- -march=x86-64-v3 (AVX2 + FMA, any x86-64 server of the last
decade) and -march=x86-64-v4 (AVX-512) -- and oracle/__init__.py loads the
widest one the host supports.  With contraction off and no reassociation the
two return the same bits (tests/test_oracle.py checks it where both load).
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
SRCS = [os.path.join(HERE, "ref_cpu.c"), os.path.join(HERE, "consumers_cpu.c"), os.path.join(HERE, "graph_cpu.c"),
        os.path.join(HERE, "kmeans_cpu.c")]
COMMON = ["-O3", "-ffp-contract=off", "-fno-math-errno", "-fopenmp", "-fPIC", "-shared", "-std=c11", "-Wall",
          "-Wextra"]
VARIANTS = {  # ISA level -> (output, -march)
    "x86-64-v3": (os.path.join(HERE, "libmlrs_oracle.so"), "-march=x86-64-v3"),
    "x86-64-v4": (os.path.join(HERE, "libmlrs_oracle_v4.so"), "-march=x86-64-v4"),
}
OUT = VARIANTS["x86-64-v3"][0]
# kept for callers that print the definition of the baseline
FLAGS = COMMON[:1] + ["-march=x86-64-v3|v4"] + COMMON[1:]


def flags_of(isa):
    return " ".join(COMMON[:1] + [VARIANTS[isa][1]] + COMMON[1:4])


def build(verbose=False):
    for isa, (out, march) in VARIANTS.items():
        tmp = out + ".tmp%d" % os.getpid()
        cmd = ["gcc"] + COMMON[:1] + [march] + COMMON[1:] + SRCS + ["-o", tmp, "-lm"]
        if verbose:
            print(" ".join(cmd))
        subprocess.run(cmd, check=True)
        os.replace(tmp, out)
    return OUT


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
