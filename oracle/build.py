"""Build the CPU oracle (test infrastructure only) into oracle/libmlrs_oracle.so.

The flags are part of the oracle's definition:
  -ffp-contract=off   every multiply and add rounds on its own; fused
                      multiply-adds appear only where ref_cpu.c calls fma()
  -march=x86-64-v3    AVX2+FMA, portable to the GPU box's host CPU (the build
                      runs in the CPU container and ships the .so over)
  -fopenmp            query blocks spread over the host cores (bench.py's CPU
                      baseline); results do not depend on the thread count
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
SRCS = [os.path.join(HERE, "ref_cpu.c"), os.path.join(HERE, "consumers_cpu.c"), os.path.join(HERE, "graph_cpu.c"),
        os.path.join(HERE, "kmeans_cpu.c")]
OUT = os.path.join(HERE, "libmlrs_oracle.so")
FLAGS = ["-O3", "-march=x86-64-v3", "-ffp-contract=off", "-fno-math-errno",
         "-fopenmp", "-fPIC", "-shared", "-std=c11", "-Wall", "-Wextra"]


def build(verbose=False):
    tmp = OUT + ".tmp%d" % os.getpid()
    cmd = ["gcc"] + FLAGS + SRCS + ["-o", tmp, "-lm"]
    if verbose:
        print(" ".join(cmd))
    subprocess.run(cmd, check=True)
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
