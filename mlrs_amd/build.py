"""Build the HIP engine into mlrs_amd/libmlrs_hip_knn.so (gfx950).

hipcc cross-compiles without a GPU, so this runs in the CPU container; the
built .so travels with the tree.  Flags:
  --offload-arch=gfx950      CDNA4 only, no other targets
  -ffp-contract=off          no implicit fused multiply-adds: the kernels'
                             exact arithmetic must match the reference's
                             operation order bit for bit
  -target-feature -packed-fp32-ops
                             no packed FP32 VALU instructions
"""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "libmlrs_hip_knn.so")
SOURCES = ["capi.hip", "knn_exact.hip", "knn_gram_f32.hip", "knn_gram_f64.hip", "knn_lowd.hip",
           "knn_consumers.hip", "knn_radius.hip", "knn_radius_gram.hip", "knn_graph.hip",
           "kmeans_loop.hip", "probe.hip", "knn_k1_resident.hip"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]


def _compile(src, objdir, verbose):
    obj = os.path.join(objdir, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC] + FLAGS + ["-c", os.path.join(CSRC, src), "-o", obj]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("hipcc failed for %s:\n%s%s" % (src, r.stdout, r.stderr))
    msgs = [l for l in (r.stdout + r.stderr).splitlines() if "packed-fp32-ops" not in l]
    if verbose and msgs:
        print("\n".join(msgs))
    return obj


def build(verbose=False, jobs=4):
    objdir = os.path.join(HERE, "_build")
    os.makedirs(objdir, exist_ok=True)
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, objdir, verbose), SOURCES))
    tmp = OUT + ".tmp%d" % os.getpid()
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC"] + objs + ["-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed:\n%s%s" % (r.stdout, r.stderr))
    _check_resolved(tmp)
    os.replace(tmp, OUT)
    return OUT


def _check_resolved(lib):
    """A shared library links with undefined symbols; one of the engine's own
    (e.g. a kernel launch stub the host pass dropped) would only fail when the
    library is loaded.  Fail the build instead."""
    r = subprocess.run(["nm", "-u", "-C", lib], capture_output=True, text=True)
    if r.returncode != 0:
        return  # no nm: nothing to check with
    own = [l.strip() for l in r.stdout.splitlines() if "mlrs" in l]
    if own:
        os.unlink(lib)
        raise RuntimeError("the engine library leaves its own symbols undefined:\n  " + "\n  ".join(own[:20]))


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
