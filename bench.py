"""Benchmark of the brute-force kNN hot path on one MI355X.

Default workload (c2): 1,000,000 x 128 index, 10,000 x 128 queries from a
100-component Gaussian mixture, f32, Euclidean, k=32 -- the configuration the
headline metric is quoted on.  One step = one full kneighbors search of all
queries against the index (row norms, the fused Gram-MFMA + exact top-k kernel
and the strip merge), inputs already resident in HBM.

Prints ONE JSON line.  `roofline` is for the dominant kernel, timed with HIP
events recorded by the engine around that kernel's launch on the stream it runs
on; `cpu_baseline` is the CPU oracle (the C restatement of the mlrs cpu-backend
arithmetic) timed on a bounded sample of the same workload on this host.

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c2] [--no-cpu]
  python bench.py --radius R [--config c2]    # radius_neighbors on the same data

With --radius a step is one radius_neighbors call (count pass, row offsets,
fill pass, boundary transform) of all queries against the index; its parity
is checked against the CPU oracle on a few query rows.
"""
import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAKS = {  # MI355X published dense peaks
    "mfma_f32": 157.3, "mfma_f64": 78.6, "valu_f32": 78.6, "valu_f64": 78.6, "hbm": 8000.0,
}
METRIC = "kNN dist-evals/s, 1M×10k d=128 k=32 f32; % of MFMA/HBM roofline"


def log(msg):
    print("[bench] " + msg, file=sys.stderr, flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--config", default="c2", choices=["c1", "c2", "c3", "c4", "c5"])
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-threads", type=int, default=0)
    ap.add_argument("--radius", type=float, default=None,
                    help="measure radius_neighbors with this radius instead of the k-nearest search")
    ap.add_argument("--calib-copy-mib", type=int, default=0,
                    help="after the timed steps, copy a buffer of this many MiB once (a plain copy kernel "
                         "of known traffic, the scale reference for rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(--gpus %d requested; run with --gpus 1)" % args.gpus, file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    from mlrs_amd import _lib, prims, synthetic

    cfg = synthetic.CONFIGS[args.config]
    dev = torch.device("cuda:0")
    log("generating %s %s" % (args.config, cfg))
    t = time.time()
    a, b = synthetic.generate(args.config)
    log("generated in %.1fs" % (time.time() - t))
    ta = torch.from_numpy(a).to(dev)
    tb = torch.from_numpy(b).to(dev)
    torch.cuda.synchronize()
    kmeans = args.config == "c5"
    k, metric = cfg["k"], cfg["metric"]
    n_query, n_index, d = a.shape[0], b.shape[0], a.shape[1]

    radius = args.radius
    if radius is not None and kmeans:
        print("--radius needs a k-nearest configuration (c1-c4)", file=sys.stderr)
        sys.exit(2)

    def step():
        if radius is not None:
            return prims.radius_neighbors(ta, tb, radius, metric)
        if kmeans:
            return prims.kmeans_assign(ta, tb)
        return prims.knn_topk(ta, tb, k, metric)

    lib = _lib.load()
    for i in range(args.warmup):
        out = step()
    torch.cuda.synchronize()
    log("warmup done (%d steps)" % args.warmup)

    _lib.check(lib.mlrs_timing_enable(1))
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        out = step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    tot_ms, launches = ctypes.c_double(), ctypes.c_int64()
    name = ctypes.create_string_buffer(64)
    _lib.check(lib.mlrs_timing_read(ctypes.byref(tot_ms), ctypes.byref(launches), name, 64))
    _lib.check(lib.mlrs_timing_enable(0))
    ms_per_step = (t1 - t0) * 1000.0 / args.steps
    kern_ms = tot_ms.value / max(1, launches.value)
    log("timed %d steps: %.3f ms/step, %s avg %.3f ms over %d launches"
        % (args.steps, ms_per_step, name.value.decode(), kern_ms, launches.value))

    if args.calib_copy_mib:
        n = args.calib_copy_mib * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        log("calibration copy: %d MiB read + %d MiB written" % (args.calib_copy_mib, args.calib_copy_mib))
        del src, dst

    # ---- parity of the measured run against the committed golden subset ----
    g = np.load(os.path.join(ROOT, "tests", "golden", "%s_golden.npz" % args.config))
    sub = g["subset"]
    if radius is not None:
        import oracle
        dist, idx, cnt = out
        cnt = cnt.cpu().numpy()
        off = np.concatenate([[0], np.cumsum(cnt)])
        rows = np.unique(np.linspace(0, n_query - 1, 8).astype(np.int64))
        wd, wi, wc = oracle.radius_neighbors(a[rows], b, radius, metric)
        woff = np.concatenate([[0], np.cumsum(wc.astype(np.int64))])
        gd, gi = dist.cpu().numpy(), idx.cpu().numpy()
        ok = all(cnt[q] == wc[j] and np.array_equal(gi[off[q]:off[q + 1]], wi[woff[j]:woff[j + 1]])
                 and np.array_equal(gd[off[q]:off[q + 1]], wd[woff[j]:woff[j + 1]]) for j, q in enumerate(rows))
        sub = rows
        matches = int(cnt.sum())
    elif kmeans:
        lab, sq = out
        ok = (np.array_equal(lab.cpu().numpy()[sub], g["labels"].astype(np.int64))
              and np.array_equal(sq.cpu().numpy()[sub], g["sqdist"]))
    else:
        dist, idx = out
        ok = (np.array_equal(idx.cpu().numpy()[sub], g["idx"].astype(np.int64))
              and np.array_equal(dist.cpu().numpy()[sub], g["dist"]))
    parity = ("bitwise-equal to the CPU oracle on %d %s rows" % (len(sub), "sampled" if radius is not None else "golden")
              if ok else "MISMATCH vs the CPU oracle")
    log(parity)

    evals = float(n_query) * float(n_index)
    value = evals / (ms_per_step / 1000.0)
    flops = 2.0 * d * evals
    kname = name.value.decode()
    f64 = cfg["dtype"] == "f64"
    if radius is not None and kname.startswith("radius_gram"):
        # the matrix-core screen: the Gram contraction, 2 d flops per pair
        bound, peak, unit = "mfma", PEAKS["mfma_f32"], "TFLOP/s"
    elif radius is not None:
        # the exact host scan: a subtract, a multiply and an add per pair and
        # feature (no fused multiply-add: the reference's operation order)
        flops = 3.0 * d * evals
        bound, peak, unit = "valu", PEAKS["valu_f64" if f64 else "valu_f32"], "TFLOP/s"
    elif kname.startswith("knn_gram_f64"):
        bound, peak, unit = "mfma", PEAKS["mfma_f64"], "TFLOP/s"
    elif kname.startswith("knn_gram_f32"):
        bound, peak, unit = "mfma", PEAKS["mfma_f32"], "TFLOP/s"
    else:
        # the low-d ALU kernel and the exact tiles of small searches: vector
        # units without packed math (an FMA counts two flops)
        bound, peak, unit = "valu", PEAKS["valu_f64" if f64 else "valu_f32"], "TFLOP/s"
    achieved = flops / (kern_ms / 1000.0) / 1e12
    traffic = None
    tfile = os.path.join(ROOT, "profiles", "traffic_%s%s.json" % ("radius_" if radius is not None else "",
                                                                   args.config))
    if os.path.exists(tfile):
        traffic = json.load(open(tfile)).get("hbm_bytes_per_launch")

    cpu = None
    if not args.no_cpu:
        import oracle
        threads = args.cpu_threads or min(16, len(os.sched_getaffinity(0)))
        # bounded sample: a prefix of the queries against the full index, run
        # repeatedly until about 10 s of CPU work has been timed
        sample = {"c1": n_query, "c2": 2000, "c3": 256, "c4": 20000, "c5": 400000}[args.config]
        if radius is not None:
            sample = {"c1": n_query, "c2": 512, "c3": 128, "c4": 20000}[args.config]
        log("CPU baseline: %d of %d queries, %d threads" % (sample, n_query, threads))

        def cpu_pass():
            if radius is not None:
                oracle.radius_neighbors(a[:sample], b, radius, metric, nthreads=threads)
            elif kmeans:
                oracle.kmeans_assign(a[:sample], b, nthreads=threads)
            else:
                oracle.knn_topk(a[:sample], b, k, metric, nthreads=threads)

        reps, dt = 0, 0.0
        while dt < 10.0 and reps < 100000:
            tc = time.perf_counter()
            cpu_pass()
            dt += time.perf_counter() - tc
            reps += 1
        cpu = {"value": float(sample) * n_index * reps / dt, "unit": "dist-evals/s", "cores": threads, "kind": "port",
               "sample": "first %d of %d queries vs the full %d-row index, %d passes in %.1f s"
                         % (sample, n_query, n_index, reps, dt)}
        log("CPU baseline %.3g evals/s" % cpu["value"])

    wl = {"c1": "c1: 10k x 1k, d=64, k=10, f32 N(0,1)",
          "c2": "c2: 1M index x 10k queries, d=128, k=32, f32, 100-comp GMM",
          "c3": "c3: 200k x 5k, d=256, k=16, f64 cosine, U[0,1)",
          "c4": "c4: 500k self-kNN, d=3, k=8, f32, 5% exact duplicates",
          "c5": "c5: k-means assign, 5M points x 1024 centroids, d=64, f32"}[args.config]
    if radius is not None:
        wl = "radius_neighbors, radius %g, on %s (%d matches, %.1f per query)" % (radius, wl, matches,
                                                                                 matches / n_query)
    line = {
        "metric": (METRIC if args.config == "c2" else "dist-evals/s (%s)" % args.config) if radius is None
        else "radius_neighbors dist-evals/s (%s)" % args.config,
        "value": value,
        "unit": "dist-evals/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f64" if cfg["dtype"] == "f64" else "f32",
        "data": "synthetic (seeded generator, mlrs_amd/synthetic.py)",
        "config": {"workload": wl, "n_index": n_index, "n_query": n_query, "d": d,
                   "k": k if radius is None else None, "radius": radius, "metric": metric,
                   "queries_per_s": n_query / (ms_per_step / 1000.0), "parity": parity},
        "roofline": {"bound": bound, "achieved": achieved, "peak": peak, "unit": unit, "frac": achieved / peak,
                     "traffic": traffic, "kernel": name.value.decode(), "kernel_ms": kern_ms},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    if not ok:
        sys.exit(1)


if __name__ == "__main__":
    main()
