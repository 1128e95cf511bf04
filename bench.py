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
  python bench.py --config c5 --fit [--fit-iters N]   # k-means fit at c5 scale
  python bench.py --config c4 --dtype f64     # a k-NN configuration in the other element type

With --radius a step is one radius_neighbors call (count pass, row offsets,
fill pass, boundary transform) of all queries against the index; its parity
is checked against the CPU oracle on a few query rows.  With --fit a step is
one k-means fit of the c5 points into 1,024 clusters from a seeded random
init (SplitMix64, as the reference draws it), tol 0, at most N Lloyd
iterations (assignment, centroid sums, relocation, host update), reported per
iteration; its parity is a fit of a 200k-row prefix against the CPU oracle's.

The CPU baseline runs the oracle on every CPU this process may use, capped
by OMP_NUM_THREADS where the host sets it (the GPU box gives one GPU's job a
16-thread CPU share that way); the line records the affinity count, the
threads used, the CPU model and the oracle's compile flags.
"""
import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAKS = {  # MI355X published dense peaks (TFLOP/s, GB/s)
    # vector FP32: the published 157.3 counts packed FP32 math (v_pk_fma_f32,
    # two lanes of f32 per instruction).  The low-d kernel is built without
    # packed FP32 ops, so its own ceiling is the non-packed rate, 78.6 TFLOP/s
    # (FP64's figure, one FMA per lane per cycle); `bench.py --probe-peak`
    # measures what register-only FMA/MFMA chains reach on the card.
    "mfma_f32": 157.3, "mfma_f64": 78.6, "valu_f32": 157.3, "valu_f64": 78.6, "hbm": 8000.0,
}
VALU_F32_NONPACKED = 78.6
METRIC = "kNN dist-evals/s, 1M×10k d=128 k=32 f32; % of MFMA/HBM roofline"


def log(msg):
    print("[bench] " + msg, file=sys.stderr, flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--config", default="c2", choices=["c1", "c2", "c3", "c4", "c5", "d256", "c2k128"])
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-threads", type=int, default=0)
    ap.add_argument("--radius", type=float, default=None,
                    help="measure radius_neighbors with this radius instead of the k-nearest search")
    ap.add_argument("--fit", action="store_true", help="k-means fit at c5 scale (with --config c5)")
    ap.add_argument("--fit-iters", type=int, default=10, help="Lloyd iterations per fit step (--fit)")
    ap.add_argument("--fit-algorithm", choices=("lloyd", "elkan"), default="lloyd",
                    help="assignment of the fit (--fit): every row each iteration, or the bound-pruned one")
    ap.add_argument("--fit-init", choices=("random", "centroids"), default="random",
                    help="initial centres of the fit (--fit): a seeded random draw of points, or c5's 1,024 "
                         "centroids (one per mixture component)")
    ap.add_argument("--probe-peak", action="store_true",
                    help="only measure the peaks the roofline fractions are stated against (mlrs_probe_peak: "
                         "FMA f32/f64 and MFMA f32/f64 chains at 1..8 waves per SIMD) and print them as one JSON line")
    ap.add_argument("--dtype", choices=("f32", "f64"), default=None,
                    help="k-NN configurations (c1-c4, d256, c2k128): run the same data in this element type "
                         "(parity then against the CPU oracle on sampled rows)")
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

    if args.probe_peak:
        lib = _lib.load()
        res = {}
        for kind, label, peak in ((0, "valu_fma_f32", PEAKS["valu_f32"]), (1, "valu_fma_f64", PEAKS["valu_f64"]),
                                  (2, "mfma_f32", PEAKS["mfma_f32"]), (3, "mfma_f64", PEAKS["mfma_f64"])):
            row = {}
            for w in (1, 2, 3, 4, 8):
                t = ctypes.c_double()
                _lib.check(lib.mlrs_probe_peak(kind, w, ctypes.byref(t), None))
                row["%d_waves_per_simd" % w] = round(t.value, 2)
            res[label] = {"tflops": row, "published_peak": peak}
            log("%s: %s (published %g)" % (label, row, peak))
        print(json.dumps({"probe": "mlrs_probe_peak", "unit": "TFLOP/s (an FMA counts two flops)", "peaks": res,
                          "device": torch.cuda.get_device_name(0)}))
        return

    cfg = dict(synthetic.CONFIGS[args.config])
    dev = torch.device("cuda:0")
    log("generating %s %s" % (args.config, cfg))
    t = time.time()
    a, b = synthetic.generate(args.config)
    log("generated in %.1fs" % (time.time() - t))
    retyped = args.dtype is not None and args.dtype != cfg["dtype"]
    if args.dtype is not None and (args.config == "c5" or args.fit):
        print("--dtype applies to the k-NN configurations", file=sys.stderr)
        sys.exit(2)
    if retyped:
        # the same values in the other element type (f32 -> f64 is exact)
        npt = np.float64 if args.dtype == "f64" else np.float32
        a, b = a.astype(npt), b.astype(npt)
        cfg["dtype"] = args.dtype
        log("element type %s" % args.dtype)
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
    if args.fit and not kmeans:
        print("--fit needs --config c5", file=sys.stderr)
        sys.exit(2)
    fit_iters = []

    def step():
        if radius is not None:
            return prims.radius_neighbors(ta, tb, radius, metric)
        if args.fit:
            if args.fit_init == "centroids":
                r = prims.kmeans_fit(ta, n_index, "array", tb, max_iter=args.fit_iters, tol=0.0,
                                     algorithm=args.fit_algorithm)
            else:
                r = prims.kmeans_fit(ta, n_index, "random", seed=7, max_iter=args.fit_iters, tol=0.0,
                                     algorithm=args.fit_algorithm)
            fit_iters.append(r[3])
            return r
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
    # the dominant kernel's time within one step (a step may launch it more
    # than once: exact tiles, one assignment per Lloyd iteration)
    kern_ms_step = tot_ms.value / args.steps
    log("timed %d steps: %.3f ms/step, %s avg %.3f ms over %d launches (%.3f ms per step)"
        % (args.steps, ms_per_step, name.value.decode(), kern_ms, launches.value, kern_ms_step))

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
    gpath = os.path.join(ROOT, "tests", "golden", "%s_golden.npz" % args.config)
    g = np.load(gpath) if (os.path.exists(gpath) and not retyped) else None
    sub = g["subset"] if g is not None else np.unique(np.linspace(0, n_query - 1, 64).astype(np.int64))
    if args.fit:
        import oracle
        fc, fl, finert, fit_n = out
        npre = 200_000
        if args.fit_init == "centroids":
            wc, wl, wi, wn = oracle.kmeans_fit(a[:npre], n_index, "array", b, max_iter=3, tol=0.0)
            gc, gl, gi, gn = prims.kmeans_fit(ta[:npre].contiguous(), n_index, "array", tb, max_iter=3, tol=0.0,
                                              algorithm=args.fit_algorithm)
        else:
            wc, wl, wi, wn = oracle.kmeans_fit(a[:npre], n_index, "random", seed=7, max_iter=3, tol=0.0)
            gc, gl, gi, gn = prims.kmeans_fit(ta[:npre].contiguous(), n_index, "random", seed=7, max_iter=3,
                                              tol=0.0, algorithm=args.fit_algorithm)
        ok = (np.array_equal(gl.cpu().numpy(), wl.astype(np.int64)) and np.array_equal(gc.cpu().numpy(), wc)
              and gi == wi and gn == wn)
        sub = np.arange(npre)
    elif radius is not None:
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
    elif g is not None:
        dist, idx = out
        ok = (np.array_equal(idx.cpu().numpy()[sub], g["idx"].astype(np.int64))
              and np.array_equal(dist.cpu().numpy()[sub], g["dist"]))
    else:
        import oracle
        dist, idx = out
        wd, wi = oracle.knn_topk(a[sub], b, k, metric)
        ok = (np.array_equal(idx.cpu().numpy()[sub], wi.astype(np.int64))
              and np.array_equal(dist.cpu().numpy()[sub], wd))
    if args.fit:
        parity = ("3-iteration fit of the first 200000 points bitwise-equal to the CPU oracle's (centres, labels, "
                  "inertia, n_iter)" if ok else "MISMATCH vs the CPU oracle")
    else:
        kind = "golden" if (g is not None and radius is None) else "sampled"
        parity = ("bitwise-equal to the CPU oracle on %d %s rows" % (len(sub), kind) if ok
                  else "MISMATCH vs the CPU oracle")
    log(parity)

    evals = float(n_query) * float(n_index)
    if args.fit:
        # one assignment per Lloyd iteration plus the final one
        iters = float(np.mean(fit_iters[-args.steps:]))
        ms_per_iter = ms_per_step / max(iters, 1.0)
        evals_step = evals * (iters + 1.0)
        value = evals_step / (ms_per_step / 1000.0)
    else:
        value = evals / (ms_per_step / 1000.0)
    flops = 2.0 * d * (evals_step if args.fit else evals)
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
    elif kname.startswith("knn_gram_f32") or kname.startswith("knn_k1_resident_f32"):
        bound, peak, unit = "mfma", PEAKS["mfma_f32"], "TFLOP/s"
    else:
        # the low-d ALU kernel and the exact tiles of small searches: vector
        # units without packed math (an FMA counts two flops)
        bound, peak, unit = "valu", PEAKS["valu_f64" if f64 else "valu_f32"], "TFLOP/s"
    achieved = flops / (kern_ms_step / 1000.0) / 1e12
    if args.fit and args.fit_algorithm == "elkan":
        # the bound-pruned fit searches only the rows its bounds leave: the
        # Lloyd fit's flops over its kernel time would overstate the rate
        achieved = None
    traffic = None
    tfile = os.path.join(ROOT, "profiles", "traffic_%s%s%s.json" % ("radius_" if radius is not None else "",
                                                                     args.config, "_" + args.dtype if retyped else ""))
    if os.path.exists(tfile):
        traffic = json.load(open(tfile)).get("hbm_bytes_per_launch")

    cpu = None
    if not args.no_cpu:
        import oracle
        affinity = len(os.sched_getaffinity(0))
        omp = os.environ.get("OMP_NUM_THREADS", "")
        threads = args.cpu_threads or (min(affinity, int(omp)) if omp.isdigit() and int(omp) > 0 else affinity)
        info = oracle.build_info()
        # bounded sample: a prefix of the queries against the full index, run
        # repeatedly until about 10 s of CPU work has been timed
        sample = {"c1": n_query, "c2": 2000, "c3": 256, "c4": 20000, "c5": 400000, "d256": 1000,
                  "c2k128": 2000}[args.config]
        if radius is not None:
            sample = {"c1": n_query, "c2": 512, "c3": 128, "c4": 20000, "d256": 256, "c2k128": 512}[args.config]
        if args.fit:
            sample = 100_000
        log("CPU baseline: %d of %d queries, %d threads (affinity %d, OMP_NUM_THREADS=%s), %s, %s"
            % (sample, n_query, threads, affinity, omp or "unset", info["cpu_model"], info["flags"]))
        cpu_iters = [0]

        def cpu_pass():
            if radius is not None:
                oracle.radius_neighbors(a[:sample], b, radius, metric, nthreads=threads)
            elif args.fit:
                r = oracle.kmeans_fit(a[:sample], n_index, "random", seed=7, max_iter=2, tol=0.0)
                cpu_iters[0] += r[3] + 1
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
        n_evals = float(sample) * n_index * (cpu_iters[0] if args.fit else reps)
        what = ("k-means fits (random init, 2 iterations) of the first %d of %d points" if args.fit
                else "first %d of %d queries vs the full %d-row index" % (sample, n_query, n_index))
        if args.fit:
            what = what % (sample, n_query)
        cpu = {"value": n_evals / dt, "unit": "dist-evals/s", "cores": threads, "kind": "port",
               "sample": "%s, %d passes in %.1f s" % (what, reps, dt),
               "affinity_cpus": affinity, "omp_num_threads": omp or None, "cpu_model": info["cpu_model"],
               "oracle_build": info["flags"]}
        log("CPU baseline %.3g evals/s" % cpu["value"])

    wl = {"c1": "c1: 10k x 1k, d=64, k=10, f32 N(0,1)",
          "c2": "c2: 1M index x 10k queries, d=128, k=32, f32, 100-comp GMM",
          "c3": "c3: 200k x 5k, d=256, k=16, f64 cosine, U[0,1)",
          "c4": "c4: 500k self-kNN, d=3, k=8, f32, 5% exact duplicates",
          "c5": "c5: k-means assign, 5M points x 1024 centroids, d=64, f32",
          "d256": "d256: 200k index x 5k queries, d=256, k=32, f32, 100-comp GMM",
          "c2k128": "c2k128: c2's data (1M index x 10k queries, d=128) with k=128, f32"}[args.config]
    if retyped:
        wl = "%s; run in %s" % (wl, args.dtype)
    if args.fit:
        wl = ("k-means fit at c5 scale: 5M points into 1024 clusters, d=64, f32, %s init, tol 0, "
              "at most %d Lloyd iterations per step, algorithm=%s"
              % ("seeded random" if args.fit_init == "random" else "the c5 centroids' (explicit)", args.fit_iters,
                 args.fit_algorithm))
    if radius is not None:
        wl = "radius_neighbors, radius %g, on %s (%d matches, %.1f per query)" % (radius, wl, matches,
                                                                                 matches / n_query)
    if args.fit:
        metric_name = "k-means fit assignment dist-evals/s (c5 scale)"
    elif radius is not None:
        metric_name = "radius_neighbors dist-evals/s (%s)" % args.config
    else:
        metric_name = METRIC if args.config == "c2" else "dist-evals/s (%s)" % args.config
        if retyped:
            metric_name = "dist-evals/s (%s in %s)" % (args.config, args.dtype)
    line = {
        "metric": metric_name,
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
        "fit": ({"iterations": float(np.mean(fit_iters[-args.steps:])), "ms_per_iteration": ms_per_iter}
                if args.fit else None),
        "roofline": {"bound": bound, "achieved": achieved, "peak": peak, "unit": unit,
                     "frac": achieved / peak if achieved is not None else None,
                     "traffic": traffic, "kernel": name.value.decode(), "kernel_ms": kern_ms,
                     "kernel_launches_per_step": launches.value / args.steps, "kernel_ms_per_step": kern_ms_step,
                     "frac_nonpacked": (achieved / VALU_F32_NONPACKED
                                        if bound == "valu" and not f64 and achieved is not None else None),
                     "basis": {"mfma": "dense MFMA peak, 2*d flops per distance evaluation",
                               "valu": ("published vector FP64 peak 78.6 TFLOP/s; 2*d flops per distance "
                                        "evaluation" if f64 else
                                        "published vector FP32 peak 157.3 TFLOP/s, which counts packed FP32 "
                                        "math; the kernel is built without packed ops, whose ceiling is "
                                        "78.6 TFLOP/s (frac_nonpacked); 2*d flops per distance "
                                        "evaluation")}[bound]},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    if not ok:
        sys.exit(1)


if __name__ == "__main__":
    main()
