"""Seeded synthetic workloads of the benchmark configurations (numpy, host).

Every generator is a pure function of its seed (numpy's PCG64 Generator), so
the same arrays come out on any machine.  Shapes and distributions follow the
five configurations the kNN path is measured on:

c1  index 10,000 x 64 and queries 1,000 x 64, iid N(0,1), f32, k=10
c2  index 1,000,000 x 128 and queries 10,000 x 128 from a 100-component
    Gaussian mixture (centres U[-10,10]^128, unit isotropic std, equal
    weights), f32, k=32
c3  index 200,000 x 256 and queries 5,000 x 256, iid U[0,1), f64, cosine, k=16
c4  500,000 x 3 points U[0,1)^3, 5% of rows overwritten by exact copies of
    other rows, queries = the index itself, f32, k=8 (self included)
c5  5,000,000 x 64 points from a 1,024-component mixture (centres N(0, 25 I),
    unit std) against 1,024 centroids = centres + N(0, 0.01 I) (variance 0.01,
    i.e. std 0.1), f32, k=1 (nearest-centre assignment)

and one more shape outside the five, an embedding-sized search:

d256 index 200,000 x 256 and queries 5,000 x 256 from c2's generator at
     d = 256 (100-component mixture, centres U[-10,10]^256, unit std), f32,
     Euclidean, k=32

and c2 at the top of the reference's metric-arm k range:

c2k128 c2's data with k=128
"""
import numpy as np

SEED = 42

CONFIGS = {
    "c1": dict(n_index=10_000, n_query=1_000, d=64, k=10, metric="euclidean", dtype="f32"),
    "c2": dict(n_index=1_000_000, n_query=10_000, d=128, k=32, metric="euclidean", dtype="f32"),
    "c3": dict(n_index=200_000, n_query=5_000, d=256, k=16, metric="cosine", dtype="f64"),
    "c4": dict(n_index=500_000, n_query=500_000, d=3, k=8, metric="euclidean", dtype="f32"),
    "c5": dict(n_index=1_024, n_query=5_000_000, d=64, k=1, metric="euclidean", dtype="f32"),
    "d256": dict(n_index=200_000, n_query=5_000, d=256, k=32, metric="euclidean", dtype="f32"),
    "c2k128": dict(n_index=1_000_000, n_query=10_000, d=128, k=128, metric="euclidean", dtype="f32"),
}


def _normal(rng, shape, dtype):
    return rng.standard_normal(shape, dtype=dtype)


def gen_c1(seed=SEED, n_index=10_000, n_query=1_000, d=64):
    rng = np.random.default_rng(seed)
    xt = _normal(rng, (n_index, d), np.float32)
    xq = _normal(rng, (n_query, d), np.float32)
    return xq, xt


def _mixture(rng, centres, n, dtype):
    comp = rng.integers(0, centres.shape[0], size=n)
    x = centres[comp].astype(dtype, copy=False)
    x += _normal(rng, x.shape, dtype)
    return x


def gen_c2(seed=SEED, n_index=1_000_000, n_query=10_000, d=128, n_comp=100):
    rng = np.random.default_rng(seed)
    centres = rng.uniform(-10.0, 10.0, size=(n_comp, d)).astype(np.float32)
    xt = _mixture(rng, centres, n_index, np.float32)
    xq = _mixture(rng, centres, n_query, np.float32)
    return xq, xt


def gen_c3(seed=SEED, n_index=200_000, n_query=5_000, d=256):
    rng = np.random.default_rng(seed)
    xt = rng.random((n_index, d), dtype=np.float64)
    xq = rng.random((n_query, d), dtype=np.float64)
    return xq, xt


def gen_c4(seed=SEED, n=500_000, d=3, dup_frac=0.05):
    rng = np.random.default_rng(seed)
    x = rng.random((n, d), dtype=np.float32)
    n_dup = int(round(n * dup_frac))
    perm = rng.permutation(n)
    dst, src = perm[:n_dup], perm[n_dup:2 * n_dup]
    x[dst] = x[src]
    return x, x


def gen_c5(seed=SEED, n_points=5_000_000, n_centres=1_024, d=64):
    rng = np.random.default_rng(seed)
    centres = (5.0 * _normal(rng, (n_centres, d), np.float64)).astype(np.float32)
    x = _mixture(rng, centres, n_points, np.float32)
    centroids = (centres.astype(np.float64) + 0.1 * rng.standard_normal((n_centres, d))).astype(np.float32)
    return x, centroids


def gen_d256(seed=SEED, n_index=200_000, n_query=5_000, d=256):
    return gen_c2(seed=seed, n_index=n_index, n_query=n_query, d=d)


GENERATORS = {"c1": gen_c1, "c2": gen_c2, "c3": gen_c3, "c4": gen_c4, "c5": gen_c5, "d256": gen_d256,
              "c2k128": gen_c2}


def generate(name, **kw):
    """(queries, index) for c1-c4; (points, centroids) for c5."""
    return GENERATORS[name](**kw)
