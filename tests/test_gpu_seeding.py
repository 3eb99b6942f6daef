"""KMeans|| seeding of the bucketing (src/bucket.cu:2833-3168) on the GPU.

Its random draws cannot match the reference's RNG, so these tests check the
algorithm's properties: C distinct data points, each in its own bucket; the
same seed gives the same build; and D^2 oversampling finds small far
clusters that a uniform sample of rows misses.  On one large tight cluster
plus 8 clusters of 10 rows far away (C = 16 buckets), a uniform sample of 16
rows hits about 1 % of the far clusters; D^2 sampling gives each far row a
probability near l*C/80 per round, so the ~1.5 C candidates cover the far
clusters and the final uniform choice of C of them keeps about 80 % (a
simulation of the same steps on 40 seeds: mean 0.81, lowest 0.5).
"""
import numpy as np
import pytest

import synth

pytestmark = pytest.mark.gpu


def _far_clusters(seed, N=20000, D=16, nfar=8, per=10):
    rng = np.random.default_rng(seed)
    X = rng.normal(size=(N, D)).astype(np.float32)
    lab = np.zeros(N, np.int64)
    cen = rng.normal(size=(nfar, D))
    cen = cen / np.linalg.norm(cen, axis=1, keepdims=True) * 1000.0
    idx = rng.choice(N, nfar * per, replace=False)
    for k in range(nfar):
        sl = idx[k * per:(k + 1) * per]
        X[sl] += cen[k].astype(np.float32)
        lab[sl] = k + 1
    return X, lab


@pytest.mark.parametrize("cfg,dtype", [("C2", "f32"), ("C2", "i8"), ("C3", "f32")])
def test_kmeans_par_seeds_are_distinct_data_points(ctx, cfg, dtype):
    X, _ = synth.generate(cfg, n=30000)
    if dtype == "i8":
        X = (X.astype(np.int64) - 128).clip(-128, 127).astype(np.int8)
    metric = synth.CONFIGS[cfg].metric
    C = 24
    print(f"kmeans|| seeds {cfg} {dtype}", flush=True)
    res = ctx.build_graph(X, n_buckets=C, nprobe=1, M=32, K=16, rounds=2, kmeans_iters=0, metric=metric,
                          last_round=True)
    cent = res.last_centroids
    assert len(cent) == C and len(np.unique(cent)) == C
    assert (np.diff(cent) > 0).all() and cent.min() >= 0 and cent.max() < len(X)
    assert (res.last_bucket[cent] == np.arange(C)).all()      # a data-point centroid sits in its own bucket
    assert (res.last_bucket >= 0).all() and (res.last_bucket < C).all()
    assert (np.bincount(res.last_bucket, minlength=C) > 0).all()


def test_kmeans_par_is_deterministic(ctx):
    X, _ = synth.generate("C2", n=20000)
    kw = dict(n_buckets=16, nprobe=1, M=32, K=16, rounds=2, kmeans_iters=0, last_round=True)
    a = ctx.build_graph(X, **kw)
    b = ctx.build_graph(X, **kw)
    c = ctx.build_graph(X, seed=7, **kw)
    np.testing.assert_array_equal(a.last_centroids, b.last_centroids)
    np.testing.assert_array_equal(a.knn_ids, b.knn_ids)
    np.testing.assert_array_equal(a.graph, b.graph)
    assert not np.array_equal(a.last_centroids, c.last_centroids)


def test_kmeans_par_finds_small_far_clusters(ctx):
    cov_kmpar, cov_uniform = [], []
    for s in range(6):
        X, lab = _far_clusters(s)
        kw = dict(n_buckets=16, nprobe=1, M=16, K=8, rounds=1, kmeans_iters=0, prune=False, last_round=True,
                  seed=100 + s)
        a = ctx.build_graph(X, seeding="kmeans||", kmeans_train_fraction=1.0, **kw)
        u = ctx.build_graph(X, seeding="uniform", **kw)
        cov_kmpar.append(len(set(lab[a.last_centroids].tolist()) - {0}) / 8)
        cov_uniform.append(len(set(lab[u.last_centroids].tolist()) - {0}) / 8)
    print(f"far-cluster coverage: kmeans|| {cov_kmpar}, uniform {cov_uniform}", flush=True)
    assert np.mean(cov_kmpar) >= 0.6 and min(cov_kmpar) >= 0.25
    assert np.mean(cov_uniform) <= 0.2


def test_kmeans_par_seeds_lloyd(ctx):
    # KMeans|| seeds moved by Lloyd iterations: a valid bucketing and a
    # table as good as the uniform seeds'
    X, _ = synth.generate("C2", n=40000)
    kw = dict(n_buckets=16, nprobe=1, M=32, K=16, rounds=2, kmeans_iters=3)
    a = ctx.build_graph(X, seeding="kmeans||", **kw)
    b = ctx.build_graph(X, seeding="uniform", **kw)
    q = np.arange(0, len(X), 40)
    ex, _ = ctx.knn_exact(X, 32, queries=q)
    rec = [np.mean([len(np.intersect1d(r.knn_ids[i], ex[k])) / 32 for k, i in enumerate(q)]) for r in (a, b)]
    print(f"recall@32 kmeans|| + Lloyd {rec[0]:.4f}, uniform + Lloyd {rec[1]:.4f}", flush=True)
    assert rec[0] >= rec[1] - 0.02


@pytest.mark.parametrize("rounds,iters,seeding", [(2, 3, "auto"), (3, 0, "auto"), (2, 0, "uniform")])
def test_device_bucket_csr_matches_host(ctx, rounds, iters, seeding):
    # the members ordered by (bucket, other top-2 centroid, id) on the device
    # and on the host: the same buckets, table and graph bit for bit
    from helpers import debug_opts
    X, _ = synth.generate("C2", n=40000)
    kw = dict(n_buckets=24, nprobe=1, M=32, K=16, rounds=rounds, kmeans_iters=iters, seeding=seeding,
              last_round=True, round1_bucket=True)
    print(f"device vs host bucket CSR rounds={rounds} iters={iters} {seeding}", flush=True)
    a = ctx.build_graph(X, **kw)
    with debug_opts(ctx, bucket_host_csr=True):
        b = ctx.build_graph(X, **kw)
    np.testing.assert_array_equal(a.round1_bucket, b.round1_bucket)
    np.testing.assert_array_equal(a.last_bucket, b.last_bucket)
    np.testing.assert_array_equal(a.knn_ids, b.knn_ids)
    np.testing.assert_array_equal(a.knn_dists.view(np.uint32), b.knn_dists.view(np.uint32))
    np.testing.assert_array_equal(a.graph, b.graph)
