"""Integer-typed datasets (.i8bin int8, .u8bin uint8) on the int8 matrix-core
kNN kernel, against the CPU oracle on the same values in float.

Every distance of integer rows is an exact integer in both paths (int32 sums
on the GPU, float64 in the oracle), so the comparisons are bit-exact.  uint8
rows are shifted by -128 on the device, which leaves L2 distances unchanged;
uint8 with the inner product keeps the fp32 kernel (the shift would change
the products), as do rows longer than 256 bytes.
"""
import numpy as np
import pytest

import gt_oracle as O
from helpers import assert_knn_equal

pytestmark = pytest.mark.gpu


def _data(n, d, dtype, seed, lo=None, hi=None):
    rng = np.random.default_rng(seed)
    if dtype == np.uint8:
        lo, hi = (0, 256) if lo is None else (lo, hi)
    else:
        lo, hi = (-128, 128) if lo is None else (lo, hi)
    return rng.integers(lo, hi, size=(n, d)).astype(dtype)


@pytest.mark.parametrize("dtype", [np.int8, np.uint8])
@pytest.mark.parametrize("n,d,k", [(2000, 128, 64), (1500, 96, 32), (900, 100, 17), (700, 256, 48),
                                   (600, 200, 8), (400, 32, 128), (300, 8, 5), (5, 16, 4)])
def test_knn_exact_bitexact(ctx, dtype, n, d, k):
    X = _data(n, d, dtype, seed=n + d)
    k = min(k, n - 1)
    print(f"int8 exact {np.dtype(dtype).name} n={n} d={d} k={k}", flush=True)
    ids, dist = ctx.knn_exact(X, k)
    rid, rd = O.knn_exact(X.astype(np.float32), k)
    assert_knn_equal(ids, dist, rid, rd)
    # the fp32 kernel on the same values gives the same lists
    fi, fd = ctx.knn_exact(X.astype(np.float32), k)
    assert_knn_equal(ids, dist, fi, fd)


@pytest.mark.parametrize("dtype", [np.int8, np.uint8])
def test_knn_exact_ip(ctx, dtype):
    X = _data(1200, 128, dtype, seed=3, lo=-20 if dtype == np.int8 else 0, hi=21)
    ids, dist = ctx.knn_exact(X, 32, metric="ip")
    rid, rd = O.knn_exact(X.astype(np.float32), 32, metric=1)
    # the library reports the inner product (descending); the oracle its negation
    np.testing.assert_array_equal(ids, rid)
    np.testing.assert_array_equal(-dist, rd)


@pytest.mark.parametrize("dtype", [np.int8, np.uint8])
@pytest.mark.parametrize("k", [1, 2, 3, 4])
def test_knn_exact_short_lists(ctx, dtype, k):
    # lists of at most 4 entries stay in registers (one partial list per
    # half-wave, merged at the end); ties are frequent on a narrow range
    X = _data(3000, 128, dtype, seed=40 + k, lo=0 if dtype == np.uint8 else -3, hi=4)
    ids, dist = ctx.knn_exact(X, k)
    rid, rd = O.knn_exact(X.astype(np.float32), k)
    assert_knn_equal(ids, dist, rid, rd)
    q = np.arange(0, 3000, 7)
    ids, dist = ctx.knn_exact(X, k, queries=q, metric="ip")
    rid, rd = O.knn_exact(X.astype(np.float32), k, queries=q, metric=1)
    np.testing.assert_array_equal(ids, rid)
    np.testing.assert_array_equal(-dist, rd)


def test_knn_exact_query_subset_split_pool(ctx):
    X = _data(40000, 128, np.int8, seed=1)
    q = np.random.default_rng(2).choice(40000, size=300, replace=False)
    ids, dist = ctx.knn_exact(X, 32, queries=q)
    rid, rd = O.knn_exact(X.astype(np.float32), 32, queries=q)
    assert_knn_equal(ids, dist, rid, rd)


def test_knn_exact_ties_and_extremes(ctx):
    # a tiny value range (massive ties) plus rows at the ends of the range
    X = _data(2000, 128, np.int8, seed=4, lo=-1, hi=2)
    X[:10] = -128
    X[10:20] = 127
    X[100] = X[200]
    ids, dist = ctx.knn_exact(X, 64)
    rid, rd = O.knn_exact(X.astype(np.float32), 64)
    assert_knn_equal(ids, dist, rid, rd)
    U = X.view(np.uint8)   # 0 and 255 rows, and everything in between
    ids, dist = ctx.knn_exact(U, 64)
    rid, rd = O.knn_exact(U.astype(np.float32), 64)
    assert_knn_equal(ids, dist, rid, rd)


def _buckets(rng, N, B):
    lab = rng.integers(0, B, size=N)
    lab[:B] = np.arange(B)
    order = np.argsort(lab, kind="stable")
    off = np.zeros(B + 1, np.int64)
    np.add.at(off, lab + 1, 1)
    return np.cumsum(off), order.astype(np.int32)


@pytest.mark.parametrize("dtype", [np.int8, np.uint8])
def test_knn_bucketed_rounds(ctx, dtype):
    rng = np.random.default_rng(11)
    N, B, M = 5000, 10, 32
    X = _data(N, 128, dtype, seed=12)
    Xf = X.astype(np.float32)
    run = ref = None
    for r in range(3):
        off, mem = _buckets(rng, N, B)
        probe = np.stack([rng.permutation(np.delete(np.arange(B), b))[:2] for b in range(B)]).astype(np.int32)
        ids, dist = ctx.knn_bucketed(X, off, mem, probe, M, running=run)
        ni, nd = O.knn_bucketed(Xf, off, mem, probe, M)
        ref = (ni, nd) if ref is None else O.merge_rounds(*ref, ni, nd)
        run = (ids, dist)
        assert_knn_equal(ids, dist, *ref)


def test_build_graph_all_probed_is_exact(ctx):
    """The whole build on int8 rows with every bucket probed: the pre-prune
    table is the exact kNN, the graph oracle prune + merge of it."""
    X = _data(6000, 128, np.int8, seed=21, lo=-40, hi=41)
    res = ctx.build_graph(X, n_buckets=12, nprobe=11, M=64, K=32, rounds=1)
    ex_i, ex_d = O.knn_exact(X.astype(np.float32), 64)
    np.testing.assert_array_equal(res.knn_ids, ex_i)
    np.testing.assert_array_equal(res.knn_dists, ex_d)
    fwd, rc, _ = O.cagra_prune(O.sanitize(res.knn_ids), 32)
    assert rc == 0
    np.testing.assert_array_equal(res.graph, O.reverse_merge(fwd))


def test_build_graph_int8_matches_fp32(ctx):
    # same values as int8 and as float: the int8 kernel and the fp32 kernel
    # build the same graph (all keys exact, all launches see the same pools:
    # the centroids are data points, so rounding them to int8 changes nothing)
    X = _data(20000, 128, np.int8, seed=22, lo=-60, hi=61)
    kw = dict(n_buckets=16, nprobe=1, M=64, K=32, rounds=2, kmeans_iters=0)
    a = ctx.build_graph(X, **kw)
    b = ctx.build_graph(X.astype(np.float32), **kw)
    np.testing.assert_array_equal(a.knn_ids, b.knn_ids)
    np.testing.assert_array_equal(a.knn_dists, b.knn_dists)
    np.testing.assert_array_equal(a.graph, b.graph)


def test_long_rows_keep_fp32_kernel(ctx):
    X = _data(800, 300, np.int8, seed=23)
    ids, dist = ctx.knn_exact(X, 16)
    rid, rd = O.knn_exact(X.astype(np.float32), 16)
    assert_knn_equal(ids, dist, rid, rd)


def test_build_graph_int8_with_lloyd_recall(ctx):
    # Lloyd-moved centroids are rounded to int8 for the assignment: a valid
    # bucketing, checked through the recall of the built table
    X = _data(30000, 64, np.uint8, seed=23)
    X[:, :8] = (np.arange(30000)[:, None] % 7 * 30).astype(np.uint8)   # some structure
    res = ctx.build_graph(X, n_buckets=24, nprobe=2, M=32, K=16, rounds=2, kmeans_iters=3)
    q = np.arange(0, 30000, 97)
    ex, _ = O.knn_exact(X.astype(np.float32), 32, queries=q)
    rec = np.mean([len(np.intersect1d(res.knn_ids[qq], ex[j])) / 32 for j, qq in enumerate(q)])
    assert rec > 0.5, rec
    assert (res.graph < 30000).all()
