"""The collect + select kNN path on fp32 rows (float data, Dp <= 160,
4 < M <= 64).

Its keys are the merging fp32 kernel's bit for bit (the same MFMA chain and
key formula), so every pass here equals the merging kernel's
(GTANN_KNN_COLLECT=0) exactly -- ids and distances, ties included -- and the
CPU oracle within the float tolerance of the fp32 path.
"""

import numpy as np
import pytest

import gt_oracle as O
from helpers import assert_knn_close, debug_opts

pytestmark = pytest.mark.gpu


def _data(n, d, seed, centres=40, sigma=0.3):
    rng = np.random.default_rng(seed)
    C = rng.normal(size=(centres, d)).astype(np.float32)
    X = C[rng.integers(0, centres, n)] + sigma * rng.normal(size=(n, d)).astype(np.float32)
    return X.astype(np.float32)


def _buckets(rng, N, B, sizes=None):
    if sizes is None:
        lab = rng.integers(0, B, size=N)
        lab[:B] = np.arange(B)
    else:
        lab = np.repeat(np.arange(B), sizes)
        rng.shuffle(lab)
    order = np.argsort(lab, kind="stable")
    off = np.zeros(B + 1, np.int64)
    np.add.at(off, lab + 1, 1)
    return np.cumsum(off), order.astype(np.int32)


def _probe(rng, B, P):
    if P == 0:
        return np.zeros((B, 0), np.int32)
    return np.stack([rng.permutation(np.delete(np.arange(B), b))[:P] for b in range(B)]).astype(np.int32)


def _merging(ctx, *args, **kw):
    with debug_opts(ctx, knn_collect=False):
        return ctx.knn_bucketed(*args, **kw)


def _equal(x, y):
    np.testing.assert_array_equal(x[0], y[0])
    np.testing.assert_array_equal(x[1].view(np.uint32), y[1].view(np.uint32))


@pytest.mark.parametrize("N,D,B,P,M,metric", [
    (6000, 128, 6, 0, 64, "l2"),
    (6000, 128, 6, 1, 64, "l2"),
    (5000, 96, 8, 2, 48, "l2"),
    (4000, 32, 5, 1, 17, "l2"),      # M <= 32: 16-key lanes
    (3000, 160, 4, 0, 32, "l2"),
    (3000, 64, 12, 0, 5, "l2"),
    (4000, 96, 6, 1, 64, "ip"),
    (3000, 128, 5, 0, 33, "ip"),
])
def test_f32_collect_equals_merging_kernel(ctx, N, D, B, P, M, metric):
    rng = np.random.default_rng(N + D + M)
    X = _data(N, D, seed=D + M)
    if metric == "ip":
        X /= np.linalg.norm(X, axis=1, keepdims=True)
    off, mem = _buckets(rng, N, B)
    probe = _probe(rng, B, P)
    print(f"f32 collect N={N} D={D} B={B} P={P} M={M} {metric}", flush=True)
    a = ctx.knn_bucketed(X, off, mem, probe, M, metric=metric)
    c = _merging(ctx, X, off, mem, probe, M, metric=metric)
    _equal(a, c)
    # a seeded pass over a second bucketing
    off2, mem2 = _buckets(np.random.default_rng(N), N, B)
    b2 = ctx.knn_bucketed(X, off2, mem2, probe, M, metric=metric, running=a)
    c2 = _merging(ctx, X, off2, mem2, probe, M, metric=metric, running=c)
    _equal(b2, c2)


def test_f32_collect_matches_oracle(ctx):
    rng = np.random.default_rng(21)
    N, D, B, M = 5000, 96, 6, 64
    X = _data(N, D, seed=22)
    off, mem = _buckets(rng, N, B)
    probe = _probe(rng, B, 1)
    print("f32 collect vs oracle", flush=True)
    ids, dist = ctx.knn_bucketed(X, off, mem, probe, M)
    ri, rd = O.knn_bucketed(X, off, mem, probe, M)
    assert_knn_close(X, np.arange(N), ids, dist, ri, rd)


def test_f32_collect_small_buckets_and_duplicates(ctx):
    # pools shorter than the threshold window and than M, a single row, and
    # 300 copies of one row (ties at distance 0 decided by id)
    rng = np.random.default_rng(5)
    sizes = [1, 2, 30, 63, 64, 65, 200, 257, 900, 2000]
    N = sum(sizes)
    X = _data(N, 128, seed=6)
    X[100:400] = X[99]
    off, mem = _buckets(rng, N, len(sizes), sizes)
    for P in (0, 1):
        probe = _probe(rng, len(sizes), P)
        print(f"f32 collect small buckets P={P}", flush=True)
        _equal(ctx.knn_bucketed(X, off, mem, probe, 64), _merging(ctx, X, off, mem, probe, 64))


def test_f32_collect_seeded_without_cap_compacts(ctx):
    # a running table of padding seeds every query with +inf: every pool row
    # passes and each query's slots are compacted many times
    rng = np.random.default_rng(9)
    N, B, M = 8000, 4, 64
    X = _data(N, 128, seed=10)
    off, mem = _buckets(rng, N, B)
    probe = _probe(rng, B, 1)
    run = (np.full((N, M), -1, np.int32), np.full((N, M), np.inf, np.float32))
    print("f32 collect seeded with +inf", flush=True)
    _equal(ctx.knn_bucketed(X, off, mem, probe, M, running=run),
           _merging(ctx, X, off, mem, probe, M, running=run))


def test_f32_build_equals_merging_kernel(ctx):
    # whole builds (2 rounds, probes, prune, reverse merge) on C3-like data
    rng = np.random.default_rng(3)
    C = rng.normal(size=(50, 96)).astype(np.float32)
    C /= np.linalg.norm(C, axis=1, keepdims=True)
    X = C[rng.integers(0, 50, 30000)] + (0.3 / np.sqrt(96)) * rng.normal(size=(30000, 96)).astype(np.float32)
    X = (X / np.linalg.norm(X, axis=1, keepdims=True)).astype(np.float32)
    kw = dict(n_buckets=24, M=64, K=32, rounds=2, nprobe=1, metric="ip")
    print("f32 collect build", flush=True)
    a = ctx.build_graph(X, **kw)
    with debug_opts(ctx, knn_collect=False):
        b = ctx.build_graph(X, **kw)
    np.testing.assert_array_equal(a.knn_ids, b.knn_ids)
    np.testing.assert_array_equal(a.knn_dists, b.knn_dists)
    np.testing.assert_array_equal(a.graph, b.graph)


@pytest.mark.parametrize("window,metric", [(2, "l2"), (32, "l2"), (32, "ip")])
def test_f32_collect_threshold_window_sizes(ctx, window, metric):
    # the threshold window's size changes how many keys are collected, never
    # the lists: the merging kernel's bit for bit
    rng = np.random.default_rng(window + 5)
    N, D, B = 8000, 96, 3
    X = _data(N, D, seed=window)
    if metric == "ip":
        X /= np.linalg.norm(X, axis=1, keepdims=True)
    off, mem = _buckets(rng, N, B)
    probe = _probe(rng, B, 1)
    print(f"f32 collect window {window} {metric}", flush=True)
    with debug_opts(ctx, knn_window=window):
        got = ctx.knn_bucketed(X, off, mem, probe, 64, metric=metric)
    _equal(got, _merging(ctx, X, off, mem, probe, 64, metric=metric))
